"""Qwen3-MoE model skeletons whose experts live in an ExpertStore: only the non-expert
weights are on the GPU. Same entry points as the reference's wisp/model.py
(load_skeleton, make_runtime, configure: model.py:20-95), plus a random-initialised
skeleton for synthetic benchmarks (no checkpoint is needed).
"""

from __future__ import annotations

import json
import os

import torch
import torch.nn as nn

from .cache import ExpertCache
from .moe import Runtime, attach


def nbytes_of(model):
    return sum(p.numel() * p.element_size() for p in model.parameters()) + sum(
        b.numel() * b.element_size() for b in model.buffers()
    )


def _meta_model(cfg, dtype):
    from transformers import AutoModelForCausalLM

    with torch.device("meta"):
        return AutoModelForCausalLM.from_config(cfg, dtype=dtype)


def _fresh_rotary(model, cfg, device):
    """The rotary table module rebuilt in float32 on `device` (its inv_freq buffer must not be
    rounded to the weights' dtype)."""
    model.model.rotary_emb = type(model.model.rotary_emb)(config=cfg).to(device)


def _gates_with_storage(model, cfg, device, dtype):
    for layer in model.model.layers:  # real storage, so attach() keeps a real router module
        layer.mlp.gate = nn.Linear(cfg.hidden_size, cfg.num_experts, bias=False, device=device, dtype=dtype)


def load_skeleton(model_dir, rt, device="cuda", dtype=torch.bfloat16):
    """Meta-initialise the model, attach paged MoE blocks, then load every NON-expert tensor of
    the checkpoint in `model_dir` (model.safetensors.index.json or a single model.safetensors)
    straight to `device` (model.py:20-55)."""
    from safetensors import safe_open
    from transformers import AutoConfig

    cfg = AutoConfig.from_pretrained(model_dir)
    if cfg.model_type == "gpt_oss":  # model.py:25-28
        from .gptoss import load_skeleton_gptoss

        return load_skeleton_gptoss(model_dir, rt, device)
    model = _meta_model(cfg, dtype)
    _gates_with_storage(model, cfg, device, dtype)
    attach(model, rt)
    index = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            where = json.load(f)["weight_map"]
    else:
        with safe_open(os.path.join(model_dir, "model.safetensors"), framework="pt", device="cpu") as h:
            where = {k: "model.safetensors" for k in h.keys()}
    wanted = {k: f for k, f in where.items() if ".mlp.experts." not in k}
    sd = {}
    for fn in sorted(set(wanted.values())):
        with safe_open(os.path.join(model_dir, fn), framework="pt", device=str(device)) as h:
            for k in h.keys():
                if k in wanted:
                    sd[k] = h.get_tensor(k).to(dtype)
    missing = model.load_state_dict(sd, strict=False, assign=True)
    bad = [k for k in missing.missing_keys if "rotary" not in k]
    assert not bad, f"missing keys: {bad[:5]}"
    _fresh_rotary(model, cfg, device)
    model.eval()
    return model, cfg


@torch.no_grad()
def random_skeleton(cfg, rt, device="cuda", dtype=torch.bfloat16, std=0.02, seed=0):
    """A random-initialised skeleton of `cfg` (non-expert weights ~ N(0, std), norms at 1)
    with paged MoE blocks attached; its experts are whatever rt's store holds."""
    model = _meta_model(cfg, dtype)
    _gates_with_storage(model, cfg, device, dtype)
    attach(model, rt)
    model.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    for name, p in model.named_parameters():
        if "norm" in name:
            p.fill_(1.0)
        else:
            p.copy_(torch.randn(p.shape, generator=gen, device=device, dtype=torch.float32).mul_(std).to(dtype))
    _fresh_rotary(model, cfg, device)
    model.eval()
    return model


def make_runtime(store, **kw):
    return Runtime(store, cache=None, **kw)


def configure(rt, nslots, policy="lru", miss_policy="transfer", decay=0.9995, n_static=0, admit_after=2.0,
              preload_keys=None, prefetch=False, cpu_threshold=4, chunk=8, vram_cap_gb=None, cpu_store=None,
              decode_on_load=False):
    """(Re)build the GPU expert cache with a new setting (model.py:62-95)."""
    if rt.cache is not None:
        rt.cache.free()
        rt.cache = None
    torch.cuda.empty_cache()
    if vram_cap_gb is not None:
        total = torch.cuda.get_device_properties(0).total_memory
        torch.cuda.set_per_process_memory_fraction(min(1.0, vram_cap_gb * 2**30 / total), 0)
    rt.cache = ExpertCache(rt.store, nslots, "cuda", policy, decay, n_static, admit_after, preload_keys, cpu_store,
                           decode_on_load)
    rt.miss_policy, rt.prefetch, rt.cpu_threshold, rt.chunk = miss_policy, prefetch, cpu_threshold, chunk
    rt.reset_stats()
    return rt.cache
