"""Qwen3-MoE model skeletons whose experts live in an ExpertStore: only the non-expert
weights are on the GPU. Entry points as the reference's wisp/model.py: load_skeleton
(model.py:20-55: a checkpoint's non-expert tensors), make_runtime and configure
(model.py:58-95); and a random-initialised skeleton of any Qwen3-MoE config for the
synthetic workloads, with the same module structure.
"""

from __future__ import annotations

import time

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


def _load_non_experts(model, ck, device):
    """Every tensor of checkpoint `ck` (a SafetensorsDir) outside the experts, assigned to
    the model's parameters on `device`; the output head is tied to the embedding when the
    config ties them and the checkpoint has none."""
    sd = ck.load([k for k in ck.names() if ".mlp.experts." not in k], device)
    res = model.load_state_dict(sd, strict=False, assign=True)
    missing = [k for k in res.missing_keys if "rotary" not in k]
    if missing == ["lm_head.weight"] and getattr(model.config, "tie_word_embeddings", False):
        model.lm_head.weight = model.model.embed_tokens.weight
        missing = []
    if missing:
        raise KeyError(f"the checkpoint lacks {missing[:5]}")


@torch.no_grad()
def load_skeleton(model_dir, rt, device="cuda"):
    """The model of `model_dir` (config.json + safetensors) built on the meta device, paged
    MoE blocks attached to rt, every non-expert tensor loaded straight to `device`
    (model.py:20-55); gpt-oss checkpoints go to gptoss.load_skeleton_gptoss. The experts
    come from rt's store (ExpertStore.from_safetensors). Returns (model, cfg)."""
    from transformers import AutoConfig

    from .store import SafetensorsDir

    cfg = AutoConfig.from_pretrained(model_dir)
    if cfg.model_type == "gpt_oss":
        from .gptoss import load_skeleton_gptoss

        return load_skeleton_gptoss(model_dir, rt, device)
    t0 = time.time()
    model = _meta_model(cfg, torch.bfloat16)
    _gates_with_storage(model, cfg, device, torch.bfloat16)
    attach(model, rt)
    _load_non_experts(model, SafetensorsDir(model_dir), device)
    _fresh_rotary(model, cfg, device)
    model.eval()
    print(f"[model] non-expert weights on {device}: {nbytes_of(model) / 2**30:.2f} GiB ({time.time() - t0:.0f}s)",
          flush=True)
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
