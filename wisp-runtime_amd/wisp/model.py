"""Qwen3-MoE model skeletons whose experts live in an ExpertStore: only the non-expert
weights are on the GPU. Runtime set-up entry points as the reference's wisp/model.py
(make_runtime, configure: model.py:58-95) and a random-initialised skeleton of any
Qwen3-MoE config for the synthetic workloads. Loading a checkpoint (the reference's
load_skeleton, model.py:20-55) is outside this build's scope: no checkpoint reaches this
path, and the synthetic skeletons carry the same module structure.
"""

from __future__ import annotations

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
