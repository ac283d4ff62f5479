"""Paged MoE block (drop-in for the Qwen3-MoE sparse block), the shared Runtime, and the
routing helpers. Same interface as the reference's wisp/moe.py (moe.py:11-222).

Routing (moe.py:67-72, graphdec.py:177-181): softmax in float32, top-k, renormalise
(norm_topk_prob), round the weights to the activation dtype (bf16), then pack
[slot ids..., weights...] as float32 for the decode kernels (moe.py:181-197).

Execution paths of PagedMoEBlock.forward:
  * one token with `fused == 2` (or always inside the graph decoder): the two gfx950
    decode kernels on the slot pool, one host sync and one native paging step per layer;
  * one token with `fused == 1`: the per-expert kernel path (moe_decode_q4);
  * more tokens (prefill, or decode without fusion): per routed expert, dequantize its
    slot (bit-exact kernel) and run the expert MLP as three bf16 GEMMs.
The reference's 'hybrid' miss policy computes misses on the host CPU; this build has no
CPU compute path, so that policy is refused.
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn
import torch.nn.functional as F


def _router_logits_returned() -> bool:
    """transformers 4.x decoder layers take (hidden, router_logits) from the MoE block;
    5.x layers add the block's output to the residual directly."""
    try:
        import transformers

        return int(transformers.__version__.split(".")[0]) < 5
    except Exception:
        return False


RETURN_ROUTER_LOGITS = _router_logits_returned()


def route(logits: torch.Tensor, k: int, norm_topk: bool = True, dtype=torch.bfloat16):
    """logits [N, E] -> (sel int64 [N, k], weights [N, k] in `dtype`)."""
    rw = F.softmax(logits, dim=1, dtype=torch.float32)
    rw, sel = torch.topk(rw, k, dim=-1)
    if norm_topk:
        rw = rw / rw.sum(dim=-1, keepdim=True)
    return sel, rw.to(dtype)


def pack_meta(slots: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """[..., k] slot ids and weights -> float32 [..., 2k] = [slots..., weights...]
    (the layout kernels.py:189-190 reads). Slot ids must be < 2^24 to be exact."""
    return torch.cat([slots.to(torch.float32), weights.to(torch.float32)], dim=-1)


class Runtime:
    """State shared by all paged blocks (moe.py:11-39)."""

    def __init__(self, store, cache=None, miss_policy="transfer", cpu_threshold=4, prefetch=False, chunk=8,
                 cpu_threads=None, fused=False):
        self.fused = int(fused) or int(os.environ.get("WISP_FUSED", "0") or 0)
        self.store, self.cache = store, cache
        self.miss_policy = miss_policy
        self.cpu_threshold = cpu_threshold
        self.prefetch = prefetch
        self.chunk = chunk
        self.recorder = None  # list -> collects (layer, sel[N, k])
        self.reset_stats()
        if cpu_threads:
            torch.set_num_threads(cpu_threads)

    def reset_stats(self):
        self.stats = dict(layer_calls=0, cpu_experts=0, gpu_experts=0, cpu_time=0.0, admitted=0, prefetched=0)


def _expert_mlp(x, W3, I, H):
    """down(SiLU(gate x) * up x) with one dequantized expert W3 [3, n] (moe.py:42-45)."""
    g = F.linear(x, W3[0].view(I, H))
    u = F.linear(x, W3[1].view(I, H))
    return F.linear(F.silu(g) * u, W3[2].view(H, I))


_mlp = _expert_mlp  # the reference's name (moe.py:42), imported by its callers (scripts/microbench.py:14)


def _gate_linear(gate, H, E):
    """The router as a plain Linear [E, H] (transformers 5 wraps it in a top-k router module)."""
    if isinstance(gate, nn.Linear):
        return gate
    lin = nn.Linear(H, E, bias=False, device=gate.weight.device, dtype=gate.weight.dtype)
    lin.weight = gate.weight
    return lin


class PagedMoEBlock(nn.Module):
    """moe.py:48-204: experts live in the expert cache's slot pool, paged from the host store."""

    def __init__(self, gate, layer_idx, rt, cfg):
        super().__init__()
        self.H, self.I = cfg.hidden_size, cfg.moe_intermediate_size
        self.E, self.top_k = cfg.num_experts, cfg.num_experts_per_tok
        self.norm_topk = cfg.norm_topk_prob
        self.gate = _gate_linear(gate, self.H, self.E)
        self.layer_idx, self.rt = layer_idx, rt
        self.next_gate = None
        self.return_router_logits = RETURN_ROUTER_LOGITS

    def set_next_gate(self, gate):
        # another block's parameter: kept out of this module's registration
        object.__setattr__(self, "next_gate", gate)

    def forward(self, hidden_states):
        rt, cache = self.rt, self.rt.cache
        B, T, H = hidden_states.shape
        x = hidden_states.reshape(-1, H)
        N = x.shape[0]
        logits = self.gate(x)
        sel, rw = route(logits, self.top_k, self.norm_topk, x.dtype)
        out = self._route_and_run(x, logits, sel, rw, N, B, T, H)
        return (out, logits) if self.return_router_logits else out

    def _route_and_run(self, x, logits, sel, rw, N, B, T, H):
        rt, cache = self.rt, self.rt.cache
        decode = N <= rt.cpu_threshold
        if decode and rt.miss_policy == "hybrid":
            raise NotImplementedError("the 'hybrid' miss policy computes on the host CPU; this build has no CPU path")
        do_pf = rt.prefetch and decode and self.next_gate is not None
        pred = torch.topk(self.next_gate(x), self.top_k, dim=-1).indices if do_pf else None
        bits = cache.store.bits
        if rt.fused == 2 and N == 1 and bits in (2, 3, 4) and not cache.decode_on_load:
            return self._forward_fast(x, rw, sel, pred, B, T, H)
        if rt.fused == 1 and N == 1 and bits == 4 and not cache.decode_on_load:
            return self._forward_per_expert(x, rw, sel, pred, B, T, H)
        return self._forward_dequant(x, rw, sel, pred, B, T, H)

    def _record(self, sel_cpu):
        rt = self.rt
        if rt.recorder is not None:
            rt.recorder.append((self.layer_idx, sel_cpu.numpy().copy()))
        rt.stats["layer_calls"] += 1

    def _prefetch_next(self, pred_cpu, used_slots):
        nb = (self.layer_idx + 1) * self.E
        keys = [nb + int(e) for e in torch.unique(pred_cpu).tolist()]
        self.rt.stats["prefetched"] += self.rt.cache.prefetch(keys, used_slots)

    def _forward_fast(self, x, rw, sel, pred, B, T, H):
        """One token: one host sync, one native paging step, two decode kernels (moe.py:174-204)."""
        from .kernels import moe_decode_fast

        rt, cache, k = self.rt, self.rt.cache, self.top_k
        parts = [sel.float(), rw.float()] + ([pred.float()] if pred is not None else [])
        row = torch.cat(parts, 1).cpu()[0]  # the single sync of this layer
        ex = row[:k].to(torch.int64)
        self._record(ex.view(1, k))
        mm = getattr(rt, "_meta", None)
        if mm is None or mm[0].numel() != 2 * k or mm[1].device != x.device:
            mm = rt._meta = (torch.empty(2 * k, dtype=torch.float32, pin_memory=True),
                             torch.empty(2 * k, dtype=torch.float32, device=x.device))
        base = self.layer_idx * self.E
        slots = cache.prepare_layer([base + int(e) for e in ex], row[k : 2 * k].numpy(), mm[0], mm[1])
        y = moe_decode_fast(cache.gpu, mm[1], x[0], k, cache.store.n, H, self.I, cache.store.bits,
                            cache.store.group)
        rt.stats["gpu_experts"] += k
        if pred is not None:
            self._prefetch_next(row[2 * k :], slots)
        return y.view(B, T, H)

    def _forward_per_expert(self, x, rw, sel, pred, B, T, H):
        """One token through moe_decode_q4 (per-expert y, then the weighted sum), moe.py:111-121."""
        from .kernels import moe_decode_q4

        rt, cache, k = self.rt, self.rt.cache, self.top_k
        sel_cpu = sel.cpu()
        self._record(sel_cpu)
        base = self.layer_idx * self.E
        slots = cache.ensure([base + int(e) for e in sel_cpu[0]])
        y = moe_decode_q4(cache.gpu, torch.tensor(slots, device=x.device), x[0], rw[0], cache.store.n, H, self.I,
                          cache.store.group)
        rt.stats["gpu_experts"] += k
        if pred is not None:
            self._prefetch_next(pred.cpu(), slots)
        return y.view(B, T, H)

    def _forward_dequant(self, x, rw, sel, pred, B, T, H):
        """Several tokens (moe.py:82-151, 'transfer' policy), experts paged in chunks of rt.chunk.
        4/3/2-bit experts with group 128: the grouped prefill kernels (dequant into LDS + bf16
        MFMA, three launches per chunk, fp32 accumulation across chunks). Otherwise: per routed
        expert, dequantize its slot and run three bf16 GEMMs on its tokens."""
        rt, cache = self.rt, self.rt.cache
        sel_cpu = sel.cpu()
        self._record(sel_cpu)
        base = self.layer_idx * self.E
        keys = [base + int(e) for e in torch.unique(sel_cpu).tolist()]
        st = cache.store
        if st.bits in (2, 3, 4) and st.group == 128 and not cache.decode_on_load and x.dtype == torch.bfloat16:
            from .kernels import moe_prefill

            acc = torch.zeros((x.shape[0], H), dtype=torch.float32, device=x.device)
            used = []
            for i in range(0, len(keys), rt.chunk):
                ck = keys[i : i + rt.chunk]
                cs = cache.ensure(ck)
                moe_prefill(cache.gpu, {kk - base: s for kk, s in zip(ck, cs)}, x, sel_cpu, rw, st.n, H, self.I,
                            st.bits, st.group, acc=acc)
                rt.stats["gpu_experts"] += len(ck)
                used = list(cs)
            if pred is not None:
                self._prefetch_next(pred.cpu(), used)
            return acc.to(x.dtype).view(B, T, H)
        out = torch.zeros_like(x)
        used = []
        for i in range(0, len(keys), rt.chunk):
            ck = keys[i : i + rt.chunk]
            cs = cache.ensure(ck)
            for kk, W3 in zip(ck, cache.weights(cs)):
                tok, pos = torch.where(sel == kk - base)
                y = _expert_mlp(x[tok], W3, self.I, H) * rw[tok, pos].unsqueeze(-1)
                out.index_add_(0, tok, y)
                rt.stats["gpu_experts"] += 1
            used = list(cs)
        if pred is not None:
            self._prefetch_next(pred.cpu(), used)
        return out.view(B, T, H)


def attach(model, rt):
    """Replace every sparse-MoE block of a Qwen3-MoE model by a PagedMoEBlock, keeping its
    router (moe.py:207-222)."""
    cfg = model.config
    blocks = []
    for i, layer in enumerate(model.model.layers):
        old = layer.mlp
        if not hasattr(old, "gate"):
            blocks.append(None)
            continue
        blk = PagedMoEBlock(old.gate, i, rt, cfg)
        layer.mlp = blk
        blocks.append(blk)
    for i, b in enumerate(blocks[:-1]):
        if b is not None:
            b.set_next_gate(blocks[i + 1].gate if blocks[i + 1] is not None else None)
    return model
