"""Routing for batch-1 MoE decode: router logits -> top-k experts -> packed meta buffer.

The reference does this inside PagedMoEBlock.forward (wisp/moe.py:67-72) and
GraphDecoder._attn_router (wisp/graphdec.py:177-181): softmax in float32, top-k,
renormalise (norm_topk_prob), round the weights to the activation dtype (bf16), then
pack [slot ids..., weights...] as float32 for the fused kernels (moe.py:181-197).
These are torch device ops on the GPU; the slot ids come from the expert cache.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


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
