"""The reference's CPU dequantize-then-matmul MoE path, restated with torch on host cores.

TEST/BENCH INFRASTRUCTURE ONLY (the `cpu_baseline` leg of bench.py): it is timed beside
the GPU kernels, never used by the product. It follows the reference's "hybrid" CPU
path: per selected expert, dequant the quantized row to bf16 [3, n]
(wisp/quant.py:76-87 via cache.py:137-142), run the expert MLP with three bf16
F.linear (wisp/moe.py:42-45), and add it scaled by its routing weight
(wisp/moe.py:159-161). scripts/microbench.py:74-88 times the same per-expert work.
"""

from __future__ import annotations

import os
import statistics
import time

import torch
import torch.nn.functional as F


def dequant_cpu(buf: torch.Tensor, n: int, bits: int, group: int = 128) -> torch.Tensor:
    """[B, nbytes] uint8 -> [B, 3, n] bf16 with torch CPU ops (quant.py:76-87 semantics)."""
    B = buf.shape[0]
    ncode = (3 * n * bits) // 8
    ng = 3 * n // group
    sc = buf[:, ncode : ncode + 2 * ng].contiguous().view(torch.float16)
    mn = buf[:, ncode + 2 * ng : ncode + 4 * ng].contiguous().view(torch.float16)
    c = buf[:, :ncode]
    if bits == 4:
        q = torch.stack([c & 15, c >> 4], -1).reshape(B, -1)
    elif bits == 2:
        q = torch.stack([(c >> (2 * i)) & 3 for i in range(4)], -1).reshape(B, -1)
    elif bits == 3:
        t = c.reshape(B, -1, 3).to(torch.int32)
        v = t[..., 0] | (t[..., 1] << 8) | (t[..., 2] << 16)
        q = torch.stack([(v >> (3 * i)) & 7 for i in range(8)], -1).reshape(B, -1)
    else:
        q = c
    w = q.reshape(B, ng, group).to(torch.float32) * sc.float().unsqueeze(-1) + mn.float().unsqueeze(-1)
    return w.to(torch.bfloat16).reshape(B, 3, n)


def _mlp(x, W3, I, H):
    g = F.linear(x, W3[0].view(I, H))
    u = F.linear(x, W3[1].view(I, H))
    return F.linear(F.silu(g) * u, W3[2].view(H, I))


def moe_layer_cpu(rows: torch.Tensor, slots, weights, x: torch.Tensor, H: int, I: int, bits: int, group: int = 128):
    """One batch-1 MoE layer: sum_j w_j * mlp_j(x) in bf16 on the host (moe.py:157-163)."""
    n = H * I
    y = torch.zeros(1, H, dtype=torch.bfloat16)
    for s, w in zip(slots, weights):
        W3 = dequant_cpu(rows[int(s)][None], n, bits, group)[0]
        y += _mlp(x.view(1, H), W3, I, H) * torch.tensor(float(w), dtype=torch.bfloat16)
    return y[0]


def time_layers(rows: torch.Tensor, routes, xs, H: int, I: int, bits: int, group: int = 128, budget_s: float = 15.0,
                warm: int = 5, threads: int | None = None):
    """Median seconds per layer over a bounded sample (stops after ~budget_s seconds), after
    `warm` untimed layers.
    `rows` are host expert buffers; `routes` is a list of (slots, weights); distinct
    experts are rotated so reads come from DRAM (microbench.py:78)."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    for i in range(warm):
        moe_layer_cpu(rows, *routes[i % len(routes)], xs[i % len(xs)], H, I, bits, group)
    ts = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while time.perf_counter() < t_end and i < 10000:
        t0 = time.perf_counter()
        moe_layer_cpu(rows, *routes[i % len(routes)], xs[i % len(xs)], H, I, bits, group)
        ts.append(time.perf_counter() - t0)
        i += 1
    return statistics.median(ts), len(ts), threads
