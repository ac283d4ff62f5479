"""Fused group-wise 4/3/2-bit dequant + GEMV for batch-1 MoE decode, on gfx950.

Same callable surface as the reference's wisp/kernels.py (imronpuji/wisp-runtime),
so the MoE layer, expert cache and graph decoder call it unchanged. The work is
done by hand-written HIP kernels in libwisp_hip.so reading the packed experts
straight out of the GPU slot pool:
  kernel 1:  a[j, r] = silu(Wg_j[r,:] . x) * (Wu_j[r,:] . x)        every expert j
  kernel 2:  out[h]  = sum_j w_j * (Wd_j[h,:] . a_j)                 (or per-expert y)
with the dequant folded into the dot product per group (kernels.py:12):
  sum_i (q_i*s + m) x_i = s*(q.x) + m*sum(x), accumulated in fp32.

Every call only enqueues kernels on the current torch stream; outputs and the
workspace come from torch.empty, so the calls can be captured into a graph. The
`block_*` / `num_warps` keyword arguments are the reference's Triton tiling knobs;
they are accepted and ignored (launch shapes are set by wisp_set_tuning).
"""

from __future__ import annotations

import torch

from . import _lib


_X_DTYPES = {torch.bfloat16: _lib.WISP_DT_BF16, torch.float16: _lib.WISP_DT_F16, torch.float32: _lib.WISP_DT_F32}


def _prep_x(x: torch.Tensor, dtypes=(torch.bfloat16,)) -> torch.Tensor:
    if x.dtype not in dtypes:
        raise TypeError(f"x must be one of {dtypes} (got {x.dtype})")
    x = x.reshape(-1).contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x


def _prep_x_any(x: torch.Tensor):
    """x of any float dtype, as the reference kernels load it (`.to(tl.float32)`,
    kernels.py:51-52): bf16, fp16 and fp32 go to the kernels as they are, float64 is
    rounded to fp32 first. Returns (x, its WISP_DT_* code)."""
    if not x.is_floating_point():
        raise TypeError(f"x must be a float tensor (got {x.dtype})")
    if x.dtype not in _X_DTYPES:
        x = x.to(torch.float32)
    x = _prep_x(x, tuple(_X_DTYPES))
    return x, _X_DTYPES[x.dtype]


def _check_pool(pool: torch.Tensor) -> None:
    assert pool.dtype == torch.uint8 and pool.dim() == 2 and pool.stride(1) == 1, (
        "pool must be a row-contiguous [nslots, slot_bytes] uint8 tensor"
    )


def _layer(pool, meta, x, k, n, H, I, group, bits):
    assert H % group == 0 and I % group == 0 and n == H * I
    assert 1 <= k <= _lib.WISP_MAX_K, f"k must be in [1, {_lib.WISP_MAX_K}]"
    _check_pool(pool)
    dev = _lib.require_gpu(pool, meta, x, what=f"moe_decode (bits={bits})")
    assert meta.dtype == torch.float32 and meta.numel() >= 2 * k, "meta must be float32 [2k]"
    meta = meta.contiguous()
    xk, xdt = _prep_x_any(x)
    assert xk.numel() == H
    act = torch.empty((k, I), dtype=torch.float32, device=dev).view(torch.int32)
    return dev, meta, xk, xdt, act


def moe_decode_fast(pool, meta, x, k, n, H, I, bits, group=128):
    """One batch-1 MoE layer: gate_up+SiLU, then down + routing-weighted sum, as two
    kernel launches (kernels.py:197-202). meta: float32 [2k] on the GPU =
    [slot_0..slot_{k-1}, w_0..w_{k-1}]; x: [H] of any float dtype. Returns [H] in
    x.dtype (the fp32 sum rounded once; float64 via fp32, as a Triton store would)."""
    dev, meta, xk, xdt, act = _layer(pool, meta, x, k, n, H, I, group, bits)
    out = torch.empty((H,), dtype=xk.dtype, device=dev)
    _lib.check(
        _lib.lib().wisp_moe_decode(
            _lib.ptr(pool), pool.stride(0), pool.shape[0], _lib.ptr(meta), k, _lib.ptr(xk), xdt, H, I, bits, group,
            _lib.ptr(act), _lib.ptr(out), xdt, _lib.stream(dev),
        ),
        "moe_decode",
    )
    return out if out.dtype == x.dtype else out.to(x.dtype)


def moe_decode_q4_fast(pool, meta, x, k, n, H, I, group=128, block_gu=32, block_down=8, num_warps=4):
    """kernels.py:188-203: 4-bit, 2 kernel launches in total, one packed routing buffer.
    meta: float32 [2k] on the GPU = [slot_0..slot_{k-1}, w_0..w_{k-1}]. Returns [H] in x.dtype."""
    return moe_decode_fast(pool, meta, x, k, n, H, I, 4, group)


def moe_decode_q3_fast(pool, meta, x, k, n, H, I, group=128, block_gu=8, block_down=8, num_warps=4):
    """kernels.py:310-322: 3-bit twin of moe_decode_q4_fast (same meta layout)."""
    return moe_decode_fast(pool, meta, x, k, n, H, I, 3, group)


def moe_decode_q2_fast(pool, meta, x, k, n, H, I, group=128, block_gu=8, block_down=8, num_warps=4):
    """2-bit twin of moe_decode_q4_fast. The reference packs 2-bit experts (quant.py:32-34)
    but has no fused 2-bit kernel; this one follows the same semantics."""
    return moe_decode_fast(pool, meta, x, k, n, H, I, 2, group)


def moe_decode_q4(pool, slots, x, w, n, H, I, group=128, block_r=32, num_warps=4):
    """kernels.py:115-137. pool: [nslots, nbytes] uint8 (4-bit experts); slots: int64 [k];
    x: [H] of any float dtype; w: [k] routing weights. Per-expert y[k, H] from the kernels, then the
    weighted sum in fp32 and the cast to x.dtype, as the reference does."""
    k = slots.numel()
    meta = torch.cat([slots.reshape(-1).to(torch.float32), w.reshape(-1).to(torch.float32)])
    dev, meta, xk, xdt, act = _layer(pool, meta, x, k, n, H, I, group, 4)
    L = _lib.lib()
    st = _lib.stream(dev)
    args = (_lib.ptr(pool), pool.stride(0), pool.shape[0], _lib.ptr(meta), k)
    _lib.check(L.wisp_moe_gate_up(*args, _lib.ptr(xk), xdt, H, I, 4, group, _lib.ptr(act), st),
               "moe_decode_q4 gate_up")
    y = torch.empty((k, H), dtype=torch.float32, device=dev)
    _lib.check(L.wisp_moe_down(*args, _lib.ptr(act), H, I, 4, group, _lib.ptr(y), st), "moe_decode_q4 down")
    return (y * w.float().unsqueeze(1)).sum(0).to(x.dtype)


def gate_up_act(pool, meta, x, k, n, H, I, bits, group=128) -> torch.Tensor:
    """Kernel 1 alone, decoded to fp32 a [k, I] (for checks of the first kernel)."""
    dev, meta, xk, xdt, act = _layer(pool, meta, x, k, n, H, I, group, bits)
    L = _lib.lib()
    st = _lib.stream(dev)
    _lib.check(
        L.wisp_moe_gate_up(
            _lib.ptr(pool), pool.stride(0), pool.shape[0], _lib.ptr(meta), k, _lib.ptr(xk), xdt, H, I, bits, group,
            _lib.ptr(act), st,
        ),
        "gate_up",
    )
    a = torch.empty((k, I), dtype=torch.float32, device=dev)
    _lib.check(L.wisp_act_read(_lib.ptr(act), k, I, bits, _lib.ptr(a), st), "act_read")
    return a


def set_tuning(gu_rows: int = 0, gu_waves: int = 0, dn_iters: int = 0) -> None:
    """Launch-shape knobs of the two decode kernels (0 keeps the current value)."""
    _lib.check(_lib.lib().wisp_set_tuning(gu_rows, gu_waves, dn_iters), "set_tuning")


_ROPE_DTYPES = {torch.float32: 0, torch.bfloat16: 1}


def rope_decode(q, k, cos, sin):
    """kernels.py:352-371. q: [1,Hq,1,D], k: [1,Hk,1,D] (HF layout, possibly strided views),
    cos/sin: [1,1,D] -> rotated (qo, ko), same shapes, contiguous, in q's dtype. One launch."""
    Hq, D = q.shape[1], q.shape[3]
    Hk = k.shape[1]
    dev = _lib.require_gpu(q, k, cos, sin, what="rope_decode")
    dt = _ROPE_DTYPES.get(q.dtype)
    if dt is None or k.dtype != q.dtype:
        raise TypeError(f"rope_decode supports float32 and bfloat16 q/k of one dtype (got {q.dtype}, {k.dtype})")
    if q.stride(3) != 1:
        q = q.contiguous()
    if k.stride(3) != 1:
        k = k.contiguous()
    cos = cos.reshape(-1).to(q.dtype).contiguous()
    sin = sin.reshape(-1).to(q.dtype).contiguous()
    assert cos.numel() == D and sin.numel() == D
    qo = torch.empty((1, Hq, 1, D), dtype=q.dtype, device=dev)
    ko = torch.empty((1, Hk, 1, D), dtype=k.dtype, device=dev)
    _lib.check(
        _lib.lib().wisp_rope_decode(
            _lib.ptr(q), q.stride(1), _lib.ptr(k), k.stride(1), _lib.ptr(cos), _lib.ptr(sin), Hq, Hk, D, dt,
            _lib.ptr(qo), _lib.ptr(ko), _lib.stream(dev),
        ),
        "rope_decode",
    )
    return qo, ko


def attn_decode(q, kc, vc, pos, scale):
    """Masked grouped attention of one decode token over a static KV cache (the
    scaled_dot_product_attention of graphdec.py:171-174), as two HIP launches.
    q: [1, Hq, 1, D] or [Hq, D] bf16; kc, vc: [1, Hk, Tmax, D] bf16 (contiguous rows);
    pos: int64 device tensor (one element, read at run time; positions <= pos attend).
    Returns [1, Hq, 1, D] bf16."""
    Hq, D = q.shape[-3] if q.dim() == 4 else q.shape[0], q.shape[-1]
    Hk, tmax = kc.shape[1], kc.shape[2]
    dev = _lib.require_gpu(q, kc, vc, pos, what="attn_decode")
    if q.dtype != torch.bfloat16 or kc.dtype != torch.bfloat16 or vc.dtype != torch.bfloat16:
        raise TypeError("attn_decode takes bfloat16 q, k and v")
    assert kc.shape == vc.shape and kc.stride(-1) == 1 and kc.stride(-2) == D and vc.stride() == kc.stride()
    assert pos.dtype == torch.int64 and pos.numel() >= 1
    q = q.reshape(Hq, D).contiguous()
    L = _lib.lib()
    ws = torch.empty(L.wisp_attn_ws_bytes(Hq, D, tmax), dtype=torch.uint8, device=dev)
    out = torch.empty((1, Hq, 1, D), dtype=torch.bfloat16, device=dev)
    _lib.check(
        L.wisp_attn_decode(
            _lib.ptr(q), _lib.ptr(kc), _lib.ptr(vc), kc.stride(1), _lib.ptr(pos), Hq, Hk, D, tmax, float(scale),
            _lib.ptr(ws), _lib.ptr(out), _lib.stream(dev),
        ),
        "attn_decode",
    )
    return out


def _prefill_plan(sel_cpu, experts, k):
    """Host-side grouping of the (token, expert) pairs whose expert is in `experts`:
    pairs sorted by expert (tokens ascending within an expert), the per-expert
    (first pair, count), and back[t, j] = pair of token t's j-th expert in ascending
    expert id (-1 when that expert is not in `experts`)."""
    import numpy as np

    T = sel_cpu.shape[0]
    flat = sel_cpu.reshape(-1)
    keep = np.isin(flat, np.asarray(experts, dtype=flat.dtype))
    idx = np.flatnonzero(keep)
    order = idx[np.argsort(flat[idx], kind="stable")]  # original pair ids, sorted by expert
    pair_of = np.full(T * k, -1, np.int64)
    pair_of[order] = np.arange(order.size)
    rank = np.argsort(sel_cpu, axis=1, kind="stable")  # token t's experts in ascending id
    back = np.take_along_axis(pair_of.reshape(T, k), rank, axis=1)
    ex_sorted = flat[order]
    uniq, first, count = np.unique(ex_sorted, return_index=True, return_counts=True)
    return order, (order // k).astype(np.int32), back.astype(np.int32), uniq, first, count


def _prefill_chunks(uniq, first, count, chunk=None):
    """Split each expert's pair range into work items of at most `chunk` pairs, the
    largest first. Each item becomes one group of the launch, so every workgroup
    of the grid has work (a launch sized for the largest group would hold idle
    workgroups that wait for a free slot before they can exit) and the longest
    items start first. Default chunk: 128 pairs, one pass of up to 8 token tiles, so an
    item dequantizes its expert's rows once for up to 128 tokens (4-bit LDS-DMA kernels;
    other shapes run a group of more than 64 pairs as passes of 64 on separate
    workgroups). Measured on C5, interleaved in one process: T = 256 98.3 -> 94.4 us and
    T = 512 117.6 -> 114.9 us against 64-pair items, 96 no better."""
    import numpy as np

    if chunk is None:
        chunk = 128
    n = (count + chunk - 1) // chunk
    ex = np.repeat(uniq, n)
    start = np.repeat(first, n) + (np.arange(n.sum()) - np.repeat(np.cumsum(n) - n, n)) * chunk
    cnt = np.minimum(np.repeat(first + count, n) - start, chunk)
    o = np.argsort(-cnt, kind="stable")
    return ex[o], start[o], cnt[o]


def moe_prefill(pool, expert_slots, x, sel, rw, n, H, I, bits, group=128, acc=None):
    """Grouped MoE over T tokens (the dequant + F.linear loop of moe.py:131-151 as three
    launches). x: [T, H] bf16; sel: [T, k] expert ids; rw: [T, k] routing weights;
    expert_slots: {expert id: slot} for the experts to run (others are skipped).
    Returns bf16 [T, H] = per token sum over its experts (ascending id) of
    w * down(SiLU(gate x) * up x); with `acc` (fp32 [T, H]) the sum is added to it instead
    (chunks of experts) and acc is returned."""
    import numpy as np

    assert n == H * I and H % group == 0 and I % group == 0
    _check_pool(pool)
    dev = _lib.require_gpu(pool, x, what="moe_prefill")
    x = x.reshape(-1, H)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16 (got {x.dtype})")
    x = x.contiguous()
    T, k = sel.shape
    sel_cpu = sel.detach().cpu().numpy()
    experts = sorted(int(e) for e in expert_slots)
    order, tok, back, uniq, first, count = _prefill_plan(sel_cpu, experts, k)
    P = int(order.size)
    if acc is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    else:
        assert acc.dtype == torch.float32 and acc.shape == (T, H) and acc.is_contiguous()
        out = None
    if P == 0:
        if out is not None:
            out.zero_()
        return acc if out is None else out
    uniq, first, count = _prefill_chunks(uniq, first, count)
    groups = np.stack([np.array([expert_slots[int(e)] for e in uniq], np.int64), first, count], 1).astype(np.int32)
    ints = torch.from_numpy(np.concatenate([groups.reshape(-1), tok, back.reshape(-1)])).to(dev, non_blocking=True)
    g_dev = ints[: groups.size]
    tok_dev = ints[groups.size : groups.size + P]
    back_dev = ints[groups.size + P :]
    w_pairs = rw.reshape(-1).to(device=dev, dtype=torch.float32)
    w_pairs = w_pairs.index_select(0, torch.from_numpy(order).to(dev, non_blocking=True)).contiguous()
    L = _lib.lib()
    ws = torch.empty(L.wisp_prefill_ws_bytes(P, H, I), dtype=torch.uint8, device=dev)
    _lib.check(
        L.wisp_moe_prefill(
            _lib.ptr(pool), pool.stride(0), pool.shape[0], _lib.ptr(g_dev), len(uniq), int(count.max()), _lib.ptr(tok_dev),
            _lib.ptr(w_pairs), _lib.ptr(back_dev), P, _lib.ptr(x), T, k, H, I, bits, group, _lib.ptr(ws),
            _lib.ptr(out), _lib.ptr(acc), _lib.stream(dev),
        ),
        "moe_prefill",
    )
    return acc if out is None else out


# ---------------------------------------------------------------------------- gpt-oss
def mxfp4_to_bf16(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """gptoss.py:22-29: blocks [..., G, 16] uint8 (two e2m1 codes per byte, low nibble
    first), scales [..., G] uint8 (power-of-two exponents, bias 127) -> [..., G*32]
    bfloat16, bit-exact with the reference (float32 product, then .to(bfloat16))."""
    assert blocks.dtype == torch.uint8 and scales.dtype == torch.uint8 and blocks.shape[-1] == 16
    assert tuple(blocks.shape[:-1]) == tuple(scales.shape), "scales must be blocks.shape[:-1]"
    dev = _lib.require_gpu(blocks, scales, what="mxfp4_to_bf16")
    b = blocks.contiguous()
    if b.data_ptr() % 16:
        b = b.clone()
    s = scales.contiguous()
    ng = s.numel()
    out = torch.empty(ng * 32, dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.lib().wisp_mxfp4_to_bf16(_lib.ptr(b), _lib.ptr(s), ng, _lib.ptr(out), _lib.stream(dev)),
               "mxfp4_to_bf16")
    return out.view(*blocks.shape[:-2], blocks.shape[-2] * 32)


def gptoss_decode(pool, meta, x, gate_up_bias, down_bias, k, n, H, I, bits, group=128, alpha=1.702, limit=7.0):
    """One token through k gpt-oss experts (PagedGptOssBlock's decode step,
    gptoss.py:126-131) as three kernel launches. meta: float32 [3k] on the GPU =
    [slot ids | routing weights | expert ids]; gate_up_bias bf16 [E, 2I], down_bias
    bf16 [E, H] indexed by expert id. Returns bf16 [H]."""
    assert n == H * I
    _check_pool(pool)
    dev = _lib.require_gpu(pool, meta, x, gate_up_bias, down_bias, what=f"gptoss_decode (bits={bits})")
    assert meta.dtype == torch.float32 and meta.numel() >= 3 * k, "meta must be float32 [3k]"
    assert gate_up_bias.dtype == torch.bfloat16 and down_bias.dtype == torch.bfloat16
    E = gate_up_bias.shape[0]
    assert gate_up_bias.shape == (E, 2 * I) and down_bias.shape == (E, H), "biases must be [E, 2I] and [E, H]"
    meta = meta.contiguous()
    x = _prep_x(x)
    assert x.numel() == H
    gub, db = gate_up_bias.contiguous(), down_bias.contiguous()
    L = _lib.lib()
    ws = torch.empty(L.wisp_gptoss_ws_bytes(k, H, I), dtype=torch.uint8, device=dev)
    out = torch.empty((H,), dtype=torch.bfloat16, device=dev)
    _lib.check(
        L.wisp_gptoss_decode(
            _lib.ptr(pool), pool.stride(0), pool.shape[0], _lib.ptr(meta), k, H, I, bits, group, _lib.ptr(x),
            _lib.ptr(gub), _lib.ptr(db), E, float(alpha), float(limit), _lib.ptr(ws), _lib.ptr(out), _lib.stream(dev),
        ),
        "gptoss_decode",
    )
    return out


# ----------------------------------------------------------------------------- decode-step dense kernels
def _bf16_vec(t, what):
    if t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise TypeError(f"{what} must be a contiguous bfloat16 tensor")
    return t


def dl_gemv(y, w0, a, *, w1=None, w2=None, r1=None, r2=None, a_row=None, b=None, norm_w=None, eps=0.0, h_out=None,
            x_out=None, res=None):
    """y[o] = bf16(W[o] . x) for a bf16 weight W [O, K] given as up to three row blocks
    (w0: rows [0, r1), w1: [r1, r2), w2: [r2, O)), one launch. With norm_w, x is the
    RMSNorm of h = a (+ b) (Qwen3MoeRMSNorm at bf16; h and x optionally stored to h_out and
    x_out); otherwise x = a. a_row (int64 device tensor): use row a_row of a [*, K]. res:
    y = bf16(res + bf16(W x)). Replaces the nn.Linear / RMSNorm / residual modules of
    graphdec.py:160-203 at batch 1. All tensors are caller-owned (graph-capture safe)."""
    blocks = [w for w in (w0, w1, w2) if w is not None]
    K = w0.shape[1]
    O = sum(w.shape[0] for w in blocks)
    r1 = w0.shape[0] if r1 is None else r1
    r2 = r1 + (w1.shape[0] if w1 is not None else 0) if r2 is None else r2
    for w in blocks:
        _bf16_vec(w, "weight")
        assert w.dim() == 2 and w.shape[1] == K
    _bf16_vec(y, "y")
    assert y.numel() == O and a.dtype == torch.bfloat16
    dev = _lib.require_gpu(y, w0, a, what="dl_gemv")
    if a_row is not None:
        assert a_row.dtype == torch.int64 and a.dim() == 2 and a.shape[1] == K and a.is_contiguous()
    else:
        assert a.numel() == K and a.is_contiguous()
    for t, n in ((b, "b"), (norm_w, "norm_w"), (h_out, "h_out"), (x_out, "x_out")):
        if t is not None:
            _bf16_vec(t, n)
            assert t.numel() == K, n
    if res is not None:
        _bf16_vec(res, "res")
        assert res.numel() == O
    p = lambda t: None if t is None else _lib.ptr(t)  # noqa: E731
    _lib.check(
        _lib.lib().wisp_dl_gemv(p(a), p(a_row), p(b), p(norm_w), float(eps), p(h_out), p(x_out), p(w0), p(w1), p(w2),
                                r1, r2, O, K, p(res), p(y), _lib.stream(dev)),
        "dl_gemv",
    )
    return y


def dl_qk_rope(qkv, q_norm_w, k_norm_w, eps, cos, sin, pos, hq, hk, d, kc, vc, qo):
    """Per-head RMSNorm of the q and k heads of qkv = [q (hq*d) | k (hk*d) | v (hk*d)],
    rope_decode at position `pos` (int64 device tensor) with the bf16 tables cos/sin
    [tmax, d], q -> qo [hq*d], k and v -> the static caches kc/vc [1, hk, tmax, d] at pos.
    Replaces graphdec.py:163-172 (q_norm, k_norm, rope_decode, index_copy_)."""
    for t, n in ((qkv, "qkv"), (q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w"), (cos, "cos"), (sin, "sin"),
                 (qo, "qo")):
        _bf16_vec(t, n)
    assert qkv.numel() == (hq + 2 * hk) * d and qo.numel() == hq * d
    assert kc.shape == vc.shape and kc.shape[1] == hk and kc.shape[3] == d and kc.stride() == vc.stride()
    assert kc.stride(-1) == 1 and kc.stride(-2) == d and cos.shape[-1] == d and sin.shape == cos.shape
    assert pos.dtype == torch.int64
    dev = _lib.require_gpu(qkv, kc, vc, pos, what="dl_qk_rope")
    _lib.check(
        _lib.lib().wisp_dl_qk_rope(_lib.ptr(qkv), _lib.ptr(q_norm_w), _lib.ptr(k_norm_w), float(eps), _lib.ptr(cos),
                                   _lib.ptr(sin), _lib.ptr(pos), hq, hk, d, _lib.ptr(kc), _lib.ptr(vc), kc.stride(1),
                                   _lib.ptr(qo), _lib.stream(dev)),
        "dl_qk_rope",
    )
    return qo


def dl_qk_rope_attn(qkv, q_norm_w, k_norm_w, eps, cos, sin, pos, hq, hk, d, kc, vc, scale):
    """dl_qk_rope followed by attn_decode on its q heads, in one pair of launches (the q/k
    head norm, rope and K/V store at pos run inside the attention workgroups; the same
    bits as the two calls). Replaces graphdec.py:163-174 at batch 1. Returns
    [1, hq, 1, d] bf16."""
    for t, n in ((qkv, "qkv"), (q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w"), (cos, "cos"), (sin, "sin")):
        _bf16_vec(t, n)
    assert qkv.numel() == (hq + 2 * hk) * d
    assert kc.shape == vc.shape and kc.shape[1] == hk and kc.shape[3] == d and kc.stride() == vc.stride()
    assert kc.stride(-1) == 1 and kc.stride(-2) == d and cos.shape[-1] == d and sin.shape == cos.shape
    assert kc.dtype == torch.bfloat16 and vc.dtype == torch.bfloat16
    assert pos.dtype == torch.int64 and pos.numel() >= 1
    dev = _lib.require_gpu(qkv, kc, vc, pos, what="dl_qk_rope_attn")
    tmax = kc.shape[2]
    L = _lib.lib()
    ws = torch.empty(L.wisp_attn_ws_bytes(hq, d, tmax), dtype=torch.uint8, device=dev)
    out = torch.empty((1, hq, 1, d), dtype=torch.bfloat16, device=dev)
    _lib.check(
        L.wisp_attn_decode_qk(_lib.ptr(qkv), _lib.ptr(q_norm_w), _lib.ptr(k_norm_w), float(eps), _lib.ptr(cos),
                              _lib.ptr(sin), _lib.ptr(pos), hq, hk, d, _lib.ptr(kc), _lib.ptr(vc), kc.stride(1), tmax,
                              float(scale), _lib.ptr(ws), _lib.ptr(out), _lib.stream(dev)),
        "dl_qk_rope_attn",
    )
    return out


def dl_route(logits, k, norm_topk, row, host_row=None, host_flag=None, seq=None):
    """route() of wisp/moe.py:41-47 at batch 1 on the device: softmax (float32) of the bf16
    router logits [E], top-k, renormalised if norm_topk, weights rounded to bf16;
    row[:k] = expert ids (float32), row[k:2k] = weights. One launch. With host_row (pinned
    float32 [>= 2k]), host_flag (pinned int32 [1]) and seq (device int32 [1]) the row is also
    written to host_row and then host_flag = ++seq, for a host that waits on the flag."""
    _bf16_vec(logits, "logits")
    assert row.dtype == torch.float32 and row.is_contiguous() and row.numel() >= 2 * k
    dev = _lib.require_gpu(logits, row, what="dl_route")
    hr = hf = sq = None
    if host_row is not None:
        assert host_row.is_pinned() and host_flag.is_pinned() and host_row.dtype == torch.float32
        assert host_row.numel() >= 2 * k and host_flag.dtype == torch.int32 and seq.is_cuda
        hr, hf, sq = _lib.ptr(host_row), _lib.ptr(host_flag), _lib.ptr(seq)
    _lib.check(_lib.lib().wisp_dl_route(_lib.ptr(logits), logits.numel(), k, int(bool(norm_topk)), _lib.ptr(row),
                                        hr, hf, sq, _lib.stream(dev)), "dl_route")
    return row
