"""CPU oracle for the fused group-wise expert dequant+GEMV path (numpy front end).

TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against. Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may
import it; the product package never does.

The arithmetic lives in ``wisp_oracle.c`` (built to ``liboracle_wisp.so`` by
``oracle/Makefile``); this module wraps it with numpy arrays and adds the
routing step of the caller, the decode attention and the grouped prefill (binary64
numpy). Each function names the reference lines it restates.

Pins of the numpy-side functions (tests/test_oracle.py): route -> torch's softmax/topk;
attn_decode -> torch's scaled_dot_product_attention with repeated KV heads, the
one-position and equal-key closed forms, a head-mapping slip; moe_prefill_f64 -> the
decode-layer oracle at one token, additivity over experts, token equivariance, a
gate/up swap.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_wisp.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle with its Makefile (gcc); returns the .so path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True, capture_output=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        L.wo_f32_to_f16.restype, L.wo_f32_to_f16.argtypes = ctypes.c_uint16, [ctypes.c_float]
        L.wo_f16_to_f32.restype, L.wo_f16_to_f32.argtypes = ctypes.c_float, [ctypes.c_uint16]
        L.wo_f32_to_bf16.restype, L.wo_f32_to_bf16.argtypes = ctypes.c_uint16, [ctypes.c_float]
        L.wo_expert_nbytes.restype, L.wo_expert_nbytes.argtypes = i64, [i64, i32, i64]
        L.wo_pack.restype, L.wo_pack.argtypes = i32, [vp, i64, i32, vp]
        L.wo_unpack.restype, L.wo_unpack.argtypes = i32, [vp, i64, i32, vp]
        L.wo_q3_field.restype, L.wo_q3_field.argtypes = i32, [vp, i64]
        L.wo_quantize.restype, L.wo_quantize.argtypes = i32, [vp, i64, i32, i64, vp, vp]
        L.wo_dequant.restype, L.wo_dequant.argtypes = i32, [vp, i64, i32, i64, vp]
        L.wo_moe_layer_f64.restype = i32
        L.wo_moe_layer_f64.argtypes = [vp, i64, i64, vp, vp, i32, vp, i64, i64, i32, i64, vp, vp, vp]
        L.wo_moe_layer_f64x.restype = i32
        L.wo_moe_layer_f64x.argtypes = [vp, i64, i64, vp, vp, i32, vp, i64, i64, i32, i64, vp, vp, vp]
        L.wo_rope.restype, L.wo_rope.argtypes = i32, [vp, i64, i32, vp, vp, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- scalar conversions
def f32_to_f16_bits(a) -> np.ndarray:
    """binary32 -> binary16 bits, RTNE (torch .half(); quant.py:70)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    f = lib().wo_f32_to_f16
    return np.fromiter((f(float(v)) for v in a), dtype=np.uint16, count=a.size)


def f32_to_bf16_bits(a) -> np.ndarray:
    """binary32 -> bf16 bits, RTNE (torch .to(bfloat16); quant.py:87). Vectorised
    integer-add form of round-to-nearest-even, identical to wo_f32_to_bf16."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- layout / packing
def expert_nbytes(n: int, bits: int, group: int) -> int:
    """quant.py:17-22. Raises ValueError where the reference asserts."""
    v = lib().wo_expert_nbytes(n, bits, group)
    if v < 0:
        raise ValueError((n, bits, group))
    return int(v)


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """quant.py:25-41."""
    q = np.ascontiguousarray(q, dtype=np.uint8).ravel()
    out = np.empty(q.size * bits // 8, dtype=np.uint8)
    if lib().wo_pack(_p(q), q.size, bits, _p(out)) != 0:
        raise ValueError(bits)
    return out


def unpack(c: np.ndarray, bits: int, m: int | None = None) -> np.ndarray:
    """quant.py:44-57 (m codes out of packed bytes)."""
    c = np.ascontiguousarray(c, dtype=np.uint8).ravel()
    m = c.size * 8 // bits if m is None else m
    out = np.empty(m, dtype=np.uint8)
    if lib().wo_unpack(_p(c), m, bits, _p(out)) != 0:
        raise ValueError(bits)
    return out


def q3_field(buf: np.ndarray, e: int) -> int:
    """kernels.py:209-217: the kernels' own statement of the 3-bit read."""
    buf = np.ascontiguousarray(buf, dtype=np.uint8)
    return int(lib().wo_q3_field(_p(buf), e))


# ---------------------------------------------------------------- quantize / dequant
def quantize(w3: np.ndarray, bits: int, group: int = 128) -> np.ndarray:
    """quant.py:60-73. w3: [3, n] (or flat 3n) float32 -> flat uint8 buffer."""
    w = np.ascontiguousarray(w3, dtype=np.float32).ravel()
    assert w.size % 3 == 0
    n = w.size // 3
    out = np.empty(expert_nbytes(n, bits, group), dtype=np.uint8)
    scratch = np.empty(w.size, dtype=np.uint8)
    if lib().wo_quantize(_p(w), n, bits, group, _p(out), _p(scratch)) != 0:
        raise ValueError((n, bits, group))
    return out


def dequant(buf: np.ndarray, n: int, bits: int, group: int = 128) -> np.ndarray:
    """quant.py:76-87. buf: [B, >=nbytes] uint8 -> [B, 3, n] bf16 bit patterns (uint16)."""
    buf = np.ascontiguousarray(buf, dtype=np.uint8)
    if buf.ndim == 1:
        buf = buf[None]
    nb = expert_nbytes(n, bits, group)
    out = np.empty((buf.shape[0], 3, n), dtype=np.uint16)
    for b in range(buf.shape[0]):
        row = np.ascontiguousarray(buf[b, :nb])
        o = out[b]
        if lib().wo_dequant(_p(row), n, bits, group, _p(o)) != 0:
            raise ValueError((n, bits, group))
    return out


# ---------------------------------------------------------------- fused layer
def moe_layer_f64(pool: np.ndarray, slots, w, x_bf16: np.ndarray, H: int, I: int, bits: int, group: int = 128):
    """Binary64 statement of one batch-1 MoE layer with the fused kernels' semantics
    (kernels.py:12, 20-69, 72-112, 140-185, 220-307): returns (a [k,I], y [k,H], out [H]),
    all float64 and unrounded. `w` are the routing weights the kernels read (float32 values).
    x_bf16: uint16 bf16 bit patterns, or x as float16/float32/float64 values (the reference
    kernels widen any float x exactly, kernels.py:51-52)."""
    pool = np.ascontiguousarray(pool, dtype=np.uint8)
    slots = np.ascontiguousarray(slots, dtype=np.int64).ravel()
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    xin = np.asarray(x_bf16)
    k = slots.size
    assert w.size == k and xin.size == H
    a = np.empty((k, I), dtype=np.float64)
    y = np.empty((k, H), dtype=np.float64)
    out = np.empty(H, dtype=np.float64)
    if xin.dtype == np.uint16:
        x = np.ascontiguousarray(xin).ravel()
        fn = lib().wo_moe_layer_f64
    else:
        assert xin.dtype in (np.float16, np.float32, np.float64), xin.dtype
        x = np.ascontiguousarray(xin, dtype=np.float64).ravel()
        fn = lib().wo_moe_layer_f64x
    rc = fn(_p(pool), pool.shape[1], pool.shape[0], _p(slots), _p(w), k, _p(x), H, I, bits, group, _p(a), _p(y),
            _p(out))
    if rc != 0:
        raise ValueError("bad arguments to moe_layer_f64")
    return a, y, out


# ---------------------------------------------------------------- routing (caller side)
def route(logits: np.ndarray, k: int, norm_topk: bool = True):
    """moe.py:67-72 / graphdec.py:177-181: softmax in float32 -> top-k -> renormalise ->
    round the weights to bf16. Returns (experts int64 [N,k], weights float32 [N,k] holding
    the bf16-rounded values, i.e. what the meta buffer carries)."""
    lg = np.asarray(logits, dtype=np.float32)
    if lg.ndim == 1:
        lg = lg[None]
    m = lg.max(axis=1, keepdims=True)
    e = np.exp((lg - m).astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    sel = np.argsort(-p, axis=1, kind="stable")[:, :k]
    rw = np.take_along_axis(p, sel, axis=1)
    if norm_topk:
        rw = (rw / rw.sum(axis=1, keepdims=True)).astype(np.float32)
    rw_b = bf16_bits_to_f32(f32_to_bf16_bits(rw)).reshape(rw.shape)
    return sel.astype(np.int64), rw_b


def meta(slots, weights) -> np.ndarray:
    """The packed routing buffer the fast kernels read (kernels.py:189-190, 167-168;
    moe.py:190-197): float32 [2k] = [slot ids as float32 ..., weights ...]."""
    s = np.asarray(slots, dtype=np.int64).ravel()
    assert np.all(s < (1 << 24)), "slot ids must be exact in float32"
    return np.concatenate([s.astype(np.float32), np.asarray(weights, dtype=np.float32).ravel()])


# ---------------------------------------------------------------- rotary (decode)
def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """kernels.py:325-349: rotate head vectors x [nh, d] (float32 values) by cos/sin [d]
    in binary32 with separately rounded products and sum. Returns float32 [nh, d]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nh, d = x.shape
    c = np.ascontiguousarray(cos, dtype=np.float32).ravel()
    s = np.ascontiguousarray(sin, dtype=np.float32).ravel()
    assert c.size == d and s.size == d
    out = np.empty_like(x)
    if lib().wo_rope(_p(x), nh, d, _p(c), _p(s), _p(out)) != 0:
        raise ValueError("bad arguments to rope")
    return out


# ---------------------------------------------------------------- decode attention
def attn_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, pos: int, scale: float) -> np.ndarray:
    """graphdec.py:171-174 in binary64: q [Hq, D], k/v [Hk, T, D] (float values), positions
    0..pos attend; query head h uses KV head h // (Hq/Hk). Returns float64 [Hq, D]."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    Hq, Hk = q.shape[0], k.shape[0]
    G = Hq // Hk
    out = np.empty_like(q)
    for h in range(Hq):
        s = (k[h // G, : pos + 1] @ q[h]) * scale
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[h // G, : pos + 1]
    return out


# ---------------------------------------------------------------- grouped prefill (moe.py:131-151)
def moe_prefill_f64(pool: np.ndarray, expert_slots: dict, x_bf16: np.ndarray, sel: np.ndarray, rw: np.ndarray,
                    H: int, I: int, bits: int, group: int = 128) -> np.ndarray:
    """The per-expert dequant -> MLP -> weighted sum of moe.py:131-151 in binary64, with the
    weights dequantized bit-exactly to bf16 (quant.py:76-87, as the reference's F.linear
    sees them) and the activation between the two GEMMs rounded to bf16 (the operand type
    of both the reference's second F.linear and the MFMA). x_bf16: uint16 [T, H];
    sel/rw: [T, k]. Experts missing from expert_slots are skipped. Returns float64 [T, H]."""
    x = bf16_bits_to_f32(np.asarray(x_bf16, np.uint16)).reshape(-1, H).astype(np.float64)
    sel = np.asarray(sel)
    rw = np.asarray(rw, np.float64)
    T = x.shape[0]
    n = H * I
    out = np.zeros((T, H), np.float64)
    for e in sorted(int(v) for v in np.unique(sel)):
        if e not in expert_slots:
            continue
        W = bf16_bits_to_f32(dequant(pool[expert_slots[e]][None], n, bits, group)[0]).astype(np.float64)
        Wg, Wu, Wd = W[0].reshape(I, H), W[1].reshape(I, H), W[2].reshape(H, I)
        tt, jj = np.nonzero(sel == e)
        g, u = x[tt] @ Wg.T, x[tt] @ Wu.T
        a = g / (1.0 + np.exp(-g)) * u
        a = bf16_bits_to_f32(f32_to_bf16_bits(a.astype(np.float32))).reshape(a.shape).astype(np.float64)
        out[tt] += rw[tt, jj][:, None] * (a @ Wd.T)
    return out


# ---------------------------------------------------------------- gpt-oss experts
# e2m1 code -> value (gptoss.py:19)
FP4 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def _bf16r(a) -> np.ndarray:
    """Round binary32 values through bf16 (RTNE) and back, as a bf16 tensor op does."""
    a = np.asarray(a, np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(a)).reshape(a.shape)


def mxfp4_to_bf16_bits(blocks, scales) -> np.ndarray:
    """gptoss.py:22-29. blocks [..., G, 16] uint8 (low nibble first), scales [..., G] uint8
    -> bf16 bits [..., G*32]: binary32 FP4[code] * 2^(scale - 127) (exact, or inf/NaN for
    scale 255), then torch's .to(bfloat16): RTNE, every NaN -> 0x7FC0."""
    b = np.asarray(blocks, np.uint8)
    s = np.asarray(scales, np.uint8)
    lut = np.array(FP4, np.float32)
    v = np.stack([lut[b & 15], lut[b >> 4]], -1).reshape(*b.shape[:-1], 32)
    with np.errstate(invalid="ignore", over="ignore"):
        p = np.ldexp(np.float32(1.0), s.astype(np.int32) - 127).astype(np.float32)  # exact powers of two
        v = (v * p[..., None]).astype(np.float32)
    out = f32_to_bf16_bits(v).reshape(v.shape)
    out[np.isnan(v)] = 0x7FC0
    return out.reshape(*b.shape[:-2], b.shape[-2] * 32)


def gptoss_act(gu: np.ndarray, alpha: float = 1.702, limit: float = 7.0) -> np.ndarray:
    """The clamped SwiGLU of gptoss.py:120-122 on bf16 values (float32 array), every
    tensor op rounded to bf16: gate = min(gu[::2], limit), up = clamp(gu[1::2]),
    act = bf16(bf16(up + 1) * bf16(gate * bf16(sigmoid(bf16(gate * alpha)))))."""
    gu = np.asarray(gu, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        gate = np.minimum(gu[..., 0::2], np.float32(limit))
        up = np.clip(gu[..., 1::2], np.float32(-limit), np.float32(limit))
        ga = _bf16r(gate * np.float32(alpha))
        sg = _bf16r(np.float32(1) / (np.float32(1) + np.exp(-ga)))
        glu = _bf16r(gate * sg)
        return _bf16r(_bf16r(up + np.float32(1)) * glu)


def gptoss_block_ref(pool: np.ndarray, expert_slot: dict, x_bf16: np.ndarray, ti: np.ndarray, sc: np.ndarray,
                     gub_bf16: np.ndarray, db_bf16: np.ndarray, H: int, I: int, bits: int, group: int = 128,
                     alpha: float = 1.702, limit: float = 7.0) -> np.ndarray:
    """PagedGptOssBlock.forward (gptoss.py:108-143) after routing: x_bf16 uint16 [N, H],
    ti [N, k] expert ids, sc [N, k] routing weights (bf16 values), biases as bf16 bits.
    Weights dequantized bit-exactly to bf16 (quant.py:76-87); GEMVs in binary64, each
    bf16 tensor of the reference rounded at the same point. N == 1 follows the decode
    path (weighted outputs summed over the k experts in float32, one rounding); N > 1
    follows the prefill path (index_add_ into bf16 in ascending expert order, a rounding
    per add). Returns bf16 bits [N, H]."""
    x = bf16_bits_to_f32(np.asarray(x_bf16, np.uint16)).reshape(-1, H).astype(np.float64)
    ti = np.asarray(ti).reshape(x.shape[0], -1)
    sc = np.asarray(sc, np.float32).reshape(ti.shape)
    gub = bf16_bits_to_f32(np.asarray(gub_bf16, np.uint16)).reshape(-1, 2 * I)
    db = bf16_bits_to_f32(np.asarray(db_bf16, np.uint16)).reshape(-1, H)
    N, n = x.shape[0], H * I

    def expert_out(e, rows):
        W = bf16_bits_to_f32(dequant(pool[expert_slot[e]][None], n, bits, group)[0]).astype(np.float64)
        gu = _bf16r(_bf16r((rows @ W[:2].reshape(H, 2 * I)).astype(np.float32)) + gub[e])
        act = gptoss_act(gu, alpha, limit).astype(np.float64)
        return _bf16r(_bf16r((act @ W[2].reshape(I, H)).astype(np.float32)) + db[e])

    if N == 1:
        y = np.zeros(H, np.float32)
        for j in range(ti.shape[1]):
            o = expert_out(int(ti[0, j]), x)[0]
            y = (y + _bf16r(o * sc[0, j])).astype(np.float32)
        return f32_to_bf16_bits(y).reshape(1, H)
    y = np.zeros((N, H), np.float32)
    for e in sorted(int(v) for v in np.unique(ti)):
        tok, pos = np.nonzero(ti == e)
        w = _bf16r(expert_out(e, x[tok]) * sc[tok, pos][:, None])
        for r, t in enumerate(tok):  # index_add_ in token order within the expert
            y[t] = _bf16r(y[t] + w[r])
    return f32_to_bf16_bits(y).reshape(N, H)
