"""GPU parity of the HIP path against the CPU oracle (oracle/), through the C ABI.

Bars (set by the task): dequant, quantize and packing bit-exact; layer outputs within
1e-3 relative L2 of the binary64 oracle of the fused semantics rounded to bf16 (the
kernels accumulate in fp32 and store bf16 once). The reference's own looser criterion
(tests/test_kernels.py:33: max|d|/max|ref| < 2e-2 against dequant->bf16->matmul) is
checked too.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from wisp import kernels, quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-3  # rel-L2 vs the oracle


def _weights(rng, n, scale=0.02):
    return (rng.standard_normal(3 * n) * scale).astype(np.float32)


def _pool(E, H, I, bits, group, seed, pad=0):
    rng = np.random.default_rng(seed)
    n = H * I
    rows = [O.quantize(_weights(rng, n), bits, group) for _ in range(E)]
    nb = rows[0].size
    pool = np.zeros((E, nb + pad), np.uint8)
    for e, r in enumerate(rows):
        pool[e, :nb] = r
    return pool


def _x(rng, H):
    return O.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32))


def _bf16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _rel_l2(got, ref):
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def _route(rng, E, k):
    sel, rw = O.route(rng.standard_normal((1, E)).astype(np.float32), k)
    return sel[0], rw[0]


# ---------------------------------------------------------------- format kernels
@pytest.mark.parametrize(
    "bits,n,group,pad",
    [(4, 256 * 128, 128, 0), (3, 256 * 128, 128, 16), (2, 256 * 128, 128, 0), (8, 256 * 128, 128, 0),
     (4, 2048 * 768, 128, 0), (3, 2048 * 768, 128, 0), (2, 2048 * 768, 128, 0),
     (4, 64 * 32, 32, 0), (3, 64 * 32, 32, 4), (2, 64 * 32, 32, 0), (8, 64 * 32, 32, 0),
     (4, 3072, 96, 0), (3, 3072, 96, 0), (2, 3072, 96, 2)],
)
def test_dequant_bit_exact(bits, n, group, pad):
    rng = np.random.default_rng(bits * 7 + group)
    rows = np.stack([O.quantize(_weights(rng, n, 0.05), bits, group) for _ in range(2)])
    if pad:
        rows = np.concatenate([rows, np.full((2, pad), 0xAB, np.uint8)], 1)
    ref = O.dequant(rows, n, bits, group)
    got = quant.dequant(torch.from_numpy(rows).to(DEV), n, bits, group)
    assert got.shape == (2, 3, n) and got.dtype == torch.bfloat16
    assert np.array_equal(_bf16(got), ref)


def test_dequant_rows_gather_and_bounds():
    H, I, bits, group = 256, 128, 4, 128
    n = H * I
    pool = _pool(5, H, I, bits, group, seed=3, pad=32)
    idx = torch.tensor([4, 0, 2, 7, -1], device=DEV)  # last two out of range
    got = _bf16(quant.dequant_rows(torch.from_numpy(pool).to(DEV), idx, n, bits, group))
    ref = O.dequant(pool[[4, 0, 2]], n, bits, group)
    assert np.array_equal(got[:3], ref)
    assert np.all((got[3:] & 0x7F80) == 0x7F80) and np.all(got[3:] & 0x7F)  # NaN rows, nothing read


@pytest.mark.parametrize("bits", [8, 4, 3, 2])
@pytest.mark.parametrize("group,n", [(128, 256 * 128), (32, 64 * 32), (128, 2048 * 768)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_quantize_bit_exact(bits, group, n, dtype):
    rng = np.random.default_rng(bits + group)
    w = _weights(rng, n, 0.05)
    w[:group] = 0.3  # a constant group: scale clamps to 1e-5 (an fp16 subnormal)
    w[group : 2 * group] = np.arange(group) % 16  # integer levels with exact ties
    if dtype == "bf16":
        w = O.bf16_bits_to_f32(O.f32_to_bf16_bits(w))
        t = torch.from_numpy(w).to(torch.bfloat16)
    else:
        t = torch.from_numpy(w)
    got = quant.quantize(t.reshape(3, n).to(DEV), bits, group).cpu().numpy()
    assert np.array_equal(got, O.quantize(w, bits, group))


@pytest.mark.parametrize("bits", [8, 4, 3, 2])
def test_pack_unpack(bits):
    q = np.random.default_rng(bits).integers(0, 2**bits, 3 * 4096).astype(np.uint8)
    packed = quant._pack(torch.from_numpy(q).to(DEV), bits)
    assert np.array_equal(packed.cpu().numpy(), O.pack(q, bits))
    back = quant._unpack(packed.reshape(1, -1), bits)
    assert np.array_equal(back.cpu().numpy()[0], q)


# ---------------------------------------------------------------- fused layer
LAYER_SHAPES = [
    # (H, I, group, E, k): reference test shapes, the BASELINE layer, the tiny-model shape,
    # and shapes that take the generic (H/32 > 64 or I/32 > 64) kernels
    (256, 128, 128, 6, 3),
    (2048, 768, 128, 10, 8),
    (64, 32, 32, 8, 2),
    (4096, 256, 128, 3, 2),
    (256, 4096, 128, 3, 2),
    (512, 384, 128, 4, 4),
]


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("H,I,group,E,k", LAYER_SHAPES)
def test_moe_decode_fast_parity(bits, H, I, group, E, k):
    rng = np.random.default_rng(1000 * bits + H + I)
    n = H * I
    pool = _pool(E, H, I, bits, group, seed=H + bits)
    sel, rw = _route(rng, E, k)
    x = _x(rng, H)
    _, _, ref = O.moe_layer_f64(pool, sel, rw, x, H, I, bits, group)
    fn = {4: kernels.moe_decode_q4_fast, 3: kernels.moe_decode_q3_fast, 2: kernels.moe_decode_q2_fast}[bits]
    meta = torch.from_numpy(O.meta(sel, rw)).to(DEV)
    got = fn(torch.from_numpy(pool).to(DEV), meta, torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV),
             k, n, H, I, group)
    torch.cuda.synchronize()
    g = O.bf16_bits_to_f32(_bf16(got)).astype(np.float64)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).astype(np.float64)
    err = _rel_l2(g, r)
    print(f"bits={bits} H={H} I={I} G={group} k={k}: rel-L2 {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("H,I,group", [(2048, 768, 128), (256, 128, 128), (4096, 256, 128), (64, 32, 32)])
def test_gate_up_activation(bits, H, I, group):
    rng = np.random.default_rng(bits + H)
    n, E, k = H * I, 4, 3
    pool = _pool(E, H, I, bits, group, seed=bits * 3 + I)
    sel, rw = _route(rng, E, k)
    x = _x(rng, H)
    a_ref, _, _ = O.moe_layer_f64(pool, sel, rw, x, H, I, bits, group)
    meta = torch.from_numpy(O.meta(sel, rw)).to(DEV)
    a = kernels.gate_up_act(torch.from_numpy(pool).to(DEV), meta,
                            torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV), k, n, H, I, bits, group)
    err = _rel_l2(a.cpu().numpy().astype(np.float64), a_ref)
    print(f"gate_up bits={bits} H={H}: rel-L2 {err:.3e}")
    # the activation is fp32 between the kernels (the reference's `a`, kernels.py:133): the only error is the
    # fp32 accumulation of the gate/up dot products and SiLU
    assert err <= 2e-7, err


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("xdt", [np.float32, np.float16])
@pytest.mark.parametrize("H,I,group", [(2048, 768, 128), (256, 128, 128)])
def test_gate_up_activation_float_x(bits, xdt, H, I, group):
    """A float32 (or float16) x, not representable in bf16, against the binary64 layer on the same
    values: the reference widens any float x exactly (kernels.py:50-51), and so does kernel 1 (every
    code x x product exact in fp32); what is left is the fp32 accumulation, as in the reference. A
    product of a code with a bf16 or fp16 x has at most 12 / 15 significant bits, so fp32 sums of
    them round rarely (<= 2e-7 measured); with a float32 x every product has 24+ bits and every
    addition rounds (3-6e-7 measured), hence 1e-6 for float32, 1000x below the layer's 1e-3 bar."""
    rng = np.random.default_rng(bits * 7 + H)
    n, E, k = H * I, 4, 3
    pool = _pool(E, H, I, bits, group, seed=bits * 5 + I)
    sel, rw = _route(rng, E, k)
    x = (rng.standard_normal(H) * (1.0 + 1e-3 * rng.standard_normal(H))).astype(xdt)
    a_ref, _, _ = O.moe_layer_f64(pool, sel, rw, x, H, I, bits, group)
    meta = torch.from_numpy(O.meta(sel, rw)).to(DEV)
    a = kernels.gate_up_act(torch.from_numpy(pool).to(DEV), meta, torch.from_numpy(x).to(DEV), k, n, H, I, bits,
                            group)
    err = _rel_l2(a.cpu().numpy().astype(np.float64), a_ref)
    print(f"gate_up float x {np.dtype(xdt).name} bits={bits} H={H}: rel-L2 {err:.3e}")
    assert err <= (1e-6 if xdt == np.float32 else 2e-7), err


@pytest.mark.parametrize("H,I,group,E,k", [(256, 128, 128, 6, 3), (2048, 768, 128, 10, 8)])
def test_moe_decode_q4_per_expert_path(H, I, group, E, k):
    """kernels.py:115-137: slots int64 + weight tensor, per-expert y then torch weighted sum."""
    rng = np.random.default_rng(H)
    n = H * I
    pool = _pool(E, H, I, 4, group, seed=E)
    sel, rw = _route(rng, E, k)
    x = _x(rng, H)
    _, y_ref, ref = O.moe_layer_f64(pool, sel, rw, x, H, I, 4, group)
    got = kernels.moe_decode_q4(torch.from_numpy(pool).to(DEV), torch.from_numpy(sel).to(DEV),
                                torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV),
                                torch.from_numpy(rw).to(torch.bfloat16).to(DEV), n, H, I, group)
    g = O.bf16_bits_to_f32(_bf16(got)).astype(np.float64)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).astype(np.float64)
    err = _rel_l2(g, r)
    print(f"moe_decode_q4 H={H}: rel-L2 {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("bits", [4, 3])
def test_reference_test_criterion(bits):
    """The reference's own check (tests/test_kernels.py:10-33): ref = dequant -> bf16 ->
    fp32 matmul, SiLU, weighted sum; max|d| / max|ref| < 2e-2. Seeds/shapes as there."""
    rng = np.random.default_rng(bits)
    H, I, E, k, group = 256, 128, 6, 3, 128
    n = H * I
    w3 = (rng.standard_normal((E, 3 * n)) * 0.05).astype(np.float32)
    w3 = O.bf16_bits_to_f32(O.f32_to_bf16_bits(w3)).reshape(E, 3 * n)
    pool = np.stack([O.quantize(w3[e], bits, group) for e in range(E)])
    slots = np.array([4, 1, 2])
    x = _x(rng, H)
    w = torch.softmax(torch.from_numpy(rng.standard_normal(k).astype(np.float32)), 0).numpy()
    W = O.bf16_bits_to_f32(O.dequant(pool[slots], n, bits, group)).astype(np.float32).reshape(k, 3, n)
    xf = O.bf16_bits_to_f32(x)
    g = W[:, 0].reshape(k, I, H) @ xf
    u = W[:, 1].reshape(k, I, H) @ xf
    a = g / (1 + np.exp(-g)) * u
    y = np.einsum("khi,ki->kh", W[:, 2].reshape(k, H, I), a)
    exp = (y * w[:, None]).sum(0)
    meta = torch.from_numpy(O.meta(slots, w)).to(DEV)
    fn = kernels.moe_decode_q4_fast if bits == 4 else kernels.moe_decode_q3_fast
    got = fn(torch.from_numpy(pool).to(DEV), meta, torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV),
             k, n, H, I)
    d = O.bf16_bits_to_f32(_bf16(got))
    assert np.abs(d - exp).max() / np.abs(exp).max() < 2e-2


def test_invalid_slot_gives_nan_not_a_fault():
    H, I, group, E, k = 256, 128, 128, 3, 2
    pool = torch.from_numpy(_pool(E, H, I, 4, group, seed=1)).to(DEV)
    x = torch.randn(H, device=DEV).to(torch.bfloat16)
    for bad in (3.0, -1.0, 1.5, float("nan")):
        meta = torch.tensor([0.0, bad, 0.5, 0.5], device=DEV)
        out = kernels.moe_decode_q4_fast(pool, meta, x, k, H * I, H, I, group)
        assert torch.isnan(out.float()).all()
    ok = kernels.moe_decode_q4_fast(pool, torch.tensor([0.0, 2.0, 0.5, 0.5], device=DEV), x, k, H * I, H, I, group)
    assert torch.isfinite(ok.float()).all()


@pytest.mark.parametrize("gu", [(4, 4), (2, 4), (8, 4), (1, 4), (4, 2), (2, 8), (4, 1), (8, 1)])
@pytest.mark.parametrize("dn", [1, 2, 4, 8])
def test_tuning_variants_agree(gu, dn):
    H, I, group, E, k, bits = 2048, 768, 128, 9, 8, 4
    rng = np.random.default_rng(42)
    pool = _pool(E, H, I, bits, group, seed=42)
    sel, rw = _route(rng, E, k)
    x = _x(rng, H)
    _, _, ref = O.moe_layer_f64(pool, sel, rw, x, H, I, bits, group)
    try:
        kernels.set_tuning(gu[0], gu[1], dn)
        got = kernels.moe_decode_fast(torch.from_numpy(pool).to(DEV),
                                      torch.from_numpy(O.meta(sel, rw)).to(DEV),
                                      torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV),
                                      k, H * I, H, I, bits)
        torch.cuda.synchronize()
    finally:
        kernels.set_tuning(2, 4, 4)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))
    assert _rel_l2(O.bf16_bits_to_f32(_bf16(got)), r) <= TOL


def test_graph_capture_with_meta_updates():
    """graphdec.py capture contract: kernel arguments frozen, slots/weights read from the
    device meta buffer at replay time (updated by an H2D copy between replays)."""
    H, I, group, E, k, bits = 2048, 768, 128, 12, 8, 4
    n = H * I
    rng = np.random.default_rng(9)
    pool_np = _pool(E, H, I, bits, group, seed=9)
    pool = torch.from_numpy(pool_np).to(DEV)
    x_np = _x(rng, H)
    x = torch.from_numpy(x_np.view(np.int16)).view(torch.bfloat16).to(DEV)
    meta_dev = torch.zeros(2 * k, device=DEV)
    meta_host = torch.zeros(2 * k).pin_memory()
    meta_dev.copy_(torch.from_numpy(O.meta(np.arange(k), np.full(k, 1.0 / k, np.float32))))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kernels.moe_decode_q4_fast(pool, meta_dev, x, k, n, H, I)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = kernels.moe_decode_q4_fast(pool, meta_dev, x, k, n, H, I)
    for it in range(4):
        sel, rw = _route(rng, E, k)
        meta_host.copy_(torch.from_numpy(O.meta(sel, rw)))
        meta_dev.copy_(meta_host, non_blocking=True)
        g.replay()
        eager = kernels.moe_decode_q4_fast(pool, meta_dev, x, k, n, H, I)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), it
        _, _, ref = O.moe_layer_f64(pool_np, sel, rw, x_np, H, I, bits, group)
        r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))
        assert _rel_l2(O.bf16_bits_to_f32(_bf16(out)), r) <= TOL


# ---------------------------------------------------------------- repeated calls, real shape
@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("k", [8, 5, 1])
def test_layer_parity_repeated_calls(bits, k):
    """moe_decode_fast at the Qwen3-30B-A3B expert shape, called repeatedly with new routes
    and inputs on one pool (nothing carried over between calls)."""
    H, I, group, E = 2048, 768, 128, 12
    n = H * I
    rng = np.random.default_rng(77 + bits + k)
    pool_np = _pool(E, H, I, bits, group, seed=bits * 11 + k)
    pool = torch.from_numpy(pool_np).to(DEV)
    for it in range(3):
        sel, rw = _route(rng, E, k)
        x = _x(rng, H)
        _, _, ref = O.moe_layer_f64(pool_np, sel, rw, x, H, I, bits, group)
        got = kernels.moe_decode_fast(pool, torch.from_numpy(O.meta(sel, rw)).to(DEV),
                                      torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV),
                                      k, n, H, I, bits, group)
        torch.cuda.synchronize()
        r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))
        err = _rel_l2(O.bf16_bits_to_f32(_bf16(got)), r)
        print(f"layer bits={bits} k={k} it={it}: rel-L2 {err:.3e}")
        assert err <= TOL, err


# ---------------------------------------------------------------- rotary (kernels.py:325-371)
def _rope_inputs(seed, Hq, Hk, D, dtype):
    g = torch.Generator().manual_seed(seed)
    # HF layout: [1,1,H,D] transposed to a [1,H,1,D] strided view
    q = torch.randn(1, 1, Hq, D, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(1, 1, Hk, D, generator=g).to(dtype).transpose(1, 2)
    pos = 1 + int(torch.randint(0, 4000, (1,), generator=g))
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.cat([inv, inv]) * pos
    cos = ang.cos().to(dtype).view(1, 1, D)
    sin = ang.sin().to(dtype).view(1, 1, D)
    return q, k, cos, sin


def _f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Hq,Hk,D", [(32, 4, 128), (16, 2, 64), (8, 8, 256), (4, 0, 128), (3, 1, 2)])
def test_rope_decode_bit_exact(dtype, Hq, Hk, D):
    q, k, cos, sin = _rope_inputs(Hq * 7 + D, Hq, Hk, D, dtype)
    qo, ko = kernels.rope_decode(q.to(DEV), k.to(DEV), cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert qo.shape == (1, Hq, 1, D) and ko.shape == (1, Hk, 1, D) and qo.dtype == dtype
    c, s = _f32(cos).ravel(), _f32(sin).ravel()
    for got, x, H in ((qo, q, Hq), (ko, k, Hk)):
        if H == 0:
            continue
        ref = O.rope(_f32(x).reshape(H, D), c, s)
        if dtype == torch.bfloat16:
            assert np.array_equal(got.view(torch.int16).cpu().numpy().reshape(H, D).view(np.uint16),
                                  O.f32_to_bf16_bits(ref).reshape(H, D))
        else:
            assert np.array_equal(_f32(got).reshape(H, D).view(np.uint32), ref.view(np.uint32))


def test_rope_decode_reference_criterion():
    """tests/test_fastattn.py:12-23 of the reference: against the library's rotate-half formula
    in bf16 (HF's apply_rotary_pos_emb), max|d| < 3e-2 max|ref|."""
    D, Hq, Hk = 128, 32, 4
    q, k, cos, sin = _rope_inputs(0, Hq, Hk, D, torch.bfloat16)
    try:
        from transformers.models.qwen3_moe import modeling_qwen3_moe as m
        qr, kr = m.apply_rotary_pos_emb(q, k, cos, sin)
    except Exception:  # library missing: the same formula, written out
        def rot(t):
            return torch.cat([-t[..., D // 2:], t[..., : D // 2]], dim=-1)
        qr, kr = q * cos + rot(q) * sin, k * cos + rot(k) * sin
    qo, ko = kernels.rope_decode(q.to(DEV), k.to(DEV), cos.to(DEV), sin.to(DEV))
    for got, ref in ((qo.cpu(), qr), (ko.cpu(), kr)):
        assert got.shape == ref.shape
        assert (got.float() - ref.float()).abs().max() < 3e-2 * ref.float().abs().max()


# ---------------------------------------------------------------- decode attention (graphdec.py:171-174)
def _bf16_np(a):
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.asarray(a, np.float32))).reshape(np.shape(a))


def _attn_case(Hq, Hk, D, T, seed):
    rng = np.random.default_rng(seed)
    q = _bf16_np(rng.standard_normal((Hq, D)))
    k = _bf16_np(rng.standard_normal((Hk, T, D)))
    v = _bf16_np(rng.standard_normal((Hk, T, D)))
    tb = lambda a: torch.from_numpy(a).to(torch.bfloat16).to(DEV)  # noqa: E731 (exact: values are bf16)
    return q, k, v, tb(q).view(1, Hq, 1, D), tb(k)[None].contiguous(), tb(v)[None].contiguous()


@pytest.mark.parametrize("Hq,Hk,D,T", [(32, 4, 128, 256), (8, 8, 64, 130), (4, 1, 256, 70), (32, 2, 128, 64),
                                       (16, 4, 128, 4096), (8, 2, 128, 6000), (32, 4, 128, 4096)])
def test_attn_decode_matches_oracle(Hq, Hk, D, T):
    """(32, 4, 128, 4096) is the C4 decoder's shape (8 query heads per KV head, 64 chunks of 64 positions,
    several merge batches); positions cover the first chunk, a chunk boundary, the middle of a chunk in the
    middle of the cache and the last position."""
    q, k, v, tq, tk, tv = _attn_case(Hq, Hk, D, T, seed=Hq + D + T)
    scale = D ** -0.5
    for pos in sorted({0, 1, 63, 64, min(100, T - 1), T // 2 + 33, T - 1}):
        if pos >= T:
            continue
        p = torch.tensor([pos], dtype=torch.int64, device=DEV)
        out = kernels.attn_decode(tq, tk, tv, p, scale)
        torch.cuda.synchronize()
        ref = O.attn_decode(q, k, v, pos, scale)
        r = _bf16_np(ref)
        got = out.float().cpu().numpy().reshape(Hq, D)
        err = np.linalg.norm(got - r) / np.linalg.norm(r)
        assert err <= 1e-3, (pos, err)
        assert np.max(np.abs(got - ref)) <= 1e-2 * np.max(np.abs(ref)), pos


def test_attn_decode_graph_follows_device_position():
    Hq, Hk, D, T = 32, 4, 128, 512
    q, k, v, tq, tk, tv = _attn_case(Hq, Hk, D, T, seed=3)
    p = torch.zeros(1, dtype=torch.int64, device=DEV)
    kernels.attn_decode(tq, tk, tv, p, 0.125)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = kernels.attn_decode(tq, tk, tv, p, 0.125)
    for pos in (5, 300, 64, 511):
        p.fill_(pos)
        g.replay()
        eager = kernels.attn_decode(tq, tk, tv, p, 0.125)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), pos
        r = _bf16_np(O.attn_decode(q, k, v, pos, 0.125))
        got = out.float().cpu().numpy().reshape(Hq, D)
        assert np.linalg.norm(got - r) / np.linalg.norm(r) <= 1e-3, pos


# ---------------------------------------------------------------- grouped prefill (moe.py:131-151)
def _prefill_case(E, H, I, T, k, bits, seed, hot=False):
    rng = np.random.default_rng(seed)
    pool = _pool(E, H, I, bits, 128, seed=seed)
    x = O.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)).reshape(T, H)
    sel, rw = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    if hot:  # every token routes to expert 0 (a group larger than one workgroup pass)
        for t in range(T):
            if 0 not in sel[t]:
                sel[t, -1] = 0
    return pool, x, sel, rw


def _run_prefill(pool_np, x, sel, rw, H, I, bits, slots=None, acc=None):
    pool = torch.from_numpy(pool_np).to(DEV)
    E = pool_np.shape[0]
    slots = {e: e for e in range(E)} if slots is None else slots
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV)
    out = kernels.moe_prefill(pool, slots, xt, torch.from_numpy(sel), torch.from_numpy(rw).to(DEV), H * I, H, I,
                              bits, acc=acc)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("E,H,I,T,k,hot", [(6, 256, 128, 1, 2, False), (6, 256, 128, 17, 2, False),
                                          (4, 256, 128, 300, 2, True), (16, 2048, 768, 64, 8, False),
                                          (12, 512, 384, 40, 4, False),
                                          # K > 2048: scale/min read from global memory, not the LDS table
                                          (4, 4096, 256, 20, 2, False), (4, 256, 4096, 20, 2, False)])
def test_moe_prefill_matches_oracle(bits, E, H, I, T, k, hot):
    pool, x, sel, rw = _prefill_case(E, H, I, T, k, bits, seed=E + T + bits, hot=hot)
    out = _run_prefill(pool, x, sel, rw, H, I, bits)
    ref = O.moe_prefill_f64(pool, {e: e for e in range(E)}, x, sel, rw, H, I, bits)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).reshape(ref.shape)
    got = out.float().cpu().numpy()
    err = np.linalg.norm(got - r) / np.linalg.norm(r)
    print(f"prefill bits={bits} T={T} H={H}: rel-L2 {err:.3e}")
    assert err <= 1e-3, err
    assert np.max(np.abs(got - ref)) <= 2e-2 * np.max(np.abs(ref))


# 4-bit with an even number (<= 16) of quant groups in both GEMMs takes the LDS-DMA form
# (hand-counted waits): tiles of 1, 2, 4 and 8 K steps, single and several passes per group.
@pytest.mark.parametrize("E,H,I,T,k,hot", [(5, 256, 256, 3, 2, False), (5, 512, 256, 33, 2, False),
                                          (6, 1024, 512, 70, 3, False), (4, 512, 256, 150, 2, True),
                                          (8, 2048, 1536, 24, 4, False), (3, 1024, 256, 1, 3, False),
                                          # the C2 expert shape with a 130-pair group: a 128-token pass
                                          (6, 2048, 768, 130, 3, True)])
def test_moe_prefill_lds_dma_shapes(E, H, I, T, k, hot):
    pool, x, sel, rw = _prefill_case(E, H, I, T, k, 4, seed=E * 7 + T, hot=hot)
    out = _run_prefill(pool, x, sel, rw, H, I, 4)
    ref = O.moe_prefill_f64(pool, {e: e for e in range(E)}, x, sel, rw, H, I, 4)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).reshape(ref.shape)
    got = out.float().cpu().numpy()
    err = np.linalg.norm(got - r) / np.linalg.norm(r)
    print(f"prefill lds-dma H={H} I={I} T={T}: rel-L2 {err:.3e}")
    assert err <= 1e-3, err


# chunks of 80, 96 and 128 pairs make passes of 5-8 token tiles (the token tile staged half
# a quant group at a time); whole experts (1 << 20) several such passes per group
@pytest.mark.parametrize("chunk", [1 << 20, 16, 48, 80, 96, 128])
def test_moe_prefill_lds_dma_any_partition_and_invalid_slot(chunk, monkeypatch):
    E, H, I, T, k = 4, 512, 256, 200, 2
    pool, x, sel, rw = _prefill_case(E, H, I, T, k, 4, seed=91, hot=True)
    base = _run_prefill(pool, x, sel, rw, H, I, 4).float()
    orig = kernels._prefill_chunks
    monkeypatch.setattr(kernels, "_prefill_chunks", lambda u, f, c, chunk_=None: orig(u, f, c, chunk))
    got = _run_prefill(pool, x, sel, rw, H, I, 4).float()
    assert torch.equal(got, base)
    bad = _run_prefill(pool, x, sel, rw, H, I, 4, slots={**{e: e for e in range(E)}, 1: 77}).float().cpu()
    hit = torch.from_numpy((sel == 1).any(axis=1))
    assert torch.isnan(bad[hit]).all() and torch.isfinite(bad[~hit]).all()


def test_moe_prefill_expert_chunks_accumulate_and_invalid_slot():
    E, H, I, T, k, bits = 6, 256, 128, 24, 2, 4
    pool, x, sel, rw = _prefill_case(E, H, I, T, k, bits, seed=31)
    acc = torch.zeros((T, H), dtype=torch.float32, device=DEV)
    for chunk in ([0, 1, 2], [3, 4, 5]):
        _run_prefill(pool, x, sel, rw, H, I, bits, slots={e: e for e in chunk}, acc=acc)
    one = _run_prefill(pool, x, sel, rw, H, I, bits).float()
    assert torch.allclose(acc.to(torch.bfloat16).float(), one, rtol=1e-2, atol=1e-3)
    ref = O.moe_prefill_f64(pool, {e: e for e in range(E)}, x, sel, rw, H, I, bits)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).reshape(ref.shape)
    got = acc.to(torch.bfloat16).float().cpu().numpy()
    assert np.linalg.norm(got - r) / np.linalg.norm(r) <= 1e-3
    # an invalid slot id poisons exactly the tokens routed to that expert
    bad = _run_prefill(pool, x, sel, rw, H, I, bits, slots={**{e: e for e in range(E)}, 2: 99}).float().cpu()
    hit = torch.from_numpy((sel == 2).any(axis=1))
    assert torch.isnan(bad[hit]).all() and torch.isfinite(bad[~hit]).all()


@pytest.mark.parametrize("bits", [4, 3])
@pytest.mark.parametrize("chunk", [1 << 20, 16])
def test_moe_prefill_any_group_partition(bits, chunk, monkeypatch):
    # the launch accepts any partition of the pairs into groups: whole experts
    # (a 300-pair group takes several passes of the grid's z workgroups) or
    # 16-pair items give the same result as the default work items
    E, H, I, T, k = 4, 256, 128, 300, 2
    pool, x, sel, rw = _prefill_case(E, H, I, T, k, bits, seed=77 + bits, hot=True)
    base = _run_prefill(pool, x, sel, rw, H, I, bits).float()
    orig = kernels._prefill_chunks
    monkeypatch.setattr(kernels, "_prefill_chunks", lambda u, f, c, chunk_=None: orig(u, f, c, chunk))
    got = _run_prefill(pool, x, sel, rw, H, I, bits).float()
    print(f"prefill partition chunk={chunk} bits={bits}: max |diff| {float((got - base).abs().max()):.3e}")
    assert torch.equal(got, base)


def test_empty_inputs_are_no_ops():
    """Empty work (the reference's loops over zero tokens or zero experts) returns empty or
    zero results without a launch: T = 0 tokens, tokens whose experts are all absent from
    the slot map (output zeros; with acc, acc unchanged), and zero dequant rows."""
    E, H, I, bits = 4, 256, 128, 4
    pool, x, sel, rw = _prefill_case(E, H, I, 5, 2, bits, seed=77)
    pt = torch.from_numpy(pool).to(DEV)
    x0 = torch.empty((0, H), dtype=torch.bfloat16, device=DEV)
    out = kernels.moe_prefill(pt, {e: e for e in range(E)}, x0, torch.empty((0, 2), dtype=torch.int64),
                              torch.empty((0, 2), dtype=torch.float32, device=DEV), H * I, H, I, bits)
    assert out.shape == (0, H)
    none = _run_prefill(pool, x, sel, rw, H, I, bits, slots={})
    assert none.shape == (5, H) and not none.float().abs().any()
    acc = torch.full((5, H), 0.5, dtype=torch.float32, device=DEV)
    _run_prefill(pool, x, sel, rw, H, I, bits, slots={}, acc=acc)
    assert torch.equal(acc, torch.full_like(acc, 0.5))
    rows = quant.dequant(pt[:0], H * I, bits)
    torch.cuda.synchronize()
    assert rows.shape == (0, 3, H * I)
