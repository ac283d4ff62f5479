"""Pins for the CPU oracle (oracle/wisp_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle fails it: known-answer
tests derived by hand from the reference's stated layout, the reference's own KATs and
bounds (tests/test_quant.py of imronpuji/wisp-runtime), a second independent statement
of the 3-bit layout (the kernels' `_q3`, kernels.py:209-217), conversions compared with
torch's own (library routines), and the fused layer compared with a dense numpy matvec.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O


# ---------------------------------------------------------------- sizes (quant.py:17-22)
def test_expert_nbytes_kats():
    # test_quant.py:37-40
    n = 1572864
    assert O.expert_nbytes(n, 16, 128) == 9437184
    assert abs(O.expert_nbytes(n, 4, 128) / O.expert_nbytes(n, 16, 128) - 0.265) < 0.01
    # docs/architecture.md:82: 4/3/2-bit experts are 2.39/1.83/1.27 MiB
    for bits, mib in ((4, 2.39), (3, 1.83), (2, 1.27)):
        assert round(O.expert_nbytes(n, bits, 128) / 2**20, 2) == mib
    # exact byte counts: codes + 2 fp16 per group
    assert O.expert_nbytes(n, 4, 128) == 2359296 + 73728 + 73728
    assert O.expert_nbytes(n, 3, 128) == 1769472 + 2 * 36864 * 2
    assert O.expert_nbytes(n, 2, 128) == 1179648 + 2 * 36864 * 2
    with pytest.raises(ValueError):
        O.expert_nbytes(100, 4, 128)  # 3n not a multiple of the group
    with pytest.raises(ValueError):
        O.expert_nbytes(2048, 5, 32)


# ---------------------------------------------------------------- packing (quant.py:25-57)
def test_pack_known_answers():
    # 4-bit: element e is the low nibble of byte e/2 when e is even (architecture.md:79)
    assert O.pack(np.array([1, 2, 3, 4], np.uint8), 4).tolist() == [0x21, 0x43]
    # 2-bit: 4 codes per byte, LSB first
    assert O.pack(np.array([1, 2, 3, 0], np.uint8), 2).tolist() == [0x39]
    # 3-bit: 8 codes -> 24-bit little endian, code i at bit 3i (hand-computed: 0x1F58D1)
    assert O.pack(np.array([1, 2, 3, 4, 5, 6, 7, 0], np.uint8), 3).tolist() == [0xD1, 0x58, 0x1F]
    assert O.pack(np.array([7] * 8, np.uint8), 3).tolist() == [0xFF, 0xFF, 0xFF]
    assert O.pack(np.array([200, 3], np.uint8), 8).tolist() == [200, 3]


@pytest.mark.parametrize("bits", [8, 4, 3, 2])
def test_pack_roundtrip(bits):
    # test_quant.py:9-12
    q = np.random.default_rng(bits).integers(0, 2**bits, 4096).astype(np.uint8)
    assert np.array_equal(O.unpack(O.pack(q, bits), bits, q.size), q)


def test_q3_layout_matches_kernel_statement():
    # unpack (quant.py:53-56) against the kernels' own 3-bit read (kernels.py:209-217)
    rng = np.random.default_rng(3)
    q = rng.integers(0, 8, 3 * 4096).astype(np.uint8)
    buf = np.concatenate([O.pack(q, 3), np.zeros(8, np.uint8)])  # trailing bytes stand in for the scales
    got = np.array([O.q3_field(buf, e) for e in range(q.size)], dtype=np.uint8)
    assert np.array_equal(got, q)


# ---------------------------------------------------------------- scalar conversions
def _f16_cases():
    rng = np.random.default_rng(0)
    specials = np.array(
        [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 70000.0, 1e-5, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
         1e-10, np.inf, -np.inf, 0.1, 0.3, 1.00048828125, 1.000732421875],
        dtype=np.float32,
    )
    mags = 10.0 ** rng.uniform(-9, 5, 20000)
    rnd = (mags * rng.choice([-1, 1], mags.size)).astype(np.float32)
    # exact halfway points between fp16 neighbours (ties)
    h = rng.integers(0, 0x7BFF, 2000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    ties = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    return np.concatenate([specials, rnd, ties])


def test_f32_to_f16_matches_torch():
    v = _f16_cases()
    ref = torch.from_numpy(v).half().view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_f16_bits(v)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    v = v[~np.isnan(v)]
    ties = (rng.integers(0, 2**16, 5000).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    v = np.concatenate([v, ties[~np.isnan(ties)]])
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(v), ref)


# ---------------------------------------------------------------- quantize (quant.py:60-73)
def _split(buf, n, bits, group):
    N = 3 * n
    ncode = N * bits // 8
    ng = N // group
    codes = O.unpack(buf[:ncode], bits, N)
    s = buf[ncode : ncode + 2 * ng].view(np.uint16)
    m = buf[ncode + 2 * ng : ncode + 4 * ng].view(np.uint16)
    return codes, s, m


def test_quantize_known_answer_round_half_even():
    # one group of 32 with min 0 and max 15: scale (15-0)/15 = 1 exactly, min 0
    n, group = 32, 32  # 3n = 96 values = 3 groups
    g0 = np.array([0, 15, 2.5, 3.5, 7.5, 0.49, 14.5, 8.5] + [1.0] * 24, np.float32)
    w = np.concatenate([g0, g0 * 2, np.full(32, 0.3, np.float32)])
    buf = O.quantize(w, 4, group)
    codes, s, m = _split(buf, n, 4, group)
    # round half to even: 2.5->2, 3.5->4, 7.5->8, 14.5->14, 8.5->8
    assert codes[:8].tolist() == [0, 15, 2, 4, 8, 0, 14, 8]
    assert s[0] == 0x3C00 and m[0] == 0x0000  # 1.0, 0.0
    # group 1: scale 2 (0x4000), identical codes
    assert s[1] == 0x4000 and codes[32:40].tolist() == [0, 15, 2, 4, 8, 0, 14, 8]
    # constant group: scale clamps to 1e-5 -> fp16 subnormal 168 * 2^-24 (0x00A8);
    # min 0.3 -> fp16 0x34CD (0.300048828125) > 0.3, so every code is clamp(round(-4.9)) = 0
    assert s[2] == 0x00A8 and m[2] == 0x34CD
    assert codes[64:].tolist() == [0] * 32


@pytest.mark.parametrize("bits", [8, 4, 3, 2])
def test_quantize_codes_are_nearest_level(bits):
    # every code is round((v - m)/s) clamped: within 1/2 level of the exact quotient
    rng = np.random.default_rng(bits)
    n, group = 2048, 32
    w = (rng.standard_normal(3 * n) * 0.02).astype(np.float32)
    buf = O.quantize(w, bits, group)
    codes, s, m = _split(buf, n, bits, group)
    sf = np.repeat(s.view(np.float16).astype(np.float64), group)
    mf = np.repeat(m.view(np.float16).astype(np.float64), group)
    r = (w.astype(np.float64) - mf) / sf
    lv = 2**bits - 1
    inside = (r > 0.5) & (r < lv - 0.5)
    assert np.all(np.abs(codes[inside] - r[inside]) <= 0.5 + 1e-4)
    assert np.all(codes <= lv)


@pytest.mark.parametrize("bits", [16, 8, 4, 3, 2])
def test_sizes_and_error_bounds(bits):
    # test_quant.py:15-24
    rng = np.random.default_rng(bits)
    n, group = 2048, 32
    w = (rng.standard_normal(3 * n) * 0.02).astype(np.float32)
    buf = O.quantize(w, bits, group)
    assert buf.size == O.expert_nbytes(n, bits, group)
    r = O.bf16_bits_to_f32(O.dequant(buf, n, bits, group)[0]).reshape(-1)
    rel = np.linalg.norm(r - w) / np.linalg.norm(w)
    assert rel < {16: 0.01, 8: 0.01, 4: 0.12, 3: 0.25, 2: 0.6}[bits], rel


def test_error_monotonic():
    # test_quant.py:27-34
    rng = np.random.default_rng(7)
    n, group = 4096, 32
    w = rng.standard_normal(3 * n).astype(np.float32)
    errs = []
    for b in (8, 4, 3, 2):
        r = O.bf16_bits_to_f32(O.dequant(O.quantize(w, b, group), n, b, group)[0]).reshape(-1)
        errs.append(np.linalg.norm(r - w) / np.linalg.norm(w))
    assert errs == sorted(errs)


# ---------------------------------------------------------------- dequant (quant.py:76-87)
def _hand_buffer(code4, s16, m16, n=32, group=32):
    """4-bit expert with every code of group g equal to code4[g] and the given fp16 bits."""
    N = 3 * n
    q = np.repeat(np.array(code4, np.uint8), group)
    return np.concatenate(
        [O.pack(q, 4), np.array(s16, np.uint16).view(np.uint8), np.array(m16, np.uint16).view(np.uint8)]
    ), N


def test_dequant_known_answers():
    # group 0: 5*0.5 - 1 = 1.5 (bf16 0x3FC0); group 1: 15*2 + 0 = 30 (0x41F0);
    # group 2: 1*(1+2^-8) + 2^-24 -> fp32 tie rounds to 1+2^-8, whose bf16 tie rounds to
    # 1.0 (0x3F80). A single rounding of the exact sum would give 0x3F81: this pins the
    # binary32 add before the bf16 cast (quant.py:86-87).
    buf, N = _hand_buffer([5, 15, 1], [0x3800, 0x4000, 0x3C04], [0xBC00, 0x0000, 0x0001])
    out = O.dequant(buf, 32, 4, 32)[0].reshape(-1)
    assert set(out[:32].tolist()) == {0x3FC0}
    assert set(out[32:64].tolist()) == {0x41F0}
    assert set(out[64:].tolist()) == {0x3F80}


def test_dequant_matches_numpy_float32_semantics():
    # separately-rounded float32 mul and add, then RTNE bf16 (numpy float32 ops are IEEE)
    rng = np.random.default_rng(11)
    for bits in (8, 4, 3, 2):
        n, group = 1024, 128
        buf = O.quantize((rng.standard_normal(3 * n) * 0.05).astype(np.float32), bits, group)
        codes, s, m = _split(buf, n, bits, group)
        sf = np.repeat(s.view(np.float16).astype(np.float32), group)
        mf = np.repeat(m.view(np.float16).astype(np.float32), group)
        ref = O.f32_to_bf16_bits(codes.astype(np.float32) * sf + mf)
        assert np.array_equal(O.dequant(buf, n, bits, group)[0].reshape(-1), ref)


# ---------------------------------------------------------------- fused layer semantics
def _dense_layer(pool, slots, w, x_bits, H, I, bits, group):
    n = H * I
    if x_bits.dtype == np.uint16:
        xf = O.bf16_bits_to_f32(x_bits).astype(np.float64)
    else:
        xf = x_bits.astype(np.float64)
    out = np.zeros(H)
    a_all, y_all = [], []
    for s, wj in zip(slots, w):
        buf = pool[s]
        codes, sc, mn = _split(buf[: O.expert_nbytes(n, bits, group)], n, bits, group)
        W = codes.astype(np.float64) * np.repeat(sc.view(np.float16).astype(np.float64), group) + np.repeat(
            mn.view(np.float16).astype(np.float64), group
        )
        g = W[:n].reshape(I, H) @ xf
        u = W[n : 2 * n].reshape(I, H) @ xf
        a = g / (1 + np.exp(-g)) * u
        y = W[2 * n :].reshape(H, I) @ a
        a_all.append(a)
        y_all.append(y)
        out += float(wj) * y
    return np.array(a_all), np.array(y_all), out


@pytest.mark.parametrize("bits,H,I,group", [(4, 256, 128, 128), (3, 256, 128, 128), (2, 128, 64, 32)])
def test_fused_oracle_matches_dense_matvec(bits, H, I, group):
    rng = np.random.default_rng(bits)
    n, E, k = H * I, 5, 3
    pool = np.stack([O.quantize((rng.standard_normal(3 * n) * 0.05).astype(np.float32), bits, group) for _ in range(E)])
    slots = [4, 0, 2]
    w = np.array([0.5, 0.3, 0.2], np.float32)
    x = O.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32))
    a, y, out = O.moe_layer_f64(pool, slots, w, x, H, I, bits, group)
    a2, y2, out2 = _dense_layer(pool, slots, w, x, H, I, bits, group)
    assert np.allclose(a, a2, rtol=1e-10, atol=1e-12)
    assert np.allclose(y, y2, rtol=1e-10, atol=1e-12)
    assert np.allclose(out, out2, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("xdt", [np.float32, np.float16])
def test_fused_oracle_float_x(xdt):
    # x given as float values (the reference loads any float x and widens it, kernels.py:51-52):
    # the same dense unfolded form, and the bf16 entry point agrees on bf16-representable x
    rng = np.random.default_rng(31)
    H, I, group, bits, n = 256, 128, 128, 4, 256 * 128
    pool = np.stack([O.quantize((rng.standard_normal(3 * n) * 0.05).astype(np.float32), bits, group) for _ in range(4)])
    slots, w = [3, 1], np.array([0.75, 0.25], np.float32)
    x = rng.standard_normal(H).astype(xdt)
    a, y, out = O.moe_layer_f64(pool, slots, w, x, H, I, bits, group)
    a2, y2, out2 = _dense_layer(pool, slots, w, x, H, I, bits, group)
    assert np.allclose(out, out2, rtol=1e-10, atol=1e-12) and np.allclose(a, a2, rtol=1e-10, atol=1e-12)
    xb = O.f32_to_bf16_bits(x.astype(np.float32))
    _, _, out3 = O.moe_layer_f64(pool, slots, w, O.bf16_bits_to_f32(xb), H, I, bits, group)
    _, _, out4 = O.moe_layer_f64(pool, slots, w, xb, H, I, bits, group)
    assert np.array_equal(out3, out4)
    assert not np.allclose(out, out4, rtol=1e-6, atol=0)  # x's low bits reach the result


# ---------------------------------------------------------------- routing (moe.py:67-72)
def test_route_matches_torch():
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((16, 128)).astype(np.float32)
    sel, rw = O.route(logits, 8)
    t = torch.from_numpy(logits)
    p = torch.softmax(t, dim=1, dtype=torch.float32)
    tw, ts = torch.topk(p, 8, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True)).to(torch.bfloat16).float()
    assert np.array_equal(sel, ts.numpy())
    assert np.allclose(rw, tw.numpy(), rtol=0, atol=0)
    m = O.meta([3, 1], [0.25, 0.75])
    assert m.dtype == np.float32 and m.tolist() == [3.0, 1.0, 0.25, 0.75]


# ---------------------------------------------------------------- rotary (kernels.py:325-349)
def test_rope_known_answer_d2():
    # d = 2: a plain 2-D rotation, (x0 + i x1) * (c + i s); values chosen so every product
    # and sum is exact in binary32
    out = O.rope(np.array([[3.0, 5.0]], np.float32), np.array([0.5, 0.5], np.float32),
                 np.array([0.25, 0.25], np.float32))
    assert out.tolist() == [[3.0 * 0.5 - 5.0 * 0.25, 5.0 * 0.5 + 3.0 * 0.25]]


def test_rope_rotation_properties():
    rng = np.random.default_rng(3)
    d, nh = 128, 6
    x = rng.standard_normal((nh, d)).astype(np.float32)
    inv = 1.0 / (10000.0 ** (np.arange(0, d, 2) / d))
    ang = np.concatenate([inv, inv]) * 7.0  # position 7, HF layout (cos/sin repeated per half)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    out = O.rope(x, c, s)
    # the textbook rotate-half statement in float64: x*cos + rotate_half(x)*sin
    rh = np.concatenate([-x[:, d // 2:], x[:, : d // 2]], axis=1).astype(np.float64)
    ref = x.astype(np.float64) * c + rh * s
    assert np.max(np.abs(out - ref)) <= 4 * np.finfo(np.float32).eps * np.max(np.abs(ref))
    # a rotation keeps each head's norm
    assert np.allclose(np.linalg.norm(out, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)
    # rotating by a then by b equals rotating by a + b
    a2 = np.concatenate([inv, inv]) * 5.0
    two = O.rope(O.rope(x, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)),
                 np.cos(a2).astype(np.float32), np.sin(a2).astype(np.float32))
    one = O.rope(x, np.cos(ang + a2).astype(np.float32), np.sin(ang + a2).astype(np.float32))
    assert np.allclose(two, one, rtol=1e-4, atol=1e-5)
    # a plausible slip (sign on the wrong half) is caught by the textbook form
    bad = x.astype(np.float64) * c - rh * s
    assert np.max(np.abs(out - bad)) > 1e-2


# ---------------------------------------------------------------- decode attention (graphdec.py:171-174)
def test_attn_oracle_special_cases():
    rng = np.random.default_rng(8)
    Hq, Hk, T, D = 8, 2, 40, 16
    q = rng.standard_normal((Hq, D))
    k = rng.standard_normal((Hk, T, D))
    v = rng.standard_normal((Hk, T, D))
    # pos 0: the only position gets all the weight
    out = O.attn_decode(q, k, v, 0, 0.25)
    assert np.array_equal(out, v[np.arange(Hq) // 4, 0])
    # equal keys: uniform weights, the mean of the attended values
    ke = np.repeat(k[:, :1], T, axis=1)
    out = O.attn_decode(q, ke, v, 17, 0.25)
    assert np.allclose(out, v[np.arange(Hq) // 4, :18].mean(axis=1), rtol=1e-12, atol=1e-12)


def test_attn_oracle_matches_torch_sdpa_repeat_kv():
    """The library routine (scaled_dot_product_attention with the KV heads repeated, as
    tests/test_fastattn.py:26-35 of the reference states the grouping), masked to t <= pos."""
    rng = np.random.default_rng(9)
    Hq, Hk, T, D, pos, scale = 32, 4, 77, 128, 50, 128 ** -0.5
    q = rng.standard_normal((Hq, D)).astype(np.float32)
    k = rng.standard_normal((Hk, T, D)).astype(np.float32)
    v = rng.standard_normal((Hk, T, D)).astype(np.float32)
    out = O.attn_decode(q, k, v, pos, scale)
    tq = torch.from_numpy(q).view(1, Hq, 1, D).double()
    tk = torch.from_numpy(k).repeat_interleave(Hq // Hk, dim=0)[None].double()
    tv = torch.from_numpy(v).repeat_interleave(Hq // Hk, dim=0)[None].double()
    mask = (torch.arange(T) <= pos).view(1, 1, 1, T)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale)
    assert np.allclose(out, ref.view(Hq, D).numpy(), rtol=1e-10, atol=1e-10)
    # a head-mapping slip (h % Hk instead of h // G) would not match
    bad = np.stack([O.attn_decode(q[h : h + 1], k[h % Hk : h % Hk + 1], v[h % Hk : h % Hk + 1], pos, scale)[0]
                    for h in range(Hq)])
    assert not np.allclose(bad, out, atol=1e-3)


# ---------------------------------------------------------------- grouped prefill oracle (moe.py:131-151)
def _pf_case(E=5, H=256, I=128, T=7, k=2, bits=4, seed=0):
    rng = np.random.default_rng(seed)
    pool = np.stack([O.quantize((rng.standard_normal(3 * H * I) * 0.02).astype(np.float32), bits, 128)
                     for _ in range(E)])
    x = O.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)).reshape(T, H)
    sel, rw = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    return pool, x, sel, rw


def test_prefill_oracle_one_token_matches_decode_oracle():
    pool, x, sel, rw = _pf_case(T=1)
    slots = {e: e for e in range(5)}
    pf = O.moe_prefill_f64(pool, slots, x, sel, rw, 256, 128, 4)[0]
    _, _, dec = O.moe_layer_f64(pool, sel[0], rw[0], x[0], 256, 128, 4)
    err = np.linalg.norm(pf - dec) / np.linalg.norm(dec)
    assert 0 < err < 1e-2  # only the bf16 rounding of W and of the activation differ
    # a gate/up swap (SiLU on the up projection) is far off
    W = [O.bf16_bits_to_f32(O.dequant(pool[e][None], 256 * 128, 4)[0]).astype(np.float64) for e in sel[0]]
    xf = O.bf16_bits_to_f32(x[0]).astype(np.float64)
    bad = sum(w * (W[j][2].reshape(256, 128) @ ((lambda g, u: u / (1 + np.exp(-u)) * g)(
        W[j][0].reshape(128, 256) @ xf, W[j][1].reshape(128, 256) @ xf))) for j, w in enumerate(rw[0]))
    assert np.linalg.norm(bad - dec) / np.linalg.norm(dec) > 0.1


def test_prefill_oracle_additive_over_experts_and_token_equivariant():
    pool, x, sel, rw = _pf_case(T=9, seed=1)
    slots = {e: e for e in range(5)}
    full = O.moe_prefill_f64(pool, slots, x, sel, rw, 256, 128, 4)
    parts = sum(O.moe_prefill_f64(pool, {e: e}, x, sel, rw, 256, 128, 4) for e in range(5))
    assert np.allclose(full, parts, rtol=1e-12, atol=1e-12)
    perm = np.random.default_rng(2).permutation(9)
    permuted = O.moe_prefill_f64(pool, slots, x[perm], sel[perm], rw[perm], 256, 128, 4)
    assert np.allclose(permuted, full[perm], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- gpt-oss
def test_mxfp4_oracle_matches_transformers():
    # the reference pins its decoder against transformers' own (tests/test_gptoss.py:11-16);
    # here that library routine pins the oracle, over every code and a wide scale range
    from transformers.integrations.mxfp4 import convert_moe_packed_tensors

    rng = np.random.default_rng(5)
    blocks = rng.integers(0, 256, (3, 8, 5, 16), dtype=np.uint8)
    blocks[0, 0, 0] = np.arange(16, dtype=np.uint8) * 17  # every code in both nibbles
    scales = rng.integers(100, 150, (3, 8, 5), dtype=np.uint8)
    ref = convert_moe_packed_tensors(torch.from_numpy(blocks), torch.from_numpy(scales))  # [E, K, out]
    got = O.mxfp4_to_bf16_bits(blocks, scales)  # [E, out, K]
    assert np.array_equal(got.transpose(0, 2, 1), ref.contiguous().view(torch.int16).numpy().view(np.uint16))


def test_mxfp4_oracle_closed_forms():
    # value = FP4[code] * 2^(scale - 127): code 1 is 0.5, code 7 is 6, code 9 is -0.5
    b = np.zeros((1, 16), np.uint8)
    b[0, :3] = [0x71, 0x09, 0x00]
    for s, want in [(127, [0x3F00, 0x40C0, 0xBF00, 0x0000]),   # 0.5, 6, -0.5, 0
                    (0, [0x0020, 0x0140, 0x8020, 0x0000]),     # scale 2^-127: bf16 subnormals 2^-128 ...
                    (255, [0x7F80, 0x7F80, 0xFF80, 0x7FC0]),   # 2^128 = inf: 0 * inf = NaN
                    (130, [0x4080, 0x4240, 0xC080, 0x0000])]:  # 4, 48, -4
        got = O.mxfp4_to_bf16_bits(b, np.array([s], np.uint8))
        assert [int(v) for v in (got[0], got[1], got[2], got[4])] == want, s


def _gptoss_reference(N, seed=1):
    """transformers' GptOssMLP (float weights ~N(0, 0.3), bf16, CPU), the reference's test model
    (tests/test_gptoss.py:39-62), with its routing."""
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssMLP

    torch.manual_seed(seed)
    cfg = GptOssConfig(hidden_size=64, intermediate_size=64, num_hidden_layers=1, num_local_experts=8,
                       num_experts_per_tok=2, num_attention_heads=2, num_key_value_heads=1, head_dim=32, vocab_size=50)
    ref = GptOssMLP(cfg).to(torch.bfloat16)
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0, 0.3)
        x = torch.randn(1, N, 64).to(torch.bfloat16)
        want, _ = ref(x)
        logits = torch.nn.functional.linear(x.reshape(-1, 64), ref.router.weight, ref.router.bias)
        tv, ti = torch.topk(logits, 2, dim=-1)
        sc = torch.nn.functional.softmax(tv, dim=1, dtype=tv.dtype)
    return ref, x, want, ti, sc


def _w3_bits(ref, e):
    H, I = 64, 64
    gu, dn = ref.experts.gate_up_proj[e].data, ref.experts.down_proj[e].data
    f = gu.reshape(-1)
    w3 = torch.stack([f[: H * I], f[H * I :], dn.reshape(-1)])
    return w3.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("N", [1, 5])
def test_gptoss_oracle_matches_transformers(N):
    # bits = 16 (raw bf16 rows): the oracle restates gptoss.py:108-143 and must reproduce
    # transformers' GptOssMLP up to accumulation order; a planted mistake (gate/up bias
    # halves swapped, or a different clamp) must not
    ref, x, want, ti, sc = _gptoss_reference(N)
    H = I = 64
    pool = np.stack([_w3_bits(ref, e).reshape(-1).view(np.uint8) for e in range(8)])
    gub = ref.experts.gate_up_proj_bias.data.contiguous().view(torch.int16).numpy().view(np.uint16)
    db = ref.experts.down_proj_bias.data.contiguous().view(torch.int16).numpy().view(np.uint16)
    xb = x.reshape(N, H).contiguous().view(torch.int16).numpy().view(np.uint16)
    args = (pool, {e: e for e in range(8)}, xb, ti.numpy(), sc.float().numpy())

    def rel(bits_out):
        got = O.bf16_bits_to_f32(bits_out).reshape(N, H)
        w = want.reshape(N, H).float().numpy()
        return np.linalg.norm(got - w) / np.linalg.norm(w)

    err = rel(O.gptoss_block_ref(*args, gub, db, H, I, 16, 64))
    print(f"gpt-oss oracle vs transformers, N={N}: rel-L2 {err:.2e}")
    assert err <= 1e-2, err
    swapped = gub.reshape(8, I, 2)[:, :, ::-1].reshape(8, 2 * I).copy()
    assert rel(O.gptoss_block_ref(*args, swapped, db, H, I, 16, 64)) > 10 * max(err, 1e-3)
    assert rel(O.gptoss_block_ref(*args, gub, db, H, I, 16, 64, limit=0.5)) > 10 * max(err, 1e-3)


def test_gptoss_oracle_decode_sum_is_one_rounding():
    # N == 1 sums the k weighted outputs in float32 and rounds once (gptoss.py:131), so with
    # one expert of weight 1 it equals the per-expert output, and it is additive over a
    # split of the expert list up to that final rounding
    ref, x, want, ti, sc = _gptoss_reference(1, seed=3)
    H = I = 64
    pool = np.stack([_w3_bits(ref, e).reshape(-1).view(np.uint8) for e in range(8)])
    gub = ref.experts.gate_up_proj_bias.data.contiguous().view(torch.int16).numpy().view(np.uint16)
    db = ref.experts.down_proj_bias.data.contiguous().view(torch.int16).numpy().view(np.uint16)
    xb = x.reshape(1, H).contiguous().view(torch.int16).numpy().view(np.uint16)
    slots = {e: e for e in range(8)}
    both = O.bf16_bits_to_f32(O.gptoss_block_ref(pool, slots, xb, ti.numpy(), sc.float().numpy(), gub, db, H, I, 16, 64))
    parts = [O.bf16_bits_to_f32(O.gptoss_block_ref(pool, slots, xb, ti.numpy()[:, j:j + 1], sc.float().numpy()[:, j:j + 1],
                                                   gub, db, H, I, 16, 64)) for j in range(2)]
    assert np.allclose(both, parts[0] + parts[1], rtol=2 ** -7, atol=1e-6)
