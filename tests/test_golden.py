"""Golden vectors written by the reference implementation itself (tests/golden/make_golden.py:
wisp/quant.py, and wisp/kernels.py under Triton's CPU interpreter), checked against the
oracle (CPU) and the HIP path through the C ABI (GPU).

Bars: quantize and dequant bit-exact (sha256 of the whole buffer); fp32 rope_decode
bit-exact (the reference rotates in binary32 with separately rounded products,
kernels.py:344).

Rounding of bf16 outputs. Triton's CPU interpreter stores float32 into a bf16 pointer by
truncation (round toward zero), whereas torch's casts and the compiled kernels round to
nearest even. So the fixtures of the Triton kernels that store bf16 themselves
(moe_decode_q4_fast, moe_decode_q3_fast, rope_decode in bf16) hold the truncated float32
result, and moe_decode_q4, whose final weighted sum and cast are torch ops
(kernels.py:137), holds the rounded one. The oracle is checked bit for bit under the
fixture's own rounding (it agrees on every element); the HIP kernels, which round to
nearest even like the compiled reference, must be within one bf16 ulp of every fixture
element and, for moe_decode_q4, within 1e-3 relative L2.
"""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
SHAPE = GOLDEN["shape"]
H, I, G, N = SHAPE["H"], SHAPE["I"], SHAPE["G"], SHAPE["n"]
TOL = 1e-3


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _expert_input(seed: int) -> np.ndarray:
    """bf16 bits [3, n], as make_golden.expert_input (numpy's frozen RandomState stream)."""
    w = (np.random.RandomState(seed).standard_normal((3, N)) * 0.05).astype(np.float32)
    return O.f32_to_bf16_bits(w).reshape(3, N)


def _x_input(seed: int) -> np.ndarray:
    return O.f32_to_bf16_bits(np.random.RandomState(seed).standard_normal(H).astype(np.float32))


def _bf16_f32(bits) -> np.ndarray:
    return O.bf16_bits_to_f32(np.asarray(bits, dtype=np.uint16))


def _rel_l2(got, ref) -> float:
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def _oracle_pool(bits: int) -> np.ndarray:
    rows = [q for q in GOLDEN["quant"] if q["bits"] == bits]
    return np.stack([O.quantize(_bf16_f32(_expert_input(q["seed"])), bits, G) for q in rows])


def _trunc_bf16(f32: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits by truncation (how the interpreter's bf16 stores round)."""
    return (np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _ulps(a_bits, b_bits) -> np.ndarray:
    """|distance| in bf16 ulps between bf16 bit patterns (sign-magnitude ordered)."""
    def order(b):
        b = np.asarray(b, dtype=np.uint16).astype(np.int64)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(order(a_bits) - order(b_bits))


def _rope_array(vals, dtype: str) -> np.ndarray:
    a = np.asarray(vals)
    return a.astype(np.int16).view(np.uint16) if dtype == "bfloat16" else a.astype(np.int32).view(np.float32)


# ---------------------------------------------------------------- oracle (CPU)
@pytest.mark.parametrize("case", range(len(GOLDEN["quant"])))
def test_oracle_quantize_dequant_bit_exact_vs_reference(case):
    q = GOLDEN["quant"][case]
    wb = _expert_input(q["seed"])
    assert _sha(wb) == q["input_sha256"]
    packed = O.quantize(_bf16_f32(wb), q["bits"], G)
    assert packed.size == q["nbytes"]
    assert packed[:64].tolist() == q["packed_head"]
    assert _sha(packed) == q["packed_sha256"]
    d = O.dequant(packed, N, q["bits"], G)[0]
    assert d.reshape(-1)[:64].tolist() == q["dequant_head"]
    assert _sha(d) == q["dequant_sha256"]


@pytest.mark.parametrize("case", range(len(GOLDEN["decode"])))
def test_oracle_decode_layer_vs_reference_kernels(case):
    c = GOLDEN["decode"][case]
    x = _x_input(c["x_seed"])
    assert _sha(x) == c["x_sha256"]
    pool = _oracle_pool(c["bits"])
    w = np.asarray(c["weights_f32"], np.float32)
    _, _, out = O.moe_layer_f64(pool, c["slots"], w, x, H, I, c["bits"], G)
    f32 = out.astype(np.float32)
    mine = O.f32_to_bf16_bits(f32) if c["fn"] == "moe_decode_q4" else _trunc_bf16(f32)
    assert np.array_equal(mine, np.asarray(c["out_bf16"], np.uint16))


@pytest.mark.parametrize("case", range(len(GOLDEN["rope"])))
def test_oracle_rope_bit_exact_vs_reference(case):
    r = GOLDEN["rope"][case]
    dt, hq, hk, d = r["dtype"], r["hq"], r["hk"], r["d"]
    conv = (lambda a: _bf16_f32(a)) if dt == "bfloat16" else (lambda a: a)
    q = conv(_rope_array(r["q"], dt)).reshape(hq, d)
    k = conv(_rope_array(r["k"], dt)).reshape(hk, d)
    cs = conv(_rope_array(r["cos"], dt)).reshape(d)
    sn = conv(_rope_array(r["sin"], dt)).reshape(d)
    qo, ko = O.rope(q, cs, sn), O.rope(k, cs, sn)
    if dt == "bfloat16":
        qo, ko = _trunc_bf16(qo), _trunc_bf16(ko)
    assert np.array_equal(qo.reshape(-1), _rope_array(r["qo"], dt).reshape(-1))
    assert np.array_equal(ko.reshape(-1), _rope_array(r["ko"], dt).reshape(-1))


# ---------------------------------------------------------------- HIP path (GPU)
def _dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).astype(np.int16)).view(torch.bfloat16).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(GOLDEN["quant"])))
def test_gpu_quantize_dequant_bit_exact_vs_reference(case):
    from wisp import quant

    q = GOLDEN["quant"][case]
    w = _dev_bf16(_expert_input(q["seed"]))
    packed = quant.quantize(w, q["bits"], G)
    torch.cuda.synchronize()
    pk = packed.cpu().numpy()
    assert pk.size == q["nbytes"] and _sha(pk) == q["packed_sha256"]
    d = quant.dequant(packed[None], N, q["bits"], G)
    dn = d.view(torch.int16).cpu().numpy().view(np.uint16)
    assert _sha(dn[0]) == q["dequant_sha256"]


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(GOLDEN["decode"])))
def test_gpu_decode_layer_vs_reference_kernels(case):
    from wisp import kernels, quant

    c = GOLDEN["decode"][case]
    rows = [q for q in GOLDEN["quant"] if q["bits"] == c["bits"]]
    pool = torch.stack([quant.quantize(_dev_bf16(_expert_input(q["seed"])), c["bits"], G) for q in rows])
    x = _dev_bf16(_x_input(c["x_seed"]))
    w = torch.tensor(c["weights_f32"], dtype=torch.float32, device="cuda")
    slots = torch.tensor(c["slots"], dtype=torch.int64, device="cuda")
    if c["fn"] == "moe_decode_q4":
        out = kernels.moe_decode_q4(pool, slots, x, w, N, H, I)
    else:
        meta = torch.cat([slots.float(), w])
        out = getattr(kernels, c["fn"])(pool, meta, x, len(c["slots"]), N, H, I)
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert int(_ulps(got, c["out_bf16"]).max()) <= 1, c["fn"]
    if c["fn"] == "moe_decode_q4":  # both rounded to nearest even
        ref = _bf16_f32(c["out_bf16"]).astype(np.float64)
        assert _rel_l2(_bf16_f32(got).astype(np.float64), ref) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(GOLDEN["rope"])))
def test_gpu_rope_vs_reference(case):
    from wisp import kernels

    r = GOLDEN["rope"][case]
    dt, hq, hk, d = r["dtype"], r["hq"], r["hk"], r["d"]

    def dev(vals, shape):
        a = _rope_array(vals, dt)
        t = torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16) if dt == "bfloat16" else torch.from_numpy(a)
        return t.reshape(shape).cuda()

    q, k = dev(r["q"], (1, hq, 1, d)), dev(r["k"], (1, hk, 1, d))
    cs, sn = dev(r["cos"], (1, 1, d)), dev(r["sin"], (1, 1, d))
    qo, ko = kernels.rope_decode(q, k, cs, sn)
    torch.cuda.synchronize()

    def raw(t):
        t = t.contiguous().cpu()
        return t.view(torch.int16).numpy().view(np.uint16) if dt == "bfloat16" else t.numpy()

    if dt == "bfloat16":  # round to nearest even vs the fixture's truncation: within one ulp
        assert int(_ulps(raw(qo).reshape(-1), _rope_array(r["qo"], dt).reshape(-1)).max()) <= 1
        assert int(_ulps(raw(ko).reshape(-1), _rope_array(r["ko"], dt).reshape(-1)).max()) <= 1
    else:
        assert np.array_equal(raw(qo).reshape(-1), _rope_array(r["qo"], dt).reshape(-1))
        assert np.array_equal(raw(ko).reshape(-1), _rope_array(r["ko"], dt).reshape(-1))
