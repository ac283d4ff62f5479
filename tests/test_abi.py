"""CPU checks of the C-ABI library and the host logic around it (no kernel launches).

The library is loaded here without a GPU: every symbol include/wisp_hip.h declares must
be exported, and argument validation must reject bad calls before anything reaches HIP.
"""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O
from wisp import _lib, kernels, quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wisp_hip.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(wisp_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 14
    for name in names:
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_abi_version_matches_header():
    m = re.search(r"#define WISP_ABI_VERSION (\d+)", open(HEADER).read())
    assert _lib.lib().wisp_abi_version() == int(m.group(1)) == _lib.ABI_VERSION


@pytest.mark.parametrize("bits", [16, 8, 4, 3, 2])
@pytest.mark.parametrize("n,group", [(1572864, 128), (2048, 32), (32768, 128), (100, 128), (96, 96)])
def test_expert_nbytes_agrees(bits, n, group):
    L = _lib.lib()
    try:
        want = O.expert_nbytes(n, bits, group)
    except ValueError:
        want = -1
    assert L.wisp_expert_nbytes(n, bits, group) == want
    if want >= 0:
        assert quant.expert_nbytes(n, bits, group) == want


def test_act_bytes():
    L = _lib.lib()
    assert L.wisp_act_bytes(8, 768) == 8 * 768 * 4
    assert L.wisp_act_bytes(0, 768) == -1


def test_tuning_validation():
    L = _lib.lib()
    assert L.wisp_set_tuning(3, 0, 0) == _lib.WISP_EINVAL
    assert b"gu_rows" in L.wisp_last_error()
    assert L.wisp_set_tuning(0, 0, 5) == _lib.WISP_EINVAL
    assert L.wisp_set_tuning(0, 0, 0) == _lib.WISP_OK
    with pytest.raises(ValueError):
        kernels.set_tuning(gu_rows=6)


FAKE = ctypes.c_void_p(0x100000)  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize(
    "args,needle",
    [
        (dict(bits=5), b"bits"),
        (dict(k=0), b"k must"),
        (dict(k=8193), b"k must"),
        (dict(x_dtype=3), b"x_dtype"),
        (dict(H=2000), b"multiples of group"),
        (dict(group=64 + 16, H=2080 // 1, I=80 * 9), b"multiple of 32"),
        (dict(slot_bytes=1000), b"smaller than one expert"),
        (dict(nslots=0), b"nslots"),
        (dict(pool=None), b"null"),
    ],
)
def test_layer_argument_validation(args, needle):
    L = _lib.lib()
    a = dict(pool=FAKE, slot_bytes=2506752, nslots=128, meta=FAKE, k=8, x=FAKE, x_dtype=_lib.WISP_DT_BF16, H=2048,
             I=768, bits=4, group=128, act=FAKE, stream=None)
    a.update(args)
    rc = L.wisp_moe_gate_up(*a.values())
    assert rc == _lib.WISP_EINVAL, rc
    assert needle in L.wisp_last_error()
    if "x_dtype" in args:
        return
    d = (a["pool"], a["slot_bytes"], a["nslots"], a["meta"], a["k"], FAKE, a["H"], a["I"], a["bits"], a["group"])
    assert L.wisp_moe_down_sum(*d, FAKE, _lib.WISP_DT_BF16, None) == _lib.WISP_EINVAL
    assert L.wisp_moe_down(*d, FAKE, None) == _lib.WISP_EINVAL
    x = (FAKE, _lib.WISP_DT_BF16)
    assert L.wisp_moe_decode(*d[:5], *x, *d[6:], FAKE, FAKE, _lib.WISP_DT_BF16, None) == _lib.WISP_EINVAL


def test_output_dtype_validation():
    L = _lib.lib()
    d = (FAKE, 2506752, 128, FAKE, 8, FAKE, 2048, 768, 4, 128)
    assert L.wisp_moe_down_sum(*d, FAKE, 7, None) == _lib.WISP_EINVAL
    assert b"out_dtype" in L.wisp_last_error()
    assert L.wisp_moe_down_sum(*d, None, _lib.WISP_DT_F32, None) == _lib.WISP_EINVAL
    assert b"null out" in L.wisp_last_error()


def test_alignment_validation():
    L = _lib.lib()
    bf = _lib.WISP_DT_BF16
    rc = L.wisp_moe_gate_up(ctypes.c_void_p(0x100004), 2506752, 128, FAKE, 8, FAKE, bf, 2048, 768, 4, 128, FAKE, None)
    assert rc == _lib.WISP_EALIGN
    rc = L.wisp_moe_gate_up(FAKE, 2506752 + 4, 128, FAKE, 8, FAKE, bf, 2048, 768, 4, 128, FAKE, None)
    assert rc == _lib.WISP_EALIGN
    rc = L.wisp_moe_gate_up(FAKE, 2506752, 128, FAKE, 8, ctypes.c_void_p(0x100008), _lib.WISP_DT_F32, 2048, 768, 4,
                            128, FAKE, None)
    assert rc == _lib.WISP_EALIGN


def test_format_entry_validation():
    L = _lib.lib()
    assert L.wisp_dequant(FAKE, 100, None, 1, 1, 1572864, 4, 128, FAKE, None) == _lib.WISP_EINVAL  # stride < nbytes
    assert L.wisp_dequant(FAKE, 2506752, None, 1, 1, 1572864, 5, 128, FAKE, None) == _lib.WISP_EINVAL
    assert L.wisp_quantize(FAKE, 2, 1572864, 4, 128, FAKE, None) == _lib.WISP_EINVAL  # dtype code
    assert L.wisp_pack(FAKE, 7, 4, FAKE, None) == _lib.WISP_EINVAL
    assert L.wisp_unpack(FAKE, 9, 3, FAKE, None) == _lib.WISP_EINVAL
    assert L.wisp_act_read(FAKE, 8, 100, 4, FAKE, None) == _lib.WISP_EINVAL
    # empty work is a no-op that succeeds without touching the device
    assert L.wisp_pack(FAKE, 0, 4, FAKE, None) == _lib.WISP_OK
    assert L.wisp_dequant(FAKE, 2506752, None, 0, 1, 1572864, 4, 128, FAKE, None) == _lib.WISP_OK


def test_rope_argument_validation():
    L = _lib.lib()
    ok = (FAKE, 128, FAKE, 128, FAKE, FAKE, 32, 4, 128, 1, FAKE, FAKE, None)
    bad_d = (FAKE, 128, FAKE, 128, FAKE, FAKE, 32, 4, 127, 1, FAKE, FAKE, None)
    assert L.wisp_rope_decode(*bad_d) == _lib.WISP_EINVAL  # odd head dim
    bad_stride = (FAKE, 64, FAKE, 128, FAKE, FAKE, 32, 4, 128, 1, FAKE, FAKE, None)
    assert L.wisp_rope_decode(*bad_stride) == _lib.WISP_EINVAL
    bad_dtype = ok[:9] + (2,) + ok[10:]
    assert L.wisp_rope_decode(*bad_dtype) == _lib.WISP_EINVAL
    null_q = (None,) + ok[1:]
    assert L.wisp_rope_decode(*null_q) == _lib.WISP_EINVAL


def test_prefill_argument_validation():
    L = _lib.lib()
    nb = 2506752

    def call(**kw):
        a = dict(pool=FAKE, slot_bytes=nb, nslots=128, groups=FAKE, ngroups=4, max_group=8, tok=FAKE, w=FAKE,
                 back=FAKE, pairs=64, x=FAKE, T=8, k=8, H=2048, I=768, bits=4, group=128, ws=FAKE, out=FAKE, acc=None)
        a.update(kw)
        return L.wisp_moe_prefill(*a.values(), None)

    assert call(group=64) == _lib.WISP_EINVAL  # one quant group per K step
    assert call(H=2176, I=768, slot_bytes=nb * 2) == _lib.WISP_EINVAL  # H % 256
    assert call(pairs=65) == _lib.WISP_EINVAL  # more pairs than T*k
    assert call(bits=8) == _lib.WISP_EINVAL
    assert call(out=None) == _lib.WISP_EINVAL  # neither out nor acc
    assert call(slot_bytes=nb - 16) == _lib.WISP_EINVAL
    assert call(x=ctypes.c_void_p(0x100002)) == _lib.WISP_EALIGN
    assert call(k=33, T=2, pairs=64) == _lib.WISP_EINVAL  # k <= 32
    assert call(out=ctypes.c_void_p(0x100004)) == _lib.WISP_EALIGN  # out: 8-byte stores
    assert call(out=None, acc=ctypes.c_void_p(0x100008)) == _lib.WISP_EALIGN  # acc: 16-byte
    assert L.wisp_prefill_ws_bytes(64, 2048, 768) == 64 * 768 * 2 + 64 * 2048 * 4


def test_decode_layer_argument_validation():
    """The graph decoder's dense kernels reject bad shapes and pointers before any launch."""
    L = _lib.lib()

    def gemv(**kw):
        a = dict(a=FAKE, a_row=None, b=None, norm_w=None, eps=1e-6, h_out=None, x_out=None, w0=FAKE, w1=None,
                 w2=None, r1=128, r2=128, O=128, K=2048, res=None, y=FAKE)
        a.update(kw)
        return L.wisp_dl_gemv(*a.values(), None)

    assert gemv(K=2052) == _lib.WISP_EINVAL  # K a multiple of 8
    assert gemv(K=16384) == _lib.WISP_EINVAL  # K <= 8192
    assert gemv(O=0, r1=0, r2=0) == _lib.WISP_EINVAL
    assert gemv(r1=64, r2=32) == _lib.WISP_EINVAL  # r1 <= r2
    assert gemv(r1=64, r2=128) == _lib.WISP_EINVAL  # rows [64, 128) need w1
    assert gemv(r1=64, r2=64) == _lib.WISP_EINVAL  # rows [64, 128) need w2
    assert gemv(b=FAKE) == _lib.WISP_EINVAL  # b, h_out, x_out only with the RMSNorm prologue
    assert gemv(y=None) == _lib.WISP_EINVAL
    assert gemv(a=ctypes.c_void_p(0x100008)) == _lib.WISP_EALIGN
    assert gemv(w0=ctypes.c_void_p(0x100004)) == _lib.WISP_EALIGN

    def rope(**kw):
        a = dict(qkv=FAKE, qn=FAKE, kn=FAKE, eps=1e-6, cos=FAKE, sin=FAKE, pos=FAKE, hq=32, hk=4, d=128, kc=FAKE,
                 vc=FAKE, hs=4096 * 128, qo=FAKE)
        a.update(kw)
        return L.wisp_dl_qk_rope(*a.values(), None)

    assert rope(d=96) == _lib.WISP_EINVAL  # head dim 64, 128 or 256
    assert rope(hk=0) == _lib.WISP_EINVAL
    assert rope(hs=64) == _lib.WISP_EINVAL  # head stride >= d
    assert rope(pos=None) == _lib.WISP_EINVAL

    def rt(**kw):
        a = dict(logits=FAKE, E=128, k=8, norm=1, row=FAKE, host_row=None, host_flag=None, seq=None)
        a.update(kw)
        return L.wisp_dl_route(*a.values(), None)

    assert rt(E=0) == _lib.WISP_EINVAL
    assert rt(E=2048) == _lib.WISP_EINVAL  # E <= 1024
    assert rt(k=17) == _lib.WISP_EINVAL  # k <= 16
    assert rt(E=4, k=5) == _lib.WISP_EINVAL  # k <= E
    assert rt(host_row=FAKE) == _lib.WISP_EINVAL  # host_row, host_flag and seq go together
    assert rt(host_row=FAKE, host_flag=FAKE) == _lib.WISP_EINVAL
    assert rt(row=None) == _lib.WISP_EINVAL


def test_expert_cache_needs_a_gpu():
    """The slot pool is device memory: without a GPU the cache refuses to build (no host pool)."""
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from wisp.cache import ExpertCache
    from wisp.store import ExpertStore

    st = ExpertStore(1, 2, 256 * 128, 4, 128, pin=False)
    with pytest.raises(RuntimeError):
        ExpertCache(st, 2, device="cuda:0")


def test_no_cpu_fallback():
    """The product path raises on CPU tensors instead of computing on the host."""
    w3 = torch.randn(3, 2048)
    with pytest.raises(RuntimeError, match="ROCm device"):
        quant.quantize(w3, 4, 128)
    with pytest.raises(RuntimeError, match="ROCm device"):
        quant.dequant(torch.zeros(1, 7680, dtype=torch.uint8), 2048, 4, 128)
    pool = torch.zeros(2, quant.expert_nbytes(256 * 128, 4, 128), dtype=torch.uint8)
    meta = torch.tensor([0.0, 1.0, 0.5, 0.5])
    with pytest.raises(RuntimeError, match="ROCm device"):
        kernels.moe_decode_q4_fast(pool, meta, torch.zeros(256, dtype=torch.bfloat16), 2, 256 * 128, 256, 128)
    # the reference's shape assertion (kernels.py:191) comes first
    with pytest.raises(AssertionError):
        kernels.moe_decode_q4_fast(pool, meta, torch.zeros(256, dtype=torch.bfloat16), 2, 256 * 128, 250, 128)
    # k beyond WISP_MAX_K is refused before any device work
    with pytest.raises(AssertionError, match="k must"):
        kernels.moe_decode_q4_fast(pool, meta, torch.zeros(256), 8193, 256 * 128, 256, 128)
    # x of a non-float dtype is refused; float64 x would be rounded to fp32 (no CPU path either way)
    with pytest.raises(RuntimeError, match="ROCm device"):
        kernels.moe_decode_q4_fast(pool, meta, torch.zeros(256, dtype=torch.float64), 2, 256 * 128, 256, 128)
    with pytest.raises(TypeError, match="float"):
        kernels._prep_x_any(torch.zeros(256, dtype=torch.int32))


def test_meta_layout_helpers():
    m = O.meta(np.array([5, 0, 3]), np.array([0.5, 0.25, 0.25], np.float32))
    assert m.tolist() == [5.0, 0.0, 3.0, 0.5, 0.25, 0.25]


@pytest.mark.parametrize("chunk", [64, 32, 1])
def test_prefill_work_items_partition_each_group(chunk):
    # work items of the grouped prefill: consecutive pieces of each expert's pair
    # range, none larger than `chunk`, largest first, covering every pair once
    rng = np.random.default_rng(chunk)
    sel = np.stack([rng.choice(16, 4, replace=False) for _ in range(97)])
    order, tok, back, uniq, first, count = kernels._prefill_plan(sel, list(range(0, 16, 2)), 4)
    ex, start, cnt = kernels._prefill_chunks(uniq, first, count, chunk)
    assert (cnt >= 1).all() and (cnt <= chunk).all()
    assert (np.diff(cnt) <= 0).all()
    covered = np.zeros(order.size, np.int64)
    for e, s, c in zip(ex, start, cnt):
        covered[s:s + c] += 1
        g = int(np.flatnonzero(uniq == e)[0])
        assert first[g] <= s and s + c <= first[g] + count[g]
    assert (covered == 1).all()
    assert kernels._prefill_chunks(uniq, first, count, 1 << 20)[2].tolist() == sorted(count.tolist(), reverse=True)
