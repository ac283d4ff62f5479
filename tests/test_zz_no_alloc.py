"""wisp_moe_decode_noalloc through the C ABI: the allocation-free layer (its activation
workspace is the library's own device array) against the existing entry point
wisp_moe_decode with a caller workspace, and against the binary64 oracle, on two calls
in a row (the second with a smaller layer, so stale scratch contents would show)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from wisp import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, H, I, bits, group, E, k):
    rng = np.random.default_rng(seed)
    n = H * I
    pool = np.stack([O.quantize((rng.standard_normal(3 * n) * 0.02).astype(np.float32), bits, group)
                     for _ in range(E)])
    sel, rw = O.route(rng.standard_normal((1, E)).astype(np.float32), k)
    x = O.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32))
    return pool, sel[0], rw[0], x


def _call_both(pool_np, sel, rw, x_np, H, I, bits, group):
    L, p = _lib.lib(), _lib.ptr
    k = len(sel)
    pool = torch.from_numpy(pool_np).to(DEV)
    meta = torch.from_numpy(O.meta(sel, rw)).to(DEV)
    x = torch.from_numpy(x_np.view(np.int16)).view(torch.bfloat16).to(DEV)
    out_ref = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    out_na = torch.full((H,), float("nan"), dtype=torch.bfloat16, device=DEV)
    act = torch.empty(L.wisp_act_bytes(k, I), dtype=torch.uint8, device=DEV)
    st = _lib.stream(torch.device(DEV))
    bf = _lib.WISP_DT_BF16
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    rc = L.wisp_moe_decode_noalloc(p(pool), pool.stride(0), pool.shape[0], p(meta), k, p(x), bf, H, I, bits, group,
                                   p(out_na), bf, st)
    _lib.check(rc, "wisp_moe_decode_noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    _lib.check(L.wisp_moe_decode(p(pool), pool.stride(0), pool.shape[0], p(meta), k, p(x), bf, H, I, bits, group,
                                 p(act), p(out_ref), bf, st), "wisp_moe_decode")
    torch.cuda.synchronize()
    return out_na, out_ref


def test_noalloc_matches_workspace_entry_two_calls():
    for seed, (H, I, bits, group, E, k) in ((1, (2048, 768, 4, 128, 10, 8)), (2, (256, 128, 3, 128, 6, 3))):
        pool, sel, rw, x = _case(seed, H, I, bits, group, E, k)
        got, ref = _call_both(pool, sel, rw, x, H, I, bits, group)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (H, I, bits)
        _, _, r64 = O.moe_layer_f64(pool, sel, rw, x, H, I, bits, group)
        r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(r64.astype(np.float32))).astype(np.float64)
        g = got.float().cpu().numpy().astype(np.float64)
        err = float(np.linalg.norm(g - r) / np.linalg.norm(r))
        print(f"noalloc H={H} I={I} bits={bits} k={k}: rel-L2 vs oracle {err:.3e}")
        assert err <= 1e-3, err


def test_noalloc_refuses_beyond_its_scratch():
    L, p = _lib.lib(), _lib.ptr
    H, I, group = 4096, 32768, 128  # k * I = 9 * 32768 > 262144
    buf = torch.zeros(64, dtype=torch.uint8, device=DEV)
    nb = O.expert_nbytes(H * I, 4, group)
    rc = L.wisp_moe_decode_noalloc(p(buf), nb, 1, p(buf), 9, p(buf), _lib.WISP_DT_BF16, H, I, 4, group, p(buf),
                                   _lib.WISP_DT_BF16, _lib.stream(torch.device(DEV)))
    assert rc == _lib.WISP_EINVAL
    assert b"no-alloc scratch" in L.wisp_last_error()
