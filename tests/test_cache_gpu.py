"""Expert cache on the GPU: the hipMalloc slot pool, pinned-host paging on the side stream,
copy ordering, decode-on-load, resize and the per-layer prepare step, against the oracle
(bookkeeping: oracle/cache_core_ref.py; bytes: the host store; math: oracle/oracle.py)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.cache_core_ref import RefCore
from wisp import _lib, kernels
from wisp.cache import ExpertCache
from wisp.store import ExpertStore

pytestmark = pytest.mark.gpu
H, I, G = 256, 128, 128
N = H * I


def _store(L, E, bits, seed=0):
    rng = np.random.default_rng(seed)
    st = ExpertStore(L, E, N, bits, G)
    for key in range(L * E):
        w = (rng.standard_normal(3 * N) * 0.02).astype(np.float32)
        st.host[key].copy_(torch.from_numpy(O.quantize(w, bits, G)))
    return st


def _rows(cache, slots):
    return cache.gpu[torch.as_tensor(slots, device=cache.device)].cpu()


def test_pool_is_a_native_allocation_viewed_by_torch():
    st = _store(1, 6, 4)
    c = ExpertCache(st, 4)
    assert st.pinned
    assert c.gpu.shape == (4, st.nbytes) and c.gpu.dtype == torch.uint8 and c.gpu.is_cuda
    assert c.gpu.data_ptr() == _lib.lib().wisp_cache_pool(c._h)
    c.free()


@pytest.mark.parametrize("copy", ["dma", "kernel"])
def test_ensure_pages_rows_and_matches_reference_bookkeeping(copy):
    st = _store(2, 6, 4, seed=1)
    c = ExpertCache(st, 5, copy=copy)
    assert c.copy == copy
    ref = RefCore(5, "lru")
    rng = np.random.default_rng(2)
    for it in range(30):
        keys = [int(v) for v in rng.choice(12, size=3, replace=False)]
        slots = c.ensure(keys)
        rslots, _ = ref.ensure(keys)
        assert slots == rslots, it
        got = _rows(c, slots)
        for j, k in enumerate(keys):
            assert torch.equal(got[j], st.host[k]), (it, k)
    assert c.core.stats == ref.counts
    assert c.n_loads == ref.counts["misses"] and c.bytes_h2d == c.n_loads * st.nbytes
    c.free()


@pytest.mark.parametrize("copy", ["dma", "kernel"])
def test_copy_waits_for_queued_reads_of_the_evicted_slot(copy):
    """cache.py:54-56: a copy into a slot starts only after the compute work queued before it."""
    st = _store(1, 4, 4, seed=3)
    c = ExpertCache(st, 1, copy=copy)
    (s,) = c.ensure([0])
    torch.cuda.synchronize()
    a = torch.randn(4096, 4096, device="cuda")
    for _ in range(8):  # keep the compute stream busy for a while
        a = a @ a
        a = a / a.norm()
    snap = c.gpu[s].clone()  # queued after the matmuls, before the eviction copy
    c.ensure([1])  # evicts key 0 from slot s
    torch.cuda.synchronize()
    assert torch.equal(snap.cpu(), st.host[0])
    assert torch.equal(c.gpu[s].cpu(), st.host[1])
    c.free()


def test_layer_through_the_cache_matches_oracle():
    st = _store(1, 10, 4, seed=4)
    c = ExpertCache(st, 10)
    rng = np.random.default_rng(5)
    sel, rw = O.route(rng.standard_normal((1, 10)).astype(np.float32), 4)
    keys = [int(v) for v in sel[0]]
    meta_host = torch.zeros(8, dtype=torch.float32).pin_memory()
    meta_dev = torch.zeros(8, dtype=torch.float32, device="cuda")
    slots = c.prepare_layer(keys, rw[0], meta_host, meta_dev)
    x = O.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32))
    out = kernels.moe_decode_q4_fast(c.gpu, meta_dev, torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda(),
                                     4, N, H, I, G)
    torch.cuda.synchronize()
    assert meta_dev.cpu().tolist() == [float(s) for s in slots] + rw[0].tolist()
    pool_np = st.host.numpy()
    _, _, ref = O.moe_layer_f64(pool_np, keys, rw[0], x, H, I, 4, G)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))
    g = out.float().cpu().numpy()
    assert np.linalg.norm(g - r) / np.linalg.norm(r) <= 1e-3
    c.free()


@pytest.mark.parametrize("bits", [4, 3])
def test_decode_on_load_holds_bit_exact_bf16(bits):
    st = _store(1, 5, bits, seed=6)
    c = ExpertCache(st, 3, decode_on_load=True, staging_rows=2)
    slots = c.ensure([4, 1, 3])
    w = c.weights(slots)
    torch.cuda.synchronize()
    for j, k in enumerate([4, 1, 3]):
        ref = O.dequant(st.host[k].numpy()[None], N, bits, G)[0]
        assert np.array_equal(w[j].view(torch.int16).cpu().numpy().view(np.uint16), ref)
    c.free()


def test_weights_batched_and_cpu_weights():
    st = _store(1, 6, 4, seed=7)
    c = ExpertCache(st, 6)
    slots = c.ensure([5, 0, 2])
    wb = c.weights_batched(torch.as_tensor(slots, device="cuda"))
    for j, k in enumerate([5, 0, 2]):
        ref = O.dequant(st.host[k].numpy()[None], N, 4, G)[0]
        assert np.array_equal(wb[j].view(torch.int16).cpu().numpy().view(np.uint16), ref)
    cw = c.cpu_weights(2)
    assert not cw.is_cuda and torch.equal(cw, wb[2].cpu())
    c.free()


def test_resize_keeps_hottest_and_recopies():
    st = _store(1, 12, 4, seed=8)
    c = ExpertCache(st, 8)
    ref = RefCore(8, "lru")
    for keys in ([0, 1, 2], [3, 4, 5], [6, 7, 8], [0, 3]):
        assert c.ensure(keys) == ref.ensure(keys)[0]
    for size in (3, 10):
        c.resize(size)
        ref, loads = ref.resized(size)
        assert c.gpu.shape[0] == size
        assert c.core.key2slot == ref.where
        for k, s in loads:
            assert torch.equal(c.gpu[s].cpu(), st.host[k])
    assert c.ensure([9, 0]) == ref.ensure([9, 0])[0]
    c.free()


def test_failed_resize_reports_the_missing_pool():
    """A resize whose new pool cannot be allocated leaves the cache without a pool: the
    calls that would touch it return an error instead of dereferencing it."""
    st = _store(1, 6, 4, seed=9)
    c = ExpertCache(st, 4)
    assert c.ensure([0, 1]) == [0, 1]
    huge = 1 << 23  # 2^23 slots of ~61 KB (512 GB): past the device memory
    with pytest.raises((RuntimeError, ValueError)):
        c.resize(huge)
    assert _lib.lib().wisp_cache_pool(c._h) is None
    with pytest.raises(RuntimeError, match="pool not allocated"):
        c.ensure([2, 3])
    assert not _lib.lib().wisp_cache_pool_dlpack(c._h)
    c.free()


def test_prefetch_and_admit_async_issue_copies():
    st = _store(1, 8, 4, seed=9)
    c = ExpertCache(st, 4, admit_after=0.5)
    slots = c.ensure([0, 1])
    n = c.prefetch([2, 3, 0], slots)
    assert n == 2
    c.sync_compute()
    torch.cuda.synchronize()
    for k in (2, 3):
        assert torch.equal(c.gpu[c.core.lookup(k)].cpu(), st.host[k])
    hk, hs, mk = c.split([4, 2])
    assert hk == [2] and mk == [4]
    assert c.admit_async(mk, hs) == 1
    c.sync_compute()
    torch.cuda.synchronize()
    assert torch.equal(c.gpu[c.core.lookup(4)].cpu(), st.host[4])
    c.free()


def test_graph_replays_follow_prepare_layer():
    """graphdec.py:216-231 contract: the kernels are captured once; the host step between
    replays pages experts in and rewrites meta, and each replay computes the new routing."""
    st = _store(1, 16, 4, seed=10)
    c = ExpertCache(st, 6)
    k = 4
    meta_host = torch.zeros(2 * k, dtype=torch.float32).pin_memory()
    meta_dev = torch.zeros(2 * k, dtype=torch.float32, device="cuda")
    rng = np.random.default_rng(11)
    x_np = O.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32))
    x = torch.from_numpy(x_np.view(np.int16)).view(torch.bfloat16).cuda()
    c.prepare_layer(list(range(k)), [0.25] * k, meta_host, meta_dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kernels.moe_decode_q4_fast(c.gpu, meta_dev, x, k, N, H, I, G)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = kernels.moe_decode_q4_fast(c.gpu, meta_dev, x, k, N, H, I, G)
    for it in range(6):
        sel, rw = O.route(rng.standard_normal((1, 16)).astype(np.float32), k)
        keys = [int(v) for v in sel[0]]
        c.prepare_layer(keys, rw[0], meta_host, meta_dev)
        g.replay()
        torch.cuda.synchronize()
        _, _, ref = O.moe_layer_f64(st.host.numpy(), keys, rw[0], x_np, H, I, 4, G)
        r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))
        got = out.float().cpu().numpy()
        assert np.linalg.norm(got - r) / np.linalg.norm(r) <= 1e-3, it
    c.free()


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_page_kernel_copies_rows_exactly(bits):
    """copy="kernel": the GPU reads the pinned store rows itself; the pages must equal the host
    rows byte for byte, for batches below, at and above one launch's 16 rows."""
    st = _store(3, 12, bits, seed=3 + bits)  # 36 distinct rows
    c = ExpertCache(st, 40, copy="kernel")
    assert c.copy == "kernel"
    rng = np.random.default_rng(bits)
    done = set()
    for n in (1, 5, 16, 17, 36):
        keys = [int(v) for v in rng.choice(36, size=n, replace=False)]
        slots = c.ensure(keys)
        got = _rows(c, slots)
        for j, k in enumerate(keys):
            assert torch.equal(got[j], st.host[k]), (n, k)
        done.update(keys)
    assert c.n_loads == len(done)
    c.free()


def test_page_kernel_follows_reference_bookkeeping_under_eviction():
    st = _store(2, 6, 4, seed=11)
    c = ExpertCache(st, 5, copy="kernel")
    ref = RefCore(5, "lru")
    rng = np.random.default_rng(12)
    for it in range(30):
        keys = [int(v) for v in rng.choice(12, size=3, replace=False)]
        slots = c.ensure(keys)
        assert slots == ref.ensure(keys)[0], it
        got = _rows(c, slots)
        for j, k in enumerate(keys):
            assert torch.equal(got[j], st.host[k]), (it, k)
    c.free()


def test_page_kernel_needs_a_pinned_store():
    st = ExpertStore(1, 4, N, 4, G, pin=False)
    assert not st.pinned
    with pytest.raises(RuntimeError):
        ExpertCache(st, 2, copy="kernel")
    c = ExpertCache(st, 2, copy="auto")  # falls back to the DMA copies
    assert c.copy == "dma"
    c.free()


@pytest.mark.parametrize("copy", ["dma", "kernel"])
def test_signaled_step_waits_pages_and_writes_meta(copy):
    """wisp_cache_prepare_signaled: a flag that never moves times out (host-side spin only); a
    moved flag is taken at once with the row's ids and weights; bad ids are refused."""
    st = _store(1, 6, 4, seed=21)
    c = ExpertCache(st, 4, copy=copy)
    row = torch.zeros(16, dtype=torch.float32, pin_memory=True)
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    meta_host = torch.zeros(8, dtype=torch.float32, pin_memory=True)
    meta_dev = torch.full((8,), -1.0, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="timed out"):
        c.prepare_signaled(row, flag, 0, 0, 4, 6, None, meta_host, meta_dev, timeout_ms=50)
    row[:4] = torch.tensor([5.0, 1.0, 2.0, 3.0])
    row[4:8] = torch.tensor([0.5, 0.25, 0.125, 0.125])
    flag[0] = 1
    assert c.prepare_signaled(row, flag, 0, 0, 4, 6, None, meta_host, meta_dev) == 1
    torch.cuda.synchronize()
    slots = meta_dev[:4].cpu().long().tolist()
    assert meta_dev[4:].cpu().tolist() == [0.5, 0.25, 0.125, 0.125]
    got = _rows(c, slots)
    for j, key in enumerate([5, 1, 2, 3]):
        assert torch.equal(got[j], st.host[key]), key
    flag[0] = 2
    row[0] = 6.0  # outside [0, n_ids)
    with pytest.raises(RuntimeError):
        c.prepare_signaled(row, flag, 1, 0, 4, 6, None, meta_host, meta_dev)
    c.free()
