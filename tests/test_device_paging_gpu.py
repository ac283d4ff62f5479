"""Device paging: the decode layer's cache step (cache_core.py:30-106: clock, notes, ensure)
and the paging of its misses run on the GPU (k_lru_step / k_route_lru + k_page_list),
checked step by step against the reference core (oracle/cache_core_ref.py) on the same key
streams -- LRU, WSA and static policies, the whole state (owners, ticks, scores, the
frequency table in insertion order, inc) -- including graph replays, repeated ids, a static
region, the 1e100 renormalisation, bad ids and a request with no evictable slot."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.cache_core_ref import RefCore
from wisp.cache import ExpertCache
from wisp.store import ExpertStore

pytestmark = pytest.mark.gpu
H, I, G = 256, 128, 128
N = H * I
DEV = "cuda"


def _store(L, E, seed=0):
    rng = np.random.default_rng(seed)
    st = ExpertStore(L, E, N, 4, G)
    for key in range(L * E):
        w = (rng.standard_normal(3 * N) * 0.02).astype(np.float32)
        st.host[key].copy_(torch.from_numpy(O.quantize(w, 4, G)))
    return st


@pytest.fixture(scope="module")
def store():
    return _store(3, 24, seed=5)


def _check_state(c, ref, st):
    core = c.core  # ends device paging: the host core now holds the device state
    assert core.key2slot == ref.where
    assert core.stats == ref.counts
    assert [int(v) for v in core.slot_key] == ref.owner
    assert [float(v) for v in core.last] == ref.t_last
    assert [float(v) for v in core.score] == ref.f_score
    assert list(core.freq.items()) == list(ref.acc.items())  # values and insertion order
    assert core.inc == ref.unit
    assert core.free == list(ref.stack)
    assert core.tick == ref.now
    for key, s in ref.where.items():  # every resident slot holds its store row
        assert torch.equal(c.gpu[s].cpu(), st.host[key]), (key, s)


def _row(ids, w):
    return torch.tensor(list(map(float, ids)) + list(map(float, w)), dtype=torch.float32, device=DEV)


@pytest.mark.parametrize("nslots,k,use_row,policy", [(10, 4, False, "lru"), (10, 8, True, "lru"),
                                                    (20, 16, False, "lru"), (9, 1, True, "lru"),
                                                    (64, 8, False, "lru"), (10, 4, False, "wsa"),
                                                    (20, 8, True, "wsa"), (12, 6, False, "static")])
def test_device_steps_match_reference_lru(store, nslots, k, use_row, policy):
    E = 24
    c = ExpertCache(store, nslots, policy=policy, copy="kernel")
    ref = RefCore(nslots, policy)
    rng = np.random.default_rng(nslots * 31 + k)
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    c.device_begin()
    assert c.device_paging
    for it in range(60):
        layer = int(rng.integers(0, 3))
        ids = rng.choice(E, size=k, replace=False).astype(np.int64)
        w = rng.random(k).astype(np.float32)
        keys = [layer * E + int(v) for v in ids]
        if use_row:
            c.device_step(_row(ids, w), None, layer * E, E, k, meta)
        else:
            c.device_step(_row(np.zeros(k), w), torch.from_numpy(ids).to(DEV), layer * E, E, k, meta)
        slots, _ = ref.ensure(keys)
        m = meta.cpu()
        assert [int(v) for v in m[:k]] == slots, it
        assert torch.equal(m[k:], torch.from_numpy(w)), it
        if it % 15 == 14:
            c.device_sync()  # state copied back, device paging stays on
            assert c.device_paging
            assert c.core.stats == ref.counts  # (ends device paging)
            c.device_begin()
    _check_state(c, ref, store)
    assert c.n_loads == ref.counts["misses"] and c.bytes_h2d == c.n_loads * store.nbytes
    c.free()


@pytest.mark.parametrize("policy,nslots", [("wsa", 16), ("lru", 16), ("wsa", 1300)])
def test_device_steps_through_the_renormalisation(store, policy, nslots):
    """decay 0.25: inc grows fourfold a step and passes 1e100 at step 167, where every
    frequency, every score and inc are divided by 1e100 (cache_core.py:34-38); steps on both
    sides, with host steps before device paging begins, equal the reference core's, scores
    and the frequency table included. 1,300 slots: the multi-wave form over 72 keys (no
    evictions: the dynamic region never fills)."""
    E, k = 24, 6
    c = ExpertCache(store, nslots, policy=policy, decay=0.25, copy="kernel")
    ref = RefCore(nslots, policy, decay=0.25)
    rng = np.random.default_rng(17)
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    for it in range(5):  # host steps first: keys already in the table when device paging begins
        keys = [int(v) for v in rng.choice(3 * E, size=k, replace=False)]
        assert c.ensure(keys) == ref.ensure(keys)[0], it
    c.device_begin()
    for it in range(220):
        layer = int(rng.integers(0, 3))
        ids = rng.choice(E, size=k, replace=False).astype(np.int64)
        c.device_step(_row(ids, np.ones(k)), None, layer * E, E, k, meta)
        slots, _ = ref.ensure([layer * E + int(v) for v in ids])
        assert [int(v) for v in meta[:k].cpu()] == slots, it
        if it in (150, 175):
            c.device_sync()
            assert c.core.inc == ref.unit, it  # (ends device paging)
            c.device_begin()
    assert ref.unit < 1e100 and ref.now == 225
    _check_state(c, ref, store)
    c.free()


@pytest.mark.parametrize("nslots,n_static", [(1500, 0), (6144, 0), (2100, 40)])
def test_device_steps_past_1024_dynamic_slots(nslots, n_static):
    """Pools of more than 1024 dynamic slots hold the eviction keys in the registers of the
    waves beside the one that routes (the multi-wave form of k_lru_step). k = 16 steps fill
    the pool to 8 free slots, then one step of 16 new keys takes the 8 free slots and evicts
    8, then random steps over 8192 keys mix hits with evicting misses; every step's meta, the
    counters at every sync and the final state match the reference LRU."""
    L, E, n, k = 64, 128, 1024, 16  # 8192 keys of 1632-byte rows
    st = ExpertStore(L, E, n, 4, 128)
    gen = torch.Generator().manual_seed(nslots)
    st.host.copy_(torch.randint(0, 256, tuple(st.host.shape), dtype=torch.uint8, generator=gen))
    pre = list(range(8000, 8000 + n_static))
    c = ExpertCache(st, nslots, n_static=n_static, preload_keys=pre or None, copy="kernel")
    ref = RefCore(nslots, "lru", n_static=n_static)
    if pre:
        ref.preload(pre)
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    rng = np.random.default_rng(nslots + n_static)
    c.device_begin()

    def step(keys, it):
        keys = [int(v) for v in keys]
        layer = keys[0] // E
        ids = np.array([v - layer * E for v in keys], dtype=np.int64)
        assert all(0 <= v < E for v in ids)
        w = rng.random(len(keys)).astype(np.float32)
        c.device_step(_row(ids, w), None, layer * E, E, len(keys), meta)
        m = meta.cpu()
        assert [int(v) for v in m[: len(keys)]] == ref.ensure(keys)[0], it

    fill = nslots - n_static - 8
    for it, k0 in enumerate(range(0, fill, k)):  # keys 0 .. fill-1, at most k of one layer per step
        layer = k0 // E
        hi = min(k0 + k, fill, (layer + 1) * E)
        step(range(k0, hi), it)
    assert ref.counts["evictions"] == 0 and len(ref.stack) == 8
    base = (fill // E + 1) * E  # 16 keys of a layer not used yet: 8 take the free slots, 8 evict
    step(range(base, base + k), "mixed")
    assert ref.counts["evictions"] == 8 and not ref.stack
    for it in range(300):
        layer = int(rng.integers(0, L))
        step(layer * E + rng.choice(E, size=k, replace=False), it)
        if it % 100 == 99:
            c.device_sync()
            assert c.core.stats == ref.counts, it  # (ends device paging)
            c.device_begin()
    assert ref.counts["evictions"] > 600
    _check_state(c, ref, st)
    c.free()


@pytest.mark.parametrize("nslots,n_static,policy", [(12000, 0, "lru"), (20000, 300, "lru"), (26880, 0, "lru"),
                                                    (14000, 200, "wsa")])
def test_device_steps_in_large_pools(nslots, n_static, policy):
    """Pools up to the device step's limit of 26,880 dynamic slots (15 waves of 28 eviction
    keys per thread): filled to 8 free slots, a mixed free/evicting step, then random steps
    over 32,768 keys taken three ways in turn -- the LRU step on the row's ids, the route +
    LRU kernel with forced ids, and a captured graph of the LRU step replayed with new ids --
    each step's meta and the final state equal to the reference LRU's."""
    L, E, n, k = 256, 128, 1024, 16  # 32768 keys of 1632-byte rows
    st = ExpertStore(L, E, n, 4, 128)
    gen = torch.Generator().manual_seed(nslots)
    st.host.copy_(torch.randint(0, 256, tuple(st.host.shape), dtype=torch.uint8, generator=gen))
    pre = list(range(32000, 32000 + n_static))
    c = ExpertCache(st, nslots, policy=policy, n_static=n_static, preload_keys=pre or None, copy="kernel")
    ref = RefCore(nslots, policy, n_static=n_static)
    if pre:
        ref.preload(pre)
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    ids = torch.zeros(k, dtype=torch.int64, device=DEV)
    row = _row(np.zeros(k), np.linspace(0.05, 0.8, k))
    # 48 router logits: the route kernel requests the key -> slot entries of ids below 64, so
    # forced ids of 64 .. 127 take its other path (a read of the entry)
    logits = torch.randn(48, device=DEV).to(torch.bfloat16)
    rng = np.random.default_rng(nslots + n_static)
    c.device_begin()
    c.device_step(row, None, 0, E, 0, meta)  # warm-up launch before capture: changes nothing
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    gbase = 7 * E  # the captured step's layer
    with torch.cuda.graph(g):
        c.device_step(row, ids, gbase, E, k, meta)

    def step(keys, it, how):
        keys = [int(v) for v in keys]
        n_k = len(keys)
        layer = keys[0] // E
        local = np.array([v - layer * E for v in keys], dtype=np.int64)
        assert all(0 <= v < E for v in local)
        if how == "graph":  # the captured step: k keys of layer gbase / E
            assert layer == gbase // E and n_k == k
            ids.copy_(torch.from_numpy(local))
            g.replay()
        elif how == "route":  # every lane's id forced: the router's own choice is replaced
            assert n_k == k
            ids.copy_(torch.from_numpy(local))
            c.device_route_step(logits, k, True, torch.zeros(2 * k, device=DEV), ids, layer * E, E, meta)
        else:
            c.device_step(_row(local, np.ones(n_k)), None, layer * E, E, n_k, meta)
        assert [int(v) for v in meta[:n_k].cpu()] == ref.ensure(keys)[0], (it, how)

    fill = nslots - n_static - 8
    for it, k0 in enumerate(range(0, fill, k)):  # keys 0 .. fill-1, at most k of one layer per step
        layer = k0 // E
        hi = min(k0 + k, fill, (layer + 1) * E)
        step(range(k0, hi), it, "route" if hi - k0 == k and it % 2 else "row")
    assert ref.counts["evictions"] == 0 and len(ref.stack) == 8
    base = (fill // E + 1) * E
    step(range(base, base + k), "mixed", "route")
    assert ref.counts["evictions"] == 8 and not ref.stack
    for it in range(150):
        how = ("row", "route", "graph")[it % 3]
        layer = gbase // E if how == "graph" else int(rng.integers(0, L))
        step(layer * E + rng.choice(E, size=k, replace=False), it, how)
    assert ref.counts["evictions"] > 200
    _check_state(c, ref, st)
    c.free()


def test_route_step_forced_ids_past_the_routers_experts():
    """The route + LRU kernel (one wave, 64 slots) with 32 router logits and forced ids over a
    layer of 160 experts: ids below 64 find their residency among the entries the kernel
    requests at its start, the others read it; every step equals the reference LRU."""
    L, E, n, k, nslots = 2, 160, 1024, 8, 64
    st = ExpertStore(L, E, n, 4, 128)
    gen = torch.Generator().manual_seed(3)
    st.host.copy_(torch.randint(0, 256, tuple(st.host.shape), dtype=torch.uint8, generator=gen))
    c = ExpertCache(st, nslots, copy="kernel")
    ref = RefCore(nslots, "lru")
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    row = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    logits = torch.randn(32, device=DEV).to(torch.bfloat16)
    rng = np.random.default_rng(21)
    c.device_begin()
    for it in range(80):
        layer = it % L
        draw = rng.choice(E, size=k, replace=False).astype(np.int64)
        c.device_route_step(logits, k, True, row, torch.from_numpy(draw).to(DEV), layer * E, E, meta)
        slots, _ = ref.ensure([layer * E + int(v) for v in draw])
        assert [int(v) for v in meta[:k].cpu()] == slots, it
    assert ref.counts["evictions"] > 200
    _check_state(c, ref, st)
    c.free()


def test_repeated_ids_and_hits_in_one_step(store):
    """Forced ids may repeat a key: the reference hands each occurrence of a missing key its
    own slot and keeps the later one in key2slot; the device step does the same. (The pool is
    large enough that no such orphaned slot is evicted: the reference raises when it evicts
    a second slot of one key.)"""
    E, nslots, k = 24, 40, 6
    c = ExpertCache(store, nslots, copy="kernel")
    ref = RefCore(nslots, "lru")
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    row = _row(np.zeros(k), np.ones(k))
    c.device_begin()
    for ids in ([1, 1, 2, 3, 3, 3], [1, 2, 4, 5, 6, 7], [8, 9, 8, 10, 11, 1], [12, 13, 14, 15, 16, 17],
                [2, 2, 2, 2, 2, 2], [18, 19, 20, 21, 22, 23]):
        c.device_step(row, torch.tensor(ids, dtype=torch.int64, device=DEV), 0, E, k, meta)
        slots, _ = ref.ensure(list(ids))
        assert [int(v) for v in meta.cpu()[:k]] == slots, ids
    _check_state(c, ref, store)
    c.free()


def test_static_region_and_host_steps_between(store):
    """A cache with a preloaded static region (never evicted), device steps alternating with
    host-side ensure calls (each ends device paging; the next begin uploads the state)."""
    E, nslots, k, n_static = 24, 14, 4, 4
    pre = [0, 5, 30, 47]
    c = ExpertCache(store, nslots, n_static=n_static, preload_keys=pre, copy="kernel")
    ref = RefCore(nslots, "lru", n_static=n_static)
    ref.preload(pre)
    rng = np.random.default_rng(9)
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    for it in range(40):
        layer = int(rng.integers(0, 3))
        ids = rng.choice(E, size=k, replace=False).astype(np.int64)
        keys = [layer * E + int(v) for v in ids]
        if it % 3 == 2:
            assert c.ensure(keys) == ref.ensure(keys)[0], it
        else:
            c.device_begin()
            c.device_step(_row(ids, np.ones(k)), None, layer * E, E, k, meta)
            assert [int(v) for v in meta.cpu()[:k]] == ref.ensure(keys)[0], it
    _check_state(c, ref, store)
    c.free()


def test_graph_replays_of_device_steps(store):
    """Three layers' paging points captured in one graph and replayed with new ids each time
    (eager work and syncs between the replays); every replay matches the reference LRU."""
    E, nslots, k = 24, 16, 8
    c = ExpertCache(store, nslots, copy="kernel")
    ref = RefCore(nslots, "lru")
    ids = torch.zeros(3, k, dtype=torch.int64, device=DEV)
    row = _row(np.zeros(k), np.linspace(0.1, 0.8, k))
    metas = [torch.zeros(2 * k, dtype=torch.float32, device=DEV) for _ in range(3)]
    c.device_begin()
    c.device_step(row, None, 0, E, 0, metas[0])  # warm-up launch: changes nothing
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for layer in range(3):
            c.device_step(row, ids[layer], layer * E, E, k, metas[layer])
    rng = np.random.default_rng(11)
    for rep in range(12):
        draw = np.stack([rng.choice(E, size=k, replace=False) for _ in range(3)]).astype(np.int64)
        ids.copy_(torch.from_numpy(draw))
        g.replay()
        x = torch.randn(512, 512, device=DEV)
        (x @ x).sum().item()  # eager work and a sync between the replays
        for layer in range(3):
            slots, _ = ref.ensure([layer * E + int(v) for v in draw[layer]])
            assert [int(v) for v in metas[layer].cpu()[:k]] == slots, (rep, layer)
    _check_state(c, ref, store)
    c.free()


def test_captured_steps_stay_valid_across_end_and_begin(store):
    """A graph of device steps captured once keeps working after device paging is ended (host
    steps change the core) and begun again; replayed while it is off it does no step and
    writes slot -1, and the state is unchanged."""
    E, nslots, k = 24, 12, 4
    c = ExpertCache(store, nslots, copy="kernel")
    ref = RefCore(nslots, "lru")
    ids = torch.zeros(k, dtype=torch.int64, device=DEV)
    row = _row(np.zeros(k), np.ones(k))
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    c.device_begin()
    c.device_step(row, None, 0, E, 0, meta)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        c.device_step(row, ids, 24, E, k, meta)
    rng = np.random.default_rng(13)
    for rep in range(6):
        draw = rng.choice(E, size=k, replace=False).astype(np.int64)
        ids.copy_(torch.from_numpy(draw))
        g.replay()
        assert [int(v) for v in meta.cpu()[:k]] == ref.ensure([24 + int(v) for v in draw])[0], rep
        host = [int(v) for v in rng.choice(E, size=k, replace=False)]
        assert c.ensure(host) == ref.ensure(host)[0], rep  # ends device paging
        assert not c.device_paging
        if rep == 3:  # replayed while off: no step
            g.replay()
            assert [int(v) for v in meta.cpu()[:k]] == [-1] * k
            assert c.core.stats == ref.counts
        c.device_begin()
    _check_state(c, ref, store)
    c.free()


@pytest.mark.parametrize("E,k,norm", [(24, 8, True), (24, 4, False), (24, 1, True), (24, 16, True)])
def test_route_step_equals_route_kernel_then_step(store, E, k, norm):
    """The fused route + LRU kernel against wisp_dl_route followed by the LRU step: the same
    row bits, the same meta, and the bookkeeping of the reference LRU, with the router's
    choice and with forced ids."""
    from wisp import kernels

    nslots = 20
    c = ExpertCache(store, nslots, copy="kernel")
    ref = RefCore(nslots, "lru")
    g = torch.Generator(device=DEV).manual_seed(E * 7 + k)
    row_a = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    row_b = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    rng = np.random.default_rng(E + k)
    c.device_begin()
    c.device_route_step(torch.zeros(E, dtype=torch.bfloat16, device=DEV), 0, norm, row_b, None, 0, E, meta)
    for it in range(30):
        layer = it % 3
        logits = torch.randn(E, generator=g, device=DEV).to(torch.bfloat16)
        kernels.dl_route(logits, k, norm, row_a)
        forced = None
        chosen = [int(v) for v in row_a[:k].cpu()]
        if it % 4 == 3:
            forced = torch.from_numpy(rng.choice(E, size=k, replace=False).astype(np.int64)).to(DEV)
        elif it % 4 == 1 and k < E:  # some lanes forced (ids outside the router's choice), the rest -1
            other = [e for e in range(E) if e not in chosen]
            f = [int(other[j]) if j % 2 == 0 and j < len(other) else -1 for j in range(k)]
            forced = torch.tensor(f, dtype=torch.int64, device=DEV)
        c.device_route_step(logits, k, norm, row_b, forced, layer * E, E, meta)
        assert torch.equal(row_a.view(torch.int32), row_b.view(torch.int32)), it
        ids = chosen
        if forced is not None:
            ids = [fv if fv >= 0 else cv for fv, cv in zip(forced.cpu().tolist(), chosen)]
        slots, _ = ref.ensure([layer * E + int(v) for v in ids])
        m = meta.cpu()
        assert [int(v) for v in m[:k]] == slots, it
        assert torch.equal(m[k:], row_a[k:].cpu()), it
    _check_state(c, ref, store)
    c.free()


def test_bad_id_and_no_evictable_slot_are_reported(store):
    E, k = 24, 4
    c = ExpertCache(store, 6, copy="kernel")
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    c.device_begin()
    c.device_step(_row([1, 2, 99, 3], np.ones(k)), None, 0, E, k, meta)  # id 99 >= n_ids
    m = meta.cpu()
    assert int(m[2]) == -1 and all(int(v) >= 0 for v in m[[0, 1, 3]])
    with pytest.raises(RuntimeError, match="outside"):
        c.device_sync()
    c.device_sync()  # reported once
    c.device_end()
    c2 = ExpertCache(store, 6, copy="kernel")
    k = 8  # more keys than slots: the reference raises on the 7th miss; here the step is refused on the host
    meta = torch.zeros(2 * k, dtype=torch.float32, device=DEV)
    c2.device_begin()
    with pytest.raises(RuntimeError, match="no evictable slot"):
        c2.device_step(_row(list(range(8)), np.ones(k)), None, 0, E, k, meta)
    logits = torch.zeros(E, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="no evictable slot"):
        c2.device_route_step(logits, k, True, torch.zeros(2 * k, device=DEV), None, 0, E, meta)
    c2.device_step(_row(list(range(6)), np.ones(6)), None, 0, E, 6, meta)  # k = the dynamic slots: placed
    assert sorted(int(v) for v in meta[:6].cpu()) == list(range(6))
    c2.device_end()
    assert not c2.device_paging and c2.core.stats["misses"] == 6
    c.free()
    c2.free()


def test_device_paging_refusals(store):
    c = ExpertCache(store, 8, copy="dma")
    with pytest.raises(RuntimeError, match="page-kernel"):
        c.device_begin()
    c.free()
    small = ExpertStore(1, 8, 1024, 4, 128)  # more dynamic slots than the device step holds keys for
    c = ExpertCache(small, 26881, copy="kernel")
    with pytest.raises(RuntimeError, match="26880 dynamic slots"):
        c.device_begin()
    c.free()

