"""Expert-cache bookkeeping: pins of the CPU restatement (oracle/cache_core_ref.py), then
the native core (libwisp_hip.so, host code) against it on random traces. CPU only."""

from collections import OrderedDict

import numpy as np
import pytest

from oracle.cache_core_ref import RefCore
from wisp.cache_core import CacheCore


# ---------------------------------------------------------------- oracle pins
def _resize_kat(make):
    """The reference's own KAT (tests/test_graphdec.py:132-144)."""
    c = make(6, "lru")
    for keys in ([1, 2], [3, 4], [5, 6], [1, 3]):
        c.ensure(keys)
    nc, loads = c.resized(3)
    assert sorted(k for k, _ in loads) in ([1, 3, 6], [1, 3, 5])
    assert all(nc.lookup(k) == s for k, s in loads)
    nc2, loads2 = nc.resized(8)
    assert len(loads2) == 3
    slots, new = nc2.ensure([1, 9])
    assert len(new) == 1 and new[0][0] == 9
    return nc, nc2


def test_oracle_resize_kat():
    nc, nc2 = _resize_kat(RefCore)
    assert len(nc.stack) == 0 and len(nc2.stack) == 4  # 5 free after resized(8), one taken by key 9


def test_oracle_lru_matches_textbook_lru():
    """Without protection conflicts (one key per call) the lru policy is textbook LRU."""
    rng = np.random.default_rng(0)
    for nslots in (1, 3, 8):
        c = RefCore(nslots, "lru")
        od = OrderedDict()
        for _ in range(400):
            k = int(rng.integers(0, 12))
            _, loads = c.ensure([k])
            if k in od:
                od.move_to_end(k)
                assert loads == []
            else:
                if len(od) == nslots:
                    od.popitem(last=False)
                od[k] = True
                assert [kk for kk, _ in loads] == [k]
            assert set(c.where) == set(od)


def test_oracle_decayed_frequency_closed_form():
    decay = 0.9
    c = RefCore(4, "wsa", decay)
    seen = {}
    for t in range(1, 60):
        keys = [t % 5, 5 + (t * 3) % 7]  # distinct keys per call, as routed experts are
        c.ensure(keys)
        for k in keys:
            seen.setdefault(k, []).append(t)
    for k, ts in seen.items():
        closed = sum(decay ** (c.now - ti) for ti in ts)
        assert c.norm_freq(k) == pytest.approx(closed, rel=1e-12)


def test_oracle_renormalisation_invariance():
    # decay 0.5 doubles the unit every step: past 1e100 after ~333 steps
    a = RefCore(4, "wsa", 0.5)
    for t in range(400):
        a.ensure([t % 3])
    assert a.unit < 1e100
    for k in range(3):
        closed = sum(0.5 ** (a.now - t) for t in range(1, a.now + 1) if (t - 1) % 3 == k)
        assert a.norm_freq(k) == pytest.approx(closed, rel=1e-12)


def test_oracle_bookkeeping_invariants_and_protection():
    rng = np.random.default_rng(1)
    c = RefCore(6, "lru")
    for _ in range(300):
        keys = [int(v) for v in rng.choice(20, size=4, replace=False)]
        slots, loads = c.ensure(keys)
        assert len(set(slots)) == len(slots)  # one call never hands a slot out twice
        assert all(c.where[k] == s for k, s in zip(keys, slots))
        assert len(c.where) <= 6
        assert set(c.where.values()) == {s for s in range(6) if c.owner[s] >= 0}
    with pytest.raises(RuntimeError):
        RefCore(2, "lru").ensure([1, 2, 3])  # more keys than slots: nothing evictable


# ---------------------------------------------------------------- native core vs oracle
def _same(nat: CacheCore, ref: RefCore):
    assert nat.tick == ref.now
    assert nat.inc == ref.unit
    assert nat.stats == ref.counts
    assert nat.free == ref.stack
    assert nat.slot_key.tolist() == ref.owner
    assert nat.last.tolist() == ref.t_last
    assert nat.score.tolist() == ref.f_score
    assert nat.key2slot == ref.where
    assert nat.freq == ref.acc


def test_native_resize_kat():
    nc, nc2 = _resize_kat(CacheCore)
    assert len(nc.free) == 0 and len(nc2.free) == 4


@pytest.mark.parametrize("policy,n_static,decay", [("lru", 0, 0.9995), ("wsa", 0, 0.99), ("wsa", 0, 0.5),
                                                   ("static", 3, 0.9), ("lru", 2, 0.9995)])
def test_native_matches_oracle_on_random_traces(policy, n_static, decay):
    rng = np.random.default_rng(hash((policy, n_static, decay)) % 2**32)
    nslots, nkeys, k = 10, 40, 3
    nat = CacheCore(nslots, policy, decay, n_static, admit_after=1.5)
    ref = RefCore(nslots, policy, decay, n_static, admit_after=1.5)
    if n_static:
        pin = [int(v) for v in rng.choice(nkeys, size=n_static, replace=False)]
        assert nat.preload(pin) == ref.preload(pin)
    for it in range(600):
        op = rng.random()
        keys = [int(v) for v in rng.choice(nkeys, size=k, replace=False)]
        if op < 0.6:
            assert nat.ensure(keys) == ref.ensure(keys)
        elif op < 0.8:
            assert nat.split(keys) == ref.split(keys)
        elif op < 0.9:
            prot = [int(v) for v in rng.choice(nslots, size=2, replace=False)]
            assert nat.admit(keys[0], prot) == ref.admit(keys[0], set(prot))
        elif ref.lookup(keys[0]) is None:  # acquire is only ever called for a non-resident key
            prot = [int(v) for v in rng.choice(nslots, size=2, replace=False)]
            try:
                r = ref.acquire(keys[0], set(prot))
            except RuntimeError:
                r = None
            if r is None:
                with pytest.raises(RuntimeError):
                    nat.acquire(keys[0], prot)
            else:
                assert nat.acquire(keys[0], prot) == r
        assert nat.norm_freq(keys[1]) == ref.norm_freq(keys[1])
        if it % 50 == 0:
            _same(nat, ref)
    _same(nat, ref)
    if n_static == 0:
        for size in (4, 16):
            n2, l2 = nat.resized(size)
            r2, rl2 = ref.resized(size)
            assert l2 == rl2
            _same(n2, r2)
            for _ in range(50):
                keys = [int(v) for v in rng.choice(nkeys, size=k, replace=False)]
                assert n2.ensure(keys) == r2.ensure(keys)
            _same(n2, r2)


def test_native_errors_match_reference_behaviour():
    c = CacheCore(2, "lru")
    with pytest.raises(RuntimeError, match="no evictable slot"):
        c.ensure([1, 2, 3])
    with pytest.raises(AssertionError):
        CacheCore(4, "fifo")
    with pytest.raises(ValueError):
        CacheCore(4, "lru", n_static=2).resized(3)  # resize with a static region
    s = CacheCore(4, "static", n_static=2)
    with pytest.raises(ValueError):
        s.preload([1, 2, 3])
