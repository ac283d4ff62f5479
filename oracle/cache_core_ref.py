"""CPU restatement of the expert-cache bookkeeping (pure Python, small traces).

TEST INFRASTRUCTURE ONLY: the checker the native core of libwisp_hip.so is compared
against; the product never imports it. It restates wisp/cache_core.py:15-149 of the
reference (imronpuji/wisp-runtime):
  - clock and decayed frequency, renormalised past 1e100 ..... cache_core.py:30-51
  - slot choice: free stack, then first-index minimum of the
    policy's key (last use for lru, decayed frequency otherwise)
    over unprotected dynamic slots .............................. cache_core.py:64-84
  - ensure (hits first, then misses in order), split, admit,
    preload, resized (hottest first, stable) ..................... cache_core.py:54-149
All arithmetic is binary64 (Python floats), in the reference's order.

Pins (tests/test_cache_core.py): the reference's own resize KAT
(tests/test_graphdec.py:132-144), a textbook LRU (OrderedDict) on traces that fit,
the closed form of the decayed frequency sum_i decay^(t - t_i), invariance of
normalised frequencies across the 1e100 renormalisation, and the bookkeeping
invariants of tests/test_paged_moe.py:103-111.
"""

from __future__ import annotations

import math

LRU, WSA, STATIC = "lru", "wsa", "static"


class RefCore:
    def __init__(self, nslots, policy=LRU, decay=0.9995, n_static=0, admit_after=2.0):
        self.nslots, self.policy, self.decay = nslots, policy, decay
        self.n_static, self.admit_after = n_static, admit_after
        self.owner = [-1] * nslots  # slot -> key
        self.t_last = [0.0] * nslots
        self.f_score = [0.0] * nslots
        self.where = {}  # key -> slot
        self.stack = [s for s in range(nslots - 1, n_static - 1, -1)]
        self.now, self.unit = 0, 1.0
        self.acc = {}  # key -> decayed count (insertion ordered)
        self.counts = {"hits": 0, "misses": 0, "evictions": 0, "calls": 0}

    def _acc_get(self, k):
        if k not in self.acc:
            self.acc[k] = 0.0
        return self.acc[k]

    def step(self):
        self.now = self.now + 1
        self.unit = self.unit / self.decay
        if self.unit > 1e100:
            for k in list(self.acc):
                self.acc[k] = self.acc[k] / 1e100
            self.f_score = [v / 1e100 for v in self.f_score]
            self.unit = self.unit / 1e100

    def note(self, keys):
        for k in keys:
            self.acc[k] = self._acc_get(k) + self.unit
            if k in self.where:
                s = self.where[k]
                self.t_last[s] = float(self.now)
                self.f_score[s] = self.acc[k]

    def norm_freq(self, k):
        return self.acc.get(k, 0.0) / self.unit

    def lookup(self, k):
        return self.where.get(k)

    def preload(self, keys):
        assert len(keys) <= self.n_static
        for s, k in enumerate(keys):
            self.owner[s] = k
            self.where[k] = s
        return [(k, s) for s, k in enumerate(keys)]

    def acquire(self, key, protected):
        if self.stack:
            s = self.stack.pop()
        else:
            key_of = self.t_last if self.policy == LRU else self.f_score
            best, s = math.inf, None
            for cand in range(self.n_static, self.nslots):
                v = math.inf if cand in protected else key_of[cand]
                if s is None or v < best:
                    best, s = v, cand
            if s is None or not math.isfinite(best):
                raise RuntimeError("no evictable slot")
            del self.where[self.owner[s]]
            self.counts["evictions"] += 1
        self.owner[s] = key
        self.where[key] = s
        self.t_last[s] = float(self.now)
        self.f_score[s] = self._acc_get(key)
        return s

    def ensure(self, keys):
        self.step()
        self.note(keys)
        self.counts["calls"] += 1
        out = [self.where.get(k) for k in keys]
        prot = {s for s in out if s is not None}
        self.counts["hits"] += sum(s is not None for s in out)
        loads = []
        for i, k in enumerate(keys):
            if out[i] is None:
                s = self.acquire(k, prot)
                out[i] = s
                prot.add(s)
                loads.append((k, s))
                self.counts["misses"] += 1
        return out, loads

    def split(self, keys):
        self.step()
        self.note(keys)
        self.counts["calls"] += 1
        hk = [k for k in keys if k in self.where]
        hs = [self.where[k] for k in hk]
        mk = [k for k in keys if k not in self.where]
        self.counts["hits"] += len(hk)
        self.counts["misses"] += len(mk)
        return hk, hs, mk

    def admit(self, key, protected):
        if key in self.where or self.norm_freq(key) < self.admit_after:
            return None
        try:
            return self.acquire(key, set(protected))
        except RuntimeError:
            return None

    def resized(self, nslots):
        assert self.n_static == 0
        nc = RefCore(nslots, self.policy, self.decay, 0, self.admit_after)
        nc.now, nc.unit = self.now, self.unit
        nc.acc = dict(self.acc)
        nc.counts = dict(self.counts)
        key_of = self.t_last if self.policy == LRU else self.f_score
        live = [s for s in range(self.nslots) if self.owner[s] >= 0]
        live = sorted(live, key=lambda s: -key_of[s])  # stable: ties keep slot order
        kept = live[:nslots]
        for ns, s in enumerate(kept):
            nc.owner[ns] = self.owner[s]
            nc.where[self.owner[s]] = ns
            nc.t_last[ns], nc.f_score[ns] = self.t_last[s], self.f_score[s]
        nc.stack = [s for s in range(nslots - 1, len(kept) - 1, -1)]
        return nc, [(nc.owner[ns], ns) for ns in range(len(kept))]
