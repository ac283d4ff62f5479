"""Expert-cache bookkeeping, the same interface as the reference's wisp/cache_core.py.

Keys are ints (layer * n_experts + expert). Slots [0, n_static) hold a fixed 'static'
resident set; slots [n_static, nslots) are managed by the policy:
  lru    : evict the least recently used
  wsa    : evict the lowest exponentially decayed access frequency
  static : (dynamic region, if any) as wsa
The state and the decisions live in the native core of libwisp_hip.so (host code, no
GPU needed); this class is its Python face. Attributes that the reference exposes as
containers (slot_key, last, score, free, key2slot, freq, stats) are snapshots here.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

_POLICIES = {"lru": 0, "wsa": 1, "static": 2}
_NAMES = {v: k for k, v in _POLICIES.items()}


def _arr(keys) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(list(keys), dtype=np.int64).reshape(-1))


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


class CacheCore:
    """cache_core.py:15-149."""

    def __init__(self, nslots, policy="lru", decay=0.9995, n_static=0, admit_after=2.0, _handle=None):
        assert policy in _POLICIES, policy
        if _handle is None:
            h = ctypes.c_void_p()
            _lib.check(
                _lib.lib().wisp_core_create(nslots, _POLICIES[policy], float(decay), n_static, float(admit_after),
                                            ctypes.byref(h)),
                "CacheCore",
            )
            _handle = h
        self._h = _handle
        self._owned = True

    @classmethod
    def _wrap(cls, handle, owned: bool) -> "CacheCore":
        c = cls.__new__(cls)
        c._h = ctypes.c_void_p(handle) if not isinstance(handle, ctypes.c_void_p) else handle
        c._owned = owned
        return c

    def _release(self):
        """Stop owning the native core (its new owner frees it)."""
        self._owned = False

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            try:
                _lib.lib().wisp_core_destroy(self._h)
            except Exception:
                pass
            self._h = None

    # -- state -----------------------------------------------------------
    def _state(self):
        s = (ctypes.c_int64 * 11)()
        d = (ctypes.c_double * 3)()
        _lib.lib().wisp_core_state(self._h, s, d)
        return list(s), list(d)

    @property
    def nslots(self) -> int:
        return self._state()[0][0]

    @property
    def policy(self) -> str:
        return _NAMES[self._state()[0][1]]

    @property
    def n_static(self) -> int:
        return self._state()[0][2]

    @property
    def tick(self) -> int:
        return self._state()[0][3]

    @property
    def decay(self) -> float:
        return self._state()[1][0]

    @property
    def admit_after(self) -> float:
        return self._state()[1][1]

    @property
    def inc(self) -> float:
        return self._state()[1][2]

    @property
    def stats(self) -> dict:
        s = self._state()[0]
        return dict(hits=s[4], misses=s[5], evictions=s[6], calls=s[7])

    def _arrays(self):
        s, _ = self._state()
        n, nfree, nfreq = s[0], s[8], s[10]
        slot_key = np.empty(n, np.int64)
        last = np.empty(n, np.float64)
        score = np.empty(n, np.float64)
        free = np.empty(max(nfree, 1), np.int64)
        fk = np.empty(max(nfreq, 1), np.int64)
        fv = np.empty(max(nfreq, 1), np.float64)
        _lib.lib().wisp_core_arrays(self._h, _p(slot_key), _p(last), _p(score), _p(free), _p(fk), _p(fv))
        return slot_key, last, score, free[:nfree], fk[:nfreq], fv[:nfreq]

    @property
    def slot_key(self) -> np.ndarray:
        return self._arrays()[0]

    @property
    def last(self) -> np.ndarray:
        return self._arrays()[1]

    @property
    def score(self) -> np.ndarray:
        return self._arrays()[2]

    @property
    def free(self) -> list:
        return [int(v) for v in self._arrays()[3]]

    @property
    def key2slot(self) -> dict:
        sk = self._arrays()[0]
        return {int(k): s for s, k in enumerate(sk) if k >= 0}

    @property
    def freq(self) -> dict:
        _, _, _, _, fk, fv = self._arrays()
        return {int(k): float(v) for k, v in zip(fk, fv)}

    # -- clock / frequency ---------------------------------------------
    def step(self):
        _lib.lib().wisp_core_step(self._h)

    def note(self, keys):
        a = _arr(keys)
        _lib.lib().wisp_core_note(self._h, _p(a), a.size)

    def norm_freq(self, k):
        return _lib.lib().wisp_core_norm_freq(self._h, int(k))

    def should_admit(self, k):
        return self.norm_freq(k) >= self.admit_after

    # -- residency -------------------------------------------------------
    def lookup(self, k):
        s = _lib.lib().wisp_core_lookup(self._h, int(k))
        return None if s < 0 else int(s)

    def preload(self, keys):
        a = _arr(keys)
        _lib.check(_lib.lib().wisp_core_preload(self._h, _p(a), a.size), "preload")
        return [(int(k), s) for s, k in enumerate(a)]

    def acquire(self, key, protected):
        p = _arr(protected)
        s = ctypes.c_int64()
        rc = _lib.lib().wisp_core_acquire(self._h, int(key), _p(p), p.size, ctypes.byref(s))
        if rc != 0:
            raise RuntimeError(_lib.lib().wisp_last_error().decode())
        return int(s.value)

    # -- high level ------------------------------------------------------
    def ensure(self, keys):
        """Make every key resident. Returns (slots aligned with keys, [(key, slot)] to load)."""
        a = _arr(keys)
        n = a.size
        slots = np.empty(max(n, 1), np.int64)
        lk = np.empty(max(n, 1), np.int64)
        ls = np.empty(max(n, 1), np.int64)
        nl = ctypes.c_int64()
        rc = _lib.lib().wisp_core_ensure(self._h, _p(a), n, _p(slots), _p(lk), _p(ls), ctypes.byref(nl))
        if rc != 0:
            raise RuntimeError(_lib.lib().wisp_last_error().decode())
        return [int(s) for s in slots[:n]], [(int(k), int(s)) for k, s in zip(lk[: nl.value], ls[: nl.value])]

    def split(self, keys):
        """Return (hit_keys, hit_slots, miss_keys); nothing is loaded."""
        a = _arr(keys)
        n = a.size
        hk, hs, mk = (np.empty(max(n, 1), np.int64) for _ in range(3))
        nh, nm = ctypes.c_int64(), ctypes.c_int64()
        _lib.lib().wisp_core_split(self._h, _p(a), n, _p(hk), _p(hs), ctypes.byref(nh), _p(mk), ctypes.byref(nm))
        return ([int(v) for v in hk[: nh.value]], [int(v) for v in hs[: nh.value]], [int(v) for v in mk[: nm.value]])

    def admit(self, key, protected):
        """Bring a key in for future use. Returns its slot, or None if not worth it / impossible."""
        p = _arr(protected)
        s = _lib.lib().wisp_core_admit(self._h, int(key), _p(p), p.size)
        return None if s < 0 else int(s)

    def resized(self, nslots):
        """New core with `nslots` slots keeping the hottest resident keys.
        Returns (core, [(key, new_slot)]) -- the caller copies those keys into the new pool."""
        h = ctypes.c_void_p()
        keys = np.empty(max(nslots, 1), np.int64)
        slots = np.empty(max(nslots, 1), np.int64)
        n = ctypes.c_int64()
        _lib.check(
            _lib.lib().wisp_core_resized(self._h, nslots, ctypes.byref(h), _p(keys), _p(slots), ctypes.byref(n)),
            "resized",
        )
        return CacheCore._wrap(h, owned=True), [(int(k), int(s)) for k, s in zip(keys[: n.value], slots[: n.value])]
