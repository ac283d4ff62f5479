"""GPU expert cache: one hipMalloc slot pool, filled from the pinned host store by
hipMemcpyAsync on a side stream. Same interface as the reference's wisp/cache.py
(ExpertCache, cache.py:9-162).

The pool, the side stream, the copy ordering (an event recorded on the compute stream
before the copies, the compute stream waiting on the copies' event afterwards) and the
bookkeeping core are native (libwisp_hip.so); `gpu` is a torch view of the pool
(DLPack), so the decode kernels and graph captures take it like the reference's tensor.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch
import torch.utils.dlpack

from . import _lib
from .cache_core import _POLICIES, CacheCore
from .quant import dequant, dequant_rows


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(list(a), dtype=np.int64).reshape(-1))


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


def _raise(rc: int) -> None:
    """RuntimeError with the library's message, as the reference cache raises (cache_core.py:80)."""
    if rc != 0:
        raise RuntimeError(_lib.lib().wisp_last_error().decode(errors="replace"))


_PyCapsule_New = ctypes.pythonapi.PyCapsule_New
_PyCapsule_New.restype = ctypes.py_object
_PyCapsule_New.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


class ExpertCache:
    def __init__(
        self,
        store,
        nslots,
        device="cuda",
        policy="lru",
        decay=0.9995,
        n_static=0,
        admit_after=2.0,
        preload_keys=None,
        cpu_store=None,
        decode_on_load=False,
        staging_rows=8,
        copy="auto",
    ):
        """copy: how misses cross PCIe. "dma" = one hipMemcpyAsync per expert row on the side
        stream (the DMA engines); "kernel" = one page kernel per batch of rows on the side
        stream, the GPU reading the pinned store directly (needs a pinned store; faster for
        several rows at once); "auto" = "kernel" when the store allows it, else "dma"."""
        assert policy in _POLICIES, policy
        assert copy in ("dma", "kernel", "auto"), copy
        self.store, self.device = store, torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        # decode_on_load: experts cross PCIe quantized, are dequantized once on arrival and
        # kept as bf16 (cache.py:25-27)
        self.decode_on_load = bool(decode_on_load) and store.bits < 16
        self.cpu_store = cpu_store
        self.nslots, self.n_static = nslots, n_static
        self.slot_bytes = 3 * store.n * 2 if self.decode_on_load else store.nbytes
        host = store.host
        assert host.dtype == torch.uint8 and host.dim() == 2 and host.is_contiguous() and not host.is_cuda
        core = CacheCore(nslots, policy, decay, n_static, admit_after)
        h = ctypes.c_void_p()
        _lib.check(
            _lib.lib().wisp_cache_create(
                core._h, self.slot_bytes, ctypes.c_void_p(host.data_ptr()), host.shape[0], host.shape[1],
                store.bits, store.n, store.group, int(self.decode_on_load), staging_rows, self.device.index,
                ctypes.byref(h),
            ),
            "ExpertCache",
        )
        core._release()  # the native cache owns the core now
        self._h = h
        self._host = host  # keep the store rows alive as long as the cache
        self.copy = "dma"
        if copy != "dma" and not self.decode_on_load:
            rc = _lib.lib().wisp_cache_set_copy_mode(self._h, 1)
            if rc == 0:
                self.copy = "kernel"
            elif copy == "kernel":
                raise RuntimeError(_lib.lib().wisp_last_error().decode())
        elif copy == "kernel":
            raise RuntimeError("copy='kernel' does not stage decode-on-load rows")
        self._view()
        self.copy_stream = torch.cuda.ExternalStream(_lib.lib().wisp_cache_copy_stream(self._h), device=self.device)
        if n_static:
            assert preload_keys is not None and len(preload_keys) <= n_static
            self._issue(self.core.preload(list(preload_keys)))
            self.sync_all()

    def _view(self):
        m = _lib.lib().wisp_cache_pool_dlpack(self._h)
        if not m:
            raise RuntimeError("ExpertCache: could not create the pool view")
        try:
            cap = _PyCapsule_New(m, b"dltensor", None)
            self.gpu = torch.utils.dlpack.from_dlpack(cap)
        except Exception:
            _lib.lib().wisp_cache_pool_dlpack_free(m)
            raise

    @property
    def core(self) -> CacheCore:
        """The bookkeeping core (owned by the native cache); ends device paging first, so the
        core holds the current state."""
        self.device_end()
        return CacheCore._wrap(_lib.lib().wisp_cache_core(self._h), owned=False)

    @property
    def bytes_h2d(self) -> int:
        self.device_sync()
        b, n = ctypes.c_int64(), ctypes.c_int64()
        _lib.lib().wisp_cache_counters(self._h, ctypes.byref(b), ctypes.byref(n))
        return b.value

    @property
    def n_loads(self) -> int:
        self.device_sync()
        b, n = ctypes.c_int64(), ctypes.c_int64()
        _lib.lib().wisp_cache_counters(self._h, ctypes.byref(b), ctypes.byref(n))
        return n.value

    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    # ---- device paging ----------------------------------------------------
    # The cache step of a decode layer on the GPU (k_lru_step + the page kernel; any
    # policy), so a captured decode step has no host decision per layer. While it is on,
    # the core's state lives in device memory; every host-side operation below ends it first.
    @property
    def device_paging(self) -> bool:
        return bool(self._h) and bool(_lib.lib().wisp_cache_device_active(self._h))

    def device_begin(self):
        """Copy the core's state to the device (any policy, copy="kernel", at most 26880
        dynamic slots); RuntimeError if this cache cannot page on the device."""
        _raise(_lib.lib().wisp_cache_device_begin(self._h, self._stream()))

    def device_step(self, row: torch.Tensor, ids, key_base: int, n_ids: int, k: int, meta: torch.Tensor):
        """Queue one layer's paging point on the current stream (capturable): keys = key_base +
        id for the route row's ids (float32 row [ids | weights] on the device), or for `ids`
        (int64 [k] on the device; a negative entry keeps the row's id) if given; meta [2k] =
        [slots | weights]; misses paged.
        k = 0: a warm-up launch of both kernels that changes nothing."""
        assert row.dtype == torch.float32 and row.is_cuda and row.numel() >= 2 * k
        assert meta.dtype == torch.float32 and meta.is_cuda and meta.numel() >= 2 * k
        idp = None
        if ids is not None:
            assert ids.dtype == torch.int64 and ids.is_cuda and ids.is_contiguous() and ids.numel() >= k
            idp = ctypes.c_void_p(ids.data_ptr())
        _raise(_lib.lib().wisp_cache_device_step(self._h, ctypes.c_void_p(row.data_ptr()), idp, key_base, n_ids, k,
                                                 ctypes.c_void_p(meta.data_ptr()), self._stream()))

    def device_route_step(self, logits: torch.Tensor, k: int, norm_topk: bool, row: torch.Tensor, ids,
                          key_base: int, n_ids: int, meta: torch.Tensor):
        """The route kernel (softmax of the bf16 router logits [E], top-k, renormalised if
        norm_topk, bf16 weights into row [ids | weights]) and device_step on its choice in
        one launch, then the page kernel. ids (int64 [k] on the device) replace the chosen
        expert ids where they are >= 0."""
        assert logits.dtype == torch.bfloat16 and logits.is_cuda and logits.is_contiguous()
        assert row.dtype == torch.float32 and row.is_cuda and row.numel() >= 2 * k
        assert meta.dtype == torch.float32 and meta.is_cuda and meta.numel() >= 2 * k
        idp = None
        if ids is not None:
            assert ids.dtype == torch.int64 and ids.is_cuda and ids.is_contiguous() and ids.numel() >= k
            idp = ctypes.c_void_p(ids.data_ptr())
        _raise(_lib.lib().wisp_cache_device_route_step(
            self._h, ctypes.c_void_p(logits.data_ptr()), logits.numel(), k, int(bool(norm_topk)),
            ctypes.c_void_p(row.data_ptr()), idp, key_base, n_ids, ctypes.c_void_p(meta.data_ptr()), self._stream()))

    def device_sync(self):
        """Wait for the current stream and copy the device state into the core (stays on)."""
        if self.device_paging:
            _raise(_lib.lib().wisp_cache_device_sync(self._h, self._stream()))

    def device_end(self):
        """device_sync, then device paging off."""
        if self.device_paging:
            _raise(_lib.lib().wisp_cache_device_end(self._h, self._stream()))

    # ---- copies ---------------------------------------------------------
    def _issue(self, pairs):
        """Async host->GPU copies of [(key, slot)] on the side stream, ordered after queued compute."""
        if not pairs:
            return
        self.device_end()
        k = _i64(p[0] for p in pairs)
        s = _i64(p[1] for p in pairs)
        _lib.check(_lib.lib().wisp_cache_issue(self._h, _p(k), _p(s), k.size, self._stream()), "ExpertCache._issue")

    def sync_compute(self):
        """Make the current compute stream wait for all issued copies."""
        _lib.check(_lib.lib().wisp_cache_sync_compute(self._h, self._stream()), "sync_compute")

    def sync_all(self):
        torch.cuda.synchronize(self.device)

    # ---- policies -------------------------------------------------------
    def ensure(self, keys):
        self.device_end()
        k = _i64(keys)
        slots = np.empty(max(k.size, 1), np.int64)
        rc = _lib.lib().wisp_cache_ensure(self._h, _p(k), k.size, _p(slots), self._stream())
        if rc != 0:
            raise RuntimeError(_lib.lib().wisp_last_error().decode())
        return [int(v) for v in slots[: k.size]]

    def prepare_layer(self, keys, weights, meta_host: torch.Tensor, meta_dev: torch.Tensor):
        """One layer's host step of the graph decoder (graphdec.py:216-231) in one native call:
        ensure `keys`, write [slots | weights] into meta_host (pinned float32 [2k]) and copy it
        to meta_dev on the current stream. Returns the slots."""
        self.device_end()
        k = _i64(keys)
        w = np.ascontiguousarray(np.asarray(weights, dtype=np.float32).reshape(-1))
        assert w.size == k.size and meta_host.numel() >= 2 * k.size and meta_dev.numel() >= 2 * k.size
        slots = np.empty(max(k.size, 1), np.int64)
        rc = _lib.lib().wisp_cache_prepare_layer(
            self._h, _p(k), _p(w), k.size, ctypes.c_void_p(meta_host.data_ptr()),
            ctypes.c_void_p(meta_dev.data_ptr()), _p(slots), self._stream(),
        )
        if rc != 0:
            raise RuntimeError(_lib.lib().wisp_last_error().decode())
        return [int(v) for v in slots[: k.size]]

    def prepare_row(self, row_dev: torch.Tensor, row_host: torch.Tensor, key_base: int, k: int, n_ids: int, ids,
                    meta_host: torch.Tensor, meta_dev: torch.Tensor):
        """prepare_layer with the router row read back natively: row_dev float32 [>= 2k]
        (device) = [expert ids | weights] is copied into the pinned row_host and waited for;
        keys = key_base + id (every id in [0, n_ids)), with `ids` (int64 numpy [k]) replacing
        the row's ids if given."""
        assert row_dev.dtype == torch.float32 and row_host.dtype == torch.float32 and row_host.numel() >= 2 * k
        self.device_end()
        assert meta_host.numel() >= 2 * k and meta_dev.numel() >= 2 * k
        idp = None
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int64)
            assert ids.size == k
            idp = _p(ids)
        rc = _lib.lib().wisp_cache_prepare_row(
            self._h, ctypes.c_void_p(row_dev.data_ptr()), ctypes.c_void_p(row_host.data_ptr()), k, key_base, n_ids, idp,
            ctypes.c_void_p(meta_host.data_ptr()), ctypes.c_void_p(meta_dev.data_ptr()), None, self._stream(),
        )
        if rc != 0:
            raise RuntimeError(_lib.lib().wisp_last_error().decode())

    def prepare_signaled(self, row_host: torch.Tensor, flag_host: torch.Tensor, flag_before: int, key_base: int,
                         k: int, n_ids: int, ids, meta_host: torch.Tensor, meta_dev: torch.Tensor,
                         timeout_ms: int = 10000) -> int:
        """prepare_row for a row the route kernel writes into the pinned row_host itself: wait
        until flag_host moves from flag_before, then ensure / copy / meta. Returns the flag."""
        assert row_host.is_pinned() and flag_host.is_pinned() and row_host.numel() >= 2 * k
        self.device_end()
        idp = None
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int64)
            assert ids.size == k
            idp = _p(ids)
        after = ctypes.c_uint32()
        rc = _lib.lib().wisp_cache_prepare_signaled(
            self._h, ctypes.c_void_p(row_host.data_ptr()), ctypes.c_void_p(flag_host.data_ptr()),
            flag_before & 0xFFFFFFFF, ctypes.byref(after), timeout_ms, k, key_base, n_ids, idp,
            ctypes.c_void_p(meta_host.data_ptr()), ctypes.c_void_p(meta_dev.data_ptr()), self._stream(),
        )
        if rc != 0:
            raise RuntimeError(_lib.lib().wisp_last_error().decode())
        return after.value

    def split(self, keys):
        return self.core.split(keys)

    def admit_async(self, miss_keys, protected_slots):
        core, prot, pairs = self.core, list(protected_slots), []
        for k in miss_keys:
            s = core.admit(k, prot)
            if s is not None:
                prot.append(s)
                pairs.append((k, s))
        self._issue(pairs)  # not waited on here; the next ensure()/sync_compute() will
        return len(pairs)

    def prefetch(self, keys, protected_slots):
        core, prot, pairs = self.core, list(protected_slots), []
        for k in keys:
            if core.lookup(k) is not None:
                continue
            try:
                s = core.acquire(k, prot)
            except RuntimeError:
                break
            prot.append(s)
            pairs.append((k, s))
        self._issue(pairs)
        return len(pairs)

    # ---- weights --------------------------------------------------------
    def weights_batched(self, idx):
        """idx: LongTensor of slots on the GPU -> [k, 3, n] bf16 (gather + dequant in one kernel)."""
        st = self.store
        if st.bits == 16 or self.decode_on_load:
            return self.gpu.index_select(0, idx).view(torch.bfloat16).view(len(idx), 3, st.n)
        return dequant_rows(self.gpu, idx, st.n, st.bits, st.group)

    def weights(self, slots):
        """List of [3, n] bf16 tensors on the GPU for the given slots."""
        st = self.store
        if st.bits == 16 or self.decode_on_load:
            return [self.gpu[s].view(torch.bfloat16).view(3, st.n) for s in slots]
        idx = torch.as_tensor(slots, device=self.device)
        return list(dequant_rows(self.gpu, idx, st.n, st.bits, st.group).unbind(0))

    def cpu_weights(self, key):
        """[3, n] bf16 on the host for store row `key` (dequantized by the GPU kernel)."""
        st = self.cpu_store if self.cpu_store is not None else self.store
        b = st.host[key]
        if st.bits == 16:
            return b.view(torch.bfloat16).view(3, st.n)
        return dequant(b[None].to(self.device), st.n, st.bits, st.group)[0].cpu()

    def resize(self, nslots):
        """Grow/shrink the slot pool in place, keeping the hottest experts. The old pool is
        released before the new one is allocated (views of it still held elsewhere keep it
        alive until they are dropped); the kept experts are re-copied from the host store."""
        assert not self.decode_on_load
        if nslots == self.nslots:
            return
        self.device_end()
        torch.cuda.synchronize(self.device)
        self.gpu = None
        _lib.check(_lib.lib().wisp_cache_resize(self._h, nslots), "ExpertCache.resize")
        self.nslots = nslots
        self._view()

    def free(self):
        """Release the pool (views still held elsewhere keep their memory until dropped)."""
        if getattr(self, "_h", None):
            self.gpu = None
            _lib.lib().wisp_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
