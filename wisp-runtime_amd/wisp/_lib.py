"""Loader for libwisp_hip.so, the gfx950 HIP library of this package.

torch is imported first on purpose: the library then binds to the HIP runtime
torch already loaded (both carry the SONAME libamdhip64.so.7), so streams and
device pointers from torch are valid in the library. There is no CPU or
eager-PyTorch fallback: if the library is missing, every GPU entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libwisp_hip.so")
ABI_VERSION = 2

WISP_OK, WISP_EINVAL, WISP_EALIGN = 0, -1, -2
WISP_DT_BF16, WISP_DT_F16, WISP_DT_F32 = 0, 1, 2
WISP_MAX_K = 8192
WISP_NOALLOC_MAX_ACT = 262144

_i64, _i32, _vp, _f64 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_double

# name -> (restype, argtypes); mirrors include/wisp_hip.h
SIGNATURES = {
    "wisp_abi_version": (_i32, []),
    "wisp_last_error": (ctypes.c_char_p, []),
    "wisp_expert_nbytes": (_i64, [_i64, _i32, _i64]),
    "wisp_act_bytes": (_i64, [_i32, _i64]),
    "wisp_quantize": (_i32, [_vp, _i32, _i64, _i32, _i64, _vp, _vp]),
    "wisp_pack": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "wisp_unpack": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "wisp_dequant": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _i32, _i64, _vp, _vp]),
    "wisp_moe_gate_up": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp, _i32, _i64, _i64, _i32, _i64, _vp, _vp]),
    "wisp_moe_down_sum": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp, _i64, _i64, _i32, _i64, _vp, _i32, _vp]),
    "wisp_moe_down": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp, _i64, _i64, _i32, _i64, _vp, _vp]),
    "wisp_moe_decode": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp, _i32, _i64, _i64, _i32, _i64, _vp, _vp, _i32, _vp]),
    "wisp_moe_decode_noalloc": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp, _i32, _i64, _i64, _i32, _i64, _vp, _i32, _vp]),
    "wisp_rope_decode": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "wisp_attn_ws_bytes": (_i64, [_i32, _i32, _i32]),
    "wisp_attn_decode": (_i32, [_vp, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, ctypes.c_float, _vp, _vp, _vp]),
    "wisp_attn_decode_qk": (_i32, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _i64, _i32,
                                   ctypes.c_float, _vp, _vp, _vp]),
    "wisp_prefill_ws_bytes": (_i64, [_i64, _i64, _i64]),
    "wisp_moe_prefill": (_i32, [_vp, _i64, _i64, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _i64, _i64,
                                _i32, _i64, _vp, _vp, _vp, _vp]),
    "wisp_mxfp4_to_bf16": (_i32, [_vp, _vp, _i64, _vp, _vp]),
    "wisp_dl_gemv": (_i32, [_vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp,
                            _vp, _vp]),
    "wisp_dl_qk_rope": (_i32, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _i64, _vp,
                               _vp]),
    "wisp_dl_route": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "wisp_gptoss_ws_bytes": (_i64, [_i32, _i64, _i64]),
    "wisp_gptoss_decode": (_i32, [_vp, _i64, _i64, _vp, _i32, _i64, _i64, _i32, _i64, _vp, _vp, _vp, _i64,
                                  ctypes.c_float, ctypes.c_float, _vp, _vp, _vp]),
    "wisp_core_create": (_i32, [_i64, _i32, _f64, _i64, _f64, _vp]),
    "wisp_core_destroy": (None, [_vp]),
    "wisp_core_step": (None, [_vp]),
    "wisp_core_note": (None, [_vp, _vp, _i64]),
    "wisp_core_norm_freq": (_f64, [_vp, _i64]),
    "wisp_core_lookup": (_i64, [_vp, _i64]),
    "wisp_core_ensure": (_i32, [_vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "wisp_core_split": (_i32, [_vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "wisp_core_acquire": (_i32, [_vp, _i64, _vp, _i64, _vp]),
    "wisp_core_admit": (_i64, [_vp, _i64, _vp, _i64]),
    "wisp_core_preload": (_i32, [_vp, _vp, _i64]),
    "wisp_core_resized": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp]),
    "wisp_core_state": (None, [_vp, _vp, _vp]),
    "wisp_core_arrays": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "wisp_cache_create": (_i32, [_vp, _i64, _vp, _i64, _i64, _i32, _i64, _i64, _i32, _i64, _i32, _vp]),
    "wisp_cache_destroy": (None, [_vp]),
    "wisp_cache_core": (_vp, [_vp]),
    "wisp_cache_pool": (_vp, [_vp]),
    "wisp_cache_copy_stream": (_vp, [_vp]),
    "wisp_cache_counters": (None, [_vp, _vp, _vp]),
    "wisp_cache_pool_dlpack": (_vp, [_vp]),
    "wisp_cache_pool_dlpack_free": (None, [_vp]),
    "wisp_cache_issue": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "wisp_cache_sync_compute": (_i32, [_vp, _vp]),
    "wisp_cache_ensure": (_i32, [_vp, _vp, _i64, _vp, _vp]),
    "wisp_cache_prepare_layer": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "wisp_cache_prepare_row": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "wisp_cache_prepare_signaled": (_i32, [_vp, _vp, _vp, ctypes.c_uint32, _vp, _i32, _i32, _i64, _i64, _vp, _vp, _vp,
                                           _vp]),
    "wisp_cache_set_copy_mode": (_i32, [_vp, _i32]),
    "wisp_cache_resize": (_i32, [_vp, _i64]),
    "wisp_cache_device_begin": (_i32, [_vp, _vp]),
    "wisp_cache_device_step": (_i32, [_vp, _vp, _vp, _i64, _i64, _i32, _vp, _vp]),
    "wisp_cache_device_route_step": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _i64, _i64, _vp, _vp]),
    "wisp_cache_device_sync": (_i32, [_vp, _vp]),
    "wisp_cache_device_end": (_i32, [_vp, _vp]),
    "wisp_cache_device_active": (_i32, [_vp]),
    "wisp_set_tuning": (_i32, [_i32, _i32, _i32]),
    "wisp_act_read": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp]),
    "wisp_probe_empty": (_i32, [_vp]),
    "wisp_probe_stamp": (_i32, [_vp, _vp]),
    "wisp_probe_read": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp]),
    "wisp_probe_skeleton": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp]),
    "wisp_probe_skeleton_sync_bytes": (_i64, []),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python wisp-runtime_amd/build_lib.py` "
                "(or __graft_entry__.build()). There is no fallback path."
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        v = L.wisp_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libwisp_hip ABI {v}, expected {ABI_VERSION}: rebuild the library")
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != WISP_OK:
        msg = lib().wisp_last_error().decode(errors="replace")
        if rc in (WISP_EINVAL, WISP_EALIGN):
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what}: {msg} (hip error {rc})")


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*tensors: torch.Tensor, what: str) -> torch.device:
    dev = None
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(f"{what} needs ROCm device tensors (got a {t.device} tensor); no CPU path is provided")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev}, {t.device})")
    return dev
