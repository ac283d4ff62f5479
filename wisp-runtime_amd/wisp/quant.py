"""Group-wise min-max (RTN) expert quantization: layout, quantize, dequant.

Same callable surface as the reference's wisp/quant.py (imronpuji/wisp-runtime),
implemented by the gfx950 HIP kernels of libwisp_hip.so. Layout per expert
(quant.py:1-8):
  bits == 16 : raw bf16                              -> 3*n*2 bytes
  bits <  16 : [ codes (packed) | scales fp16 | mins fp16 ]
An expert holds gate [I,H], up [I,H], down [H,I] flat as [3, n]; groups are
`group` consecutive flat elements; w = q*s + m.

Device tensors only: quantize/dequant/_pack/_unpack raise on CPU tensors (the
CPU restatement used to check these kernels is test infrastructure, oracle/).
"""

from __future__ import annotations

import torch

from . import _lib

SUPPORTED_BITS = (16, 8, 4, 3, 2)


def expert_nbytes(n: int, bits: int, group: int) -> int:
    """Bytes of one expert (quant.py:17-22)."""
    if bits == 16:
        return 3 * n * 2
    assert bits in SUPPORTED_BITS, bits
    assert (3 * n) % group == 0 and (3 * n * bits) % 8 == 0, "3*n must be divisible by group and by 8/bits"
    return (3 * n * bits) // 8 + 4 * (3 * n // group)


def _pack(q: torch.Tensor, bits: int) -> torch.Tensor:
    """q: flat uint8 codes (< 2**bits) -> packed uint8 (quant.py:25-41)."""
    dev = _lib.require_gpu(q, what="_pack")
    q = q.reshape(-1).to(torch.uint8).contiguous()
    out = torch.empty(q.numel() * bits // 8, dtype=torch.uint8, device=dev)
    _lib.check(_lib.lib().wisp_pack(_lib.ptr(q), q.numel(), bits, _lib.ptr(out), _lib.stream(dev)), "_pack")
    return out


def _unpack(c: torch.Tensor, bits: int) -> torch.Tensor:
    """c: [B, nbytes] uint8 -> [B, m] uint8 codes (quant.py:44-57)."""
    dev = _lib.require_gpu(c, what="_unpack")
    B = c.shape[0]
    c = c.contiguous()
    m = c[0].numel() * 8 // bits
    out = torch.empty((B, m), dtype=torch.uint8, device=dev)
    _lib.check(
        _lib.lib().wisp_unpack(_lib.ptr(c), B * m, bits, _lib.ptr(out), _lib.stream(dev)),
        "_unpack",
    )
    return out


@torch.no_grad()
def quantize(w3: torch.Tensor, bits: int, group: int = 128, out: torch.Tensor | None = None) -> torch.Tensor:
    """w3: [3, n] (any float dtype) on the GPU -> flat uint8 buffer (quant.py:60-73), bit-exact.
    out: an optional contiguous uint8 device buffer of expert_nbytes(n, bits, group) to write."""
    dev = _lib.require_gpu(w3, what="quantize")
    if bits == 16:
        b = w3.to(torch.bfloat16).contiguous().view(torch.uint8).reshape(-1)
        return b if out is None else out.copy_(b)
    w = w3.reshape(-1)
    if w.dtype not in (torch.float32, torch.bfloat16):
        w = w.float()  # the reference's .float(): exact for fp16, RTNE for fp64
    w = w.contiguous()
    n = w.numel() // 3
    nb = expert_nbytes(n, bits, group)
    if out is None:
        out = torch.empty(nb, dtype=torch.uint8, device=dev)
    assert out.dtype == torch.uint8 and out.is_contiguous() and out.numel() == nb and out.device == dev, (
        "out must be a contiguous uint8 buffer of expert_nbytes on w3's device")
    _lib.check(
        _lib.lib().wisp_quantize(
            _lib.ptr(w), 1 if w.dtype == torch.bfloat16 else 0, n, bits, group, _lib.ptr(out), _lib.stream(dev)
        ),
        "quantize",
    )
    return out


def dequant(buf: torch.Tensor, n: int, bits: int, group: int = 128) -> torch.Tensor:
    """buf: [B, >=nbytes] uint8 rows on the GPU -> [B, 3, n] bfloat16 (quant.py:76-87), bit-exact."""
    B = buf.shape[0]
    if bits == 16:
        return buf.contiguous().view(torch.bfloat16).view(B, 3, n)
    dev = _lib.require_gpu(buf, what="dequant")
    if buf.dim() != 2 or buf.stride(1) != 1:
        buf = buf.reshape(B, -1).contiguous()
    out = torch.empty((B, 3, n), dtype=torch.bfloat16, device=dev)
    if B == 0:  # an empty batch dequantizes to an empty tensor, as the reference's torch ops do
        return out
    _lib.check(
        _lib.lib().wisp_dequant(
            _lib.ptr(buf), buf.stride(0), None, B, B, n, bits, group, _lib.ptr(out), _lib.stream(dev)
        ),
        "dequant",
    )
    return out


def dequant_fast(buf, n, bits, group=128):
    """quant.py:94-111. The reference fuses dequant() with torch.compile; here dequant()
    is already one fused HIP kernel, so this is the same call (bit-identical by construction)."""
    return dequant(buf, n, bits, group)


def dequant_rows(pool: torch.Tensor, idx: torch.Tensor, n: int, bits: int, group: int = 128) -> torch.Tensor:
    """index_select(pool, 0, idx) + dequant in one kernel (cache.py:121-127, weights_batched).
    Rows with an index outside [0, pool.shape[0]) come back as NaN (no out-of-bounds read)."""
    k = idx.numel()
    if bits == 16:
        return pool.index_select(0, idx).view(torch.bfloat16).view(k, 3, n)
    dev = _lib.require_gpu(pool, idx, what="dequant_rows")
    assert pool.dim() == 2 and pool.stride(1) == 1, "pool must be a row-contiguous [nslots, nbytes] uint8 tensor"
    idx = idx.reshape(-1).to(torch.int64).contiguous()
    out = torch.empty((k, 3, n), dtype=torch.bfloat16, device=dev)
    _lib.check(
        _lib.lib().wisp_dequant(
            _lib.ptr(pool), pool.stride(0), _lib.ptr(idx), k, pool.shape[0], n, bits, group, _lib.ptr(out),
            _lib.stream(dev),
        ),
        "dequant_rows",
    )
    return out
