"""Block-scaled E4M3 quantization (MXFP8) and its 128x4 swizzled scale layout.

Reference interface: src/qwen_image_accel/kernels/mxfp8.py (Quantized :11-17,
padded_rows :20-22, quantize :59-67).  The arithmetic runs in libqim's
``qim_mx_quantize`` HIP kernel.

Besides the reference's row-major codes, the quantizers can write the codes in
the GEMM's tiled layout (``TiledQuantized``; no reference counterpart): rows in
super-blocks of 256 (the last holds 128 when the padded row count is an odd
multiple of 128), each 64-byte K-slab of a super-block contiguous, and inside
it the 16-byte chunk c of row r at chunk c ^ (((r >> 1) ^ (r >> 2)) & 3).  A
16-row group of one slab is then the 1 KiB LDS image one DMA instruction of
the GEMM loads.  Scales are the same swizzled bytes in both forms.
"""
from typing import NamedTuple

import torch

from qwen_image_accel import _native


class Quantized(NamedTuple):
    """An MXFP8 activation: padded E4M3 values plus their swizzled E8M0 scales."""

    values: torch.Tensor     # (rows padded to 128, K) float8_e4m3fn
    scales: torch.Tensor     # flat float8_e8m0fnu in the 128x4 block order
    rows: int                # live rows, before padding
    shape: torch.Size        # logical shape of the tensor this came from

    tiled = False            # codes row-major (the reference's layout)


class TiledQuantized(Quantized):
    """A ``Quantized`` whose ``values`` bytes are in the GEMM's tiled layout."""

    __slots__ = ()
    tiled = True


def padded_rows(rows):
    """MXFP8 scales are tiled over 128 rows, so M is padded to a multiple of 128."""
    return (rows + 127) // 128 * 128


BLOCK = 32        # MX block length along K
ROW_TILE = 128    # rows per scale tile
K_TILE = 128      # 4 scale blocks: one 512-byte swizzle tile


def empty_quantized(rows, k, device, shape=None, tiled=False):
    """Allocate the output buffers of a quantization of (rows, k)."""
    padded = padded_rows(rows)
    q = torch.empty((padded, k), device=device, dtype=torch.float8_e4m3fn)
    s = torch.empty(padded * k // BLOCK, device=device, dtype=torch.uint8)
    kind = TiledQuantized if tiled else Quantized
    return kind(q, s.view(torch.float8_e8m0fnu), rows,
                torch.Size((rows, k)) if shape is None else torch.Size(shape))


def quantize(x, *, tiled=False):
    """Quantize a BF16 ``(M, K)`` activation (unit column stride) to MXFP8.

    Like the reference this function is unguarded: it expects a CUDA bf16
    tensor with K % 128 == 0 and raises ``_native.Unsupported`` otherwise.
    ``tiled=True`` writes the codes in the GEMM's tiled layout and returns a
    ``TiledQuantized`` (same bytes, reordered; same scales).
    """
    m, k = x.shape
    if x.dtype != torch.bfloat16 or not x.is_cuda or x.stride(1) != 1:
        raise _native.Unsupported("quantize", _native.QIM_ERR_LAYOUT,
                                  "expects a CUDA bfloat16 (M, K) tensor with unit column stride")
    out = empty_quantized(m, k, x.device, x.shape, tiled)
    _native.call("qim_mx_quantize_tiled" if tiled else "qim_mx_quantize", _native.ptr(x), x.stride(0), m,
                 k, _native.ptr(out.values), _native.ptr(out.scales), _native.stream(x.device))
    return out


def _chunk_order(rows, device):
    """(rows, 4) chunk permutation of the tiled layout: c ^ swizzle(r); an involution."""
    r = torch.arange(rows, device=device).unsqueeze(1)
    c = torch.arange(4, device=device).unsqueeze(0)
    return c ^ (((r >> 1) ^ (r >> 2)) & 3)


def _retile(codes, to_tiled):
    rows, k = codes.shape
    if rows % 128 or k % 64:
        raise ValueError(f"tiled codes need rows % 128 == 0 and K % 64 == 0, got {tuple(codes.shape)}")
    src = codes.contiguous().view(torch.uint8).reshape(-1)
    out = torch.empty_like(src)
    for r0 in range(0, rows, 256):
        n = min(256, rows - r0)
        block = src[r0 * k:(r0 + n) * k]
        order = _chunk_order(n, codes.device).view(n, 1, 4, 1).expand(n, k // 64, 4, 16)
        if to_tiled:   # (n, slab, chunk, byte) -> chunks permuted -> (slab, n, chunk, byte)
            tiled = block.view(n, k // 64, 4, 16).gather(2, order).permute(1, 0, 2, 3)
        else:          # (slab, n, chunk, byte) -> (n, slab, chunk, byte) -> chunks restored
            tiled = block.view(k // 64, n, 4, 16).permute(1, 0, 2, 3).gather(2, order)
        out[r0 * k:(r0 + n) * k] = tiled.reshape(-1)
    return out.view(codes.dtype).view(rows, k)


def tile_codes(codes):
    """Row-major ``(R, K)`` E4M3 codes -> the same codes in the tiled layout (a copy)."""
    return _retile(codes, True)


def untile_codes(codes):
    """Tiled ``(R, K)`` E4M3 codes -> row-major (a copy)."""
    return _retile(codes, False)


def as_tiled(q):
    """A ``Quantized`` in the tiled layout (itself if it already is)."""
    return q if q.tiled else TiledQuantized(tile_codes(q.values), q.scales, q.rows, q.shape)


def as_row_major(q):
    """A ``Quantized`` in the reference's row-major layout (itself if it already is)."""
    return Quantized(untile_codes(q.values), q.scales, q.rows, q.shape) if q.tiled else q
