"""Block-scaled E4M3 quantization (MXFP8) and its 128x4 swizzled scale layout.

Reference interface: src/qwen_image_accel/kernels/mxfp8.py (Quantized :11-17,
padded_rows :20-22, quantize :59-67).  The arithmetic runs in libqim's
``qim_mx_quantize`` HIP kernel.
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


def padded_rows(rows):
    """MXFP8 scales are tiled over 128 rows, so M is padded to a multiple of 128."""
    return (rows + 127) // 128 * 128


BLOCK = 32        # MX block length along K
ROW_TILE = 128    # rows per scale tile
K_TILE = 128      # 4 scale blocks: one 512-byte swizzle tile


def empty_quantized(rows, k, device, shape=None):
    """Allocate the output buffers of a quantization of (rows, k)."""
    padded = padded_rows(rows)
    q = torch.empty((padded, k), device=device, dtype=torch.float8_e4m3fn)
    s = torch.empty(padded * k // BLOCK, device=device, dtype=torch.uint8)
    return Quantized(q, s.view(torch.float8_e8m0fnu), rows,
                     torch.Size((rows, k)) if shape is None else torch.Size(shape))


def quantize(x):
    """Quantize a BF16 ``(M, K)`` activation (unit column stride) to MXFP8.

    Like the reference this function is unguarded: it expects a CUDA bf16
    tensor with K % 128 == 0 and raises ``_native.Unsupported`` otherwise.
    """
    m, k = x.shape
    if x.dtype != torch.bfloat16 or not x.is_cuda or x.stride(1) != 1:
        raise _native.Unsupported("quantize", _native.QIM_ERR_LAYOUT,
                                  "expects a CUDA bfloat16 (M, K) tensor with unit column stride")
    out = empty_quantized(m, k, x.device, x.shape)
    _native.call("qim_mx_quantize", _native.ptr(x), x.stride(0), m, k, _native.ptr(out.values),
                 _native.ptr(out.scales), _native.stream(x.device))
    return out
