"""Fused MXFP8 producers: FP8 straight out of the LayerNorm and the SwiGLU.

Reference interface: src/qwen_image_accel/kernels/epilogue.py
``layer_norm_scale_quantize(x, scale, norm)`` (:76-92, kernel :23-73) and
``swiglu_quantize(gate, value)`` (:123-136, kernel :95-120).  Each returns a ``Quantized``
byte-identical to ``quantize`` of the unfused bf16 result, or ``None`` when the
inputs are unsupported (the caller then takes the unfused path,
optimizations/quantized_decode.py:99-105).  ``tiled=True`` (no reference
counterpart) writes the codes in the GEMM's tiled layout (``TiledQuantized``).
"""
import torch

from qwen_image_accel import _native
from qwen_image_accel.kernels.layernorm import _flags, native_supported
from qwen_image_accel.kernels.mxfp8 import empty_quantized


def layer_norm_scale_quantize(x, scale, norm, *, shift=None, gate=None, residual=None,
                              add_one=False, tiled=False):
    """LayerNorm, modulation and MXFP8 quantization in one pass, or None."""
    if not native_supported(x, scale, norm, shift, gate, residual) or x.shape[-1] % 128:
        return None
    b, s, d = x.shape
    out = empty_quantized(b * s, d, x.device, x.shape, tiled)
    flags = _flags(add_one) | (_native.ADALN_TILED if tiled else 0)
    _native.call("qim_adaln_quantize", _native.ptr(x), _native.ptr(scale), _native.ptr(shift),
                 _native.ptr(gate), _native.ptr(residual), _native.ptr(out.values),
                 _native.ptr(out.scales), b * s, d, s, float(norm.eps), flags,
                 _native.stream(x.device))
    return out


def _rows_ok(t):
    return t.ndim == 2 and t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def swiglu_quantize(gate, value, *, tiled=False):
    """SwiGLU and MXFP8 quantization in one pass, or None when unsupported.

    Unlike the reference, row-strided operands (e.g. the two halves of one
    (M, 2F) projection) are accepted without a copy.
    """
    if (gate.dtype != torch.bfloat16 or value.dtype != torch.bfloat16
            or not gate.is_cuda or gate.shape != value.shape or value.device != gate.device
            or gate.ndim != 2 or gate.shape[-1] % 128 or gate.numel() == 0
            or not _rows_ok(gate) or not _rows_ok(value)):
        return None
    rows, width = gate.shape
    out = empty_quantized(rows, width, gate.device, gate.shape, tiled)
    _native.call("qim_swiglu_quantize_tiled" if tiled else "qim_swiglu_quantize", _native.ptr(gate),
                 gate.stride(0), _native.ptr(value),
                 value.stride(0), _native.ptr(out.values), _native.ptr(out.scales), rows, width,
                 _native.stream(gate.device))
    return out
