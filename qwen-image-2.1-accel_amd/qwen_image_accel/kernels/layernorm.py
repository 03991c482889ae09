"""LayerNorm x timestep scale (AdaLN modulate), with optional MMDiT extras.

Reference interface: src/qwen_image_accel/kernels/layernorm.py:58-86
``layer_norm_scale(x, scale, norm)`` = eager ``norm(x) * scale`` with the bf16
rounding of each op.  The keyword-only extras default to the reference's
behaviour; with them the call computes the full modulated residual branch
``residual + gate * ((1 + scale) * LN(x) + shift)`` in one HBM pass, a bf16
rounding after every eager op.  The kernel is libqim's ``qim_adaln`` (any
D % 8 == 0 up to 16384; the reference kernel is fixed to D = 4096).

Unsupported inputs (CPU tensors, other dtypes, non-contiguous x, an affine
norm) take the eager composition, as the reference's guard does
(kernels/layernorm.py:59-73).
"""
import torch

from qwen_image_accel import _native


def _eager(x, scale, norm, shift, gate, residual, add_one):
    s = 1 + scale if add_one else scale
    y = norm(x) * s
    if shift is not None:
        y = y + shift
    if gate is not None:
        y = gate * y
    if residual is not None:
        y = residual + y
    return y


def _vec_ok(v, x):
    b, _, d = x.shape
    return (v is None or (v.shape == (b, 1, d) and v.dtype == torch.bfloat16
                          and v.device == x.device and v.is_contiguous()))


def native_supported(x, scale, norm, shift=None, gate=None, residual=None):
    """True when the HIP kernel handles these operands (the guard of
    kernels/layernorm.py:59-72, generalised in D)."""
    if (x.ndim != 3 or not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous()
            or x.numel() == 0):
        return False
    d = x.shape[-1]
    if d % 8 or d > 16384:
        return False
    if not (_vec_ok(scale, x) and _vec_ok(shift, x) and _vec_ok(gate, x)):
        return False
    if scale is None:
        return False
    if residual is not None and (residual.shape != x.shape or residual.dtype != torch.bfloat16
                                 or residual.device != x.device or not residual.is_contiguous()):
        return False
    if getattr(norm, "elementwise_affine", False) or tuple(norm.normalized_shape) != (d,):
        return False
    return True


def _flags(add_one):
    return _native.ADALN_ADD_ONE if add_one else 0


def layer_norm_scale(x, scale, norm, *, shift=None, gate=None, residual=None, add_one=False):
    """``norm(x) * scale`` (+ shift, x gate, + residual) with eager bf16 rounding."""
    if not native_supported(x, scale, norm, shift, gate, residual):
        return _eager(x, scale, norm, shift, gate, residual, add_one)
    b, s, d = x.shape
    out = torch.empty_like(x)
    _native.call("qim_adaln", _native.ptr(x), _native.ptr(scale), _native.ptr(shift),
                 _native.ptr(gate), _native.ptr(residual), _native.ptr(out), b * s, d, s,
                 float(norm.eps), _flags(add_one), _native.stream(x.device))
    return out
