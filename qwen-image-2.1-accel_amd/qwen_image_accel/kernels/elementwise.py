"""BF16 gated residual and complex rotary embedding.

Reference interface: src/qwen_image_accel/kernels/elementwise.py --
``residual(h, x, gate)`` (:26-34) and ``rope_qk(q, k, freqs)`` (:63-69).
Kernels: libqim's ``qim_gated_residual`` and ``qim_rope_qk``.
"""
import torch

from qwen_image_accel import _native
from qwen_image_accel.kernels.bf16 import HEAD_DIMS


def residual(h, x, gate):
    """``h + gate * x`` with the product rounded to bf16 before the add.

    h, x: (B, S, D); gate: (B, 1, D).  Unsupported inputs take the eager path
    (reference guard, kernels/elementwise.py:27-28)."""
    if (h.dtype == torch.bfloat16 and h.is_contiguous() and x.is_contiguous() and h.is_cuda
            and h.ndim == 3 and x.shape == h.shape and x.dtype == torch.bfloat16
            and x.device == h.device and gate.dtype == torch.bfloat16 and gate.device == h.device
            and gate.shape == (h.shape[0], 1, h.shape[2]) and gate.is_contiguous()
            and h.shape[-1] % 8 == 0 and h.numel() > 0):
        b, s, d = h.shape
        out = torch.empty_like(h)
        _native.call("qim_gated_residual", _native.ptr(h), _native.ptr(x), _native.ptr(gate),
                     _native.ptr(out), b * s, d, s, _native.stream(h.device))
        return out
    return h + gate * x


def rope_qk(q, k, freqs):
    """Complex RoPE of q and k (B, S, H, D) with freqs (S, D/2) complex64.

    Unguarded like the reference: expects contiguous CUDA bf16 q, k."""
    out_q, out_k = torch.empty_like(q), torch.empty_like(k)
    b, s, h, d = q.shape
    if d not in HEAD_DIMS:
        raise _native.Unsupported("rope_qk", _native.QIM_ERR_SHAPE, f"head dim {d}")
    f = torch.view_as_real(freqs.contiguous())
    _native.call("qim_rope_qk", _native.ptr(q), _native.ptr(k), _native.ptr(f),
                 _native.ptr(out_q), _native.ptr(out_k), b, s, h, d, _native.stream(q.device))
    return out_q, out_k
