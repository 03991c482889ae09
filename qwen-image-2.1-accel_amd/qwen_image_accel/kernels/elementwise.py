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


MOD_COPY, MOD_ONE_PLUS, MOD_TANH = 0, 1, 2


def modulation_values(mod, kinds):
    """The per-step modulation terms (reference optimizations/fusion.py:48-53,
    ``1 + s`` and ``tanh(g)`` of the modulation chunks) in one launch.

    mod: (..., P, D) contiguous bf16 on the GPU; row i of each group of P rows
    is copied (MOD_COPY), mapped to bf16(1 + x) (MOD_ONE_PLUS) or to
    bf16(tanh(x)) (MOD_TANH; tanh in float64, rounded to fp32, then to bf16),
    i.e. kinds[i].  Returns (P, ..., D): term i is the contiguous ``out[i]``."""
    p, d = len(kinds), mod.shape[-1]
    if not (mod.is_cuda and mod.dtype == torch.bfloat16 and mod.is_contiguous() and mod.ndim >= 2
            and mod.shape[-2] == p and 1 <= p <= 16 and d % 8 == 0 and mod.numel() > 0
            and all(k in (MOD_COPY, MOD_ONE_PLUS, MOD_TANH) for k in kinds)):
        raise _native.Unsupported("modulation_values", _native.QIM_ERR_ARG,
                                  f"{tuple(mod.shape)} {mod.dtype} kinds={kinds}")
    out = torch.empty((p,) + tuple(mod.shape[:-2]) + (d,), dtype=mod.dtype, device=mod.device)
    bits = sum(k << (2 * i) for i, k in enumerate(kinds))
    _native.call("qim_modulation_values", _native.ptr(mod), mod.numel() // d, d, bits, p, _native.ptr(out),
                 _native.stream(mod.device))
    return out


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
