"""BF16 SwiGLU and per-head QK RMSNorm with the reference's rounding points.

Reference interface: src/qwen_image_accel/kernels/bf16.py -- ``swiglu`` (:27-36),
``install_swiglu`` (:39-43), ``rms_norm`` (:58-63), ``install_qk_norm``
(:66-77).  Kernels: libqim's ``qim_swiglu`` and ``qim_rms_norm``.
"""
import types

import torch
import torch.nn.functional as F

from qwen_image_accel import _native

HEAD_DIMS = (64, 128, 256)


def _rows_view(t):
    """(rows, width, row stride) of a tensor whose last dim is contiguous and
    whose leading dims flatten to rows, or None."""
    if t.ndim < 1 or t.numel() == 0 or t.stride(-1) != 1:
        return None
    width = t.shape[-1]
    if t.is_contiguous():
        return t.numel() // width, width, width
    if t.ndim == 2:
        return t.shape[0], width, t.stride(0)
    return None


def swiglu(gate, value):
    """``F.silu(gate) * value`` with bf16(silu) rounded before an fp32 multiply.

    Row-strided 2-D operands (the two halves of one (M, 2F) projection) are
    accepted; other unsupported inputs take the eager path, as in the
    reference (kernels/bf16.py:28-32).
    """
    if (gate.dtype == torch.bfloat16 and value.dtype == torch.bfloat16
            and gate.is_cuda and value.is_cuda and gate.shape == value.shape
            and gate.device == value.device):
        gv, vv = _rows_view(gate), _rows_view(value)
        if (gv is not None and vv is not None and gv[1] % 8 == 0 and gv[2] % 8 == 0
                and vv[2] % 8 == 0 and gate.data_ptr() % 16 == 0 and value.data_ptr() % 16 == 0):
            rows, width = gv[0], gv[1]
            out = torch.empty(gate.shape, device=gate.device, dtype=torch.bfloat16)
            _native.call("qim_swiglu", _native.ptr(gate), gv[2], _native.ptr(value), vv[2],
                         _native.ptr(out), width, rows, width, _native.stream(gate.device))
            return out
    return F.silu(gate) * value


def install_swiglu(transformer):
    """Route every block's SwiGLU MLP through ``swiglu`` (kernels/bf16.py:39-43)."""
    for block in transformer.transformer_blocks:
        def forward(self, hidden_states):
            return self.out(swiglu(self.gate_layer(hidden_states), self.proj(hidden_states)))
        block.img_mlp.forward = types.MethodType(forward, block.img_mlp)


def rms_norm(x, weight, eps):
    """Diffusers RMSNorm over the last dim (64, 128 or 256), bf16 weight.

    Unguarded like the reference: the caller checks dtype and contiguity."""
    out = torch.empty_like(x)
    d = x.shape[-1]
    _native.call("qim_rms_norm", _native.ptr(x), _native.ptr(weight), _native.ptr(out),
                 x.numel() // d, d, float(eps), _native.stream(x.device))
    return out


def install_qk_norm(transformer):
    """Route every block's Q/K RMSNorm through ``rms_norm`` when the input is a
    contiguous CUDA bf16 tensor (kernels/bf16.py:66-77)."""
    for block in transformer.transformer_blocks:
        for norm in (block.attn.norm_q, block.attn.norm_k):
            eager = norm.forward

            def forward(self, x, _eager=eager):
                if (x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous()
                        and x.shape[-1] in HEAD_DIMS and self.weight is not None
                        and self.weight.dtype == torch.bfloat16 and self.weight.is_contiguous()
                        and getattr(self, "bias", None) is None):
                    return rms_norm(x, self.weight, self.eps)
                return _eager(x)
            norm.forward = types.MethodType(forward, norm)
