"""Fused Q/K RMSNorm + RoPE + prefix K/V packing of cached decode.

Reference interface: src/qwen_image_accel/kernels/attention.py:92-159
``prepare_attention_inputs(q, k, v, norm_q, norm_k, freqs, cached_k, cached_v)``
-> ``(rope(norm_q(q)), cat[ck, rope(norm_k(k))], cat[cv, v])`` or ``None``.
Kernel: libqim's ``qim_qk_norm_rope_pack``; any head count (the reference's
kernel is fixed to 32 x 128) and head dims 64/128/256.  No buffer persists
across calls.
"""
import torch

from qwen_image_accel import _native
from qwen_image_accel.kernels import mxfp8
from qwen_image_accel.kernels.bf16 import HEAD_DIMS


def _norm_ok(norm, d, device):
    w = getattr(norm, "weight", None)
    return (w is not None and getattr(norm, "bias", None) is None and w.shape == (d,)
            and w.dtype == torch.bfloat16 and w.device == device and w.is_contiguous())


def prepare_attention_inputs(q, k, v, norm_q, norm_k, freqs, cached_k, cached_v):
    """Return fused Q/K/V, or None when the original operators should be used."""
    if (q.ndim != 4 or q.shape[-1] not in HEAD_DIMS or q.shape[1] == 0
            or k.shape != q.shape or v.shape != q.shape
            or freqs is None or freqs.dtype != torch.complex64
            or freqs.shape != (q.shape[1], q.shape[-1] // 2) or not freqs.is_contiguous()
            or freqs.device != q.device
            or cached_k.ndim != 4 or cached_k.shape[0] != q.shape[0]
            or cached_k.shape[2:] != q.shape[2:] or cached_v.shape != cached_k.shape):
        return None
    for t in (q, k, v, cached_k, cached_v):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.device != q.device:
            return None
    for t in (cached_k, cached_v):
        if not t.is_contiguous():
            return None
    # q, k, v: contiguous, or column blocks of one fused QKV output -- packed
    # heads and one token stride shared by the three (the kernel's ldt).
    b, s, h, d = q.shape
    ldt = q.stride(1)
    for t in (q, k, v):
        if t.stride() != (s * ldt, ldt, d, 1):
            return None
    if not (_norm_ok(norm_q, d, q.device) and _norm_ok(norm_k, d, q.device)):
        return None
    p = cached_k.shape[1]
    oq = torch.empty((b, s, h, d), device=q.device, dtype=q.dtype)
    ok = torch.empty((b, s + p, h, d), device=q.device, dtype=q.dtype)
    ov = torch.empty_like(ok)
    f = torch.view_as_real(freqs)
    _native.call("qim_qk_norm_rope_pack", _native.ptr(q), _native.ptr(k), _native.ptr(v),
                 _native.ptr(cached_k) if p else None, _native.ptr(cached_v) if p else None,
                 _native.ptr(norm_q.weight), _native.ptr(norm_k.weight), _native.ptr(f),
                 _native.ptr(oq), _native.ptr(ok), _native.ptr(ov), b, s, p, h, d, ldt,
                 float(norm_q.eps), float(norm_k.eps), _native.stream(q.device))
    return oq, ok, ov


def workspace(b, s, t, h, device, d=128):
    """A workspace for ``attention`` / ``attention_mxfp8`` of this shape (V^T
    tiles first, then the split items' partial results)."""
    with torch.cuda.device(device):
        nbytes = _native.lib().qim_attention_workspace_bytes(b, s, t, h, d)
    if nbytes <= 0:
        raise _native.Unsupported("attention", _native.QIM_ERR_SHAPE, f"head dim {d} (128 only)")
    return torch.empty(nbytes, device=device, dtype=torch.uint8)


def _common(name, q, k, v, ws):
    b, s, h, d = q.shape
    t = k.shape[1]
    for x, n in ((q, s), (k, t), (v, t)):
        if x is None:
            continue
        if (x.dtype != torch.bfloat16 or not x.is_cuda or x.shape != (b, n, h, d) or x.stride(3) != 1
                or x.stride(2) != d or x.stride(0) != n * x.stride(1)):
            raise _native.Unsupported(name, _native.QIM_ERR_LAYOUT,
                                      "expects bf16 (B, N, H, D) tensors with packed heads and token rows")
    if v is None and ws is None:
        raise ValueError(f"{name}: v=None needs the workspace holding V^T")
    if ws is None:
        ws = workspace(b, s, t, h, q.device, d)
    vp, ldv = (None, 0) if v is None else (_native.ptr(v), v.stride(1))
    return b, s, t, h, d, vp, ldv, ws


def attention(q, k, v, scale=None, out=None, *, workspace=None):
    """softmax(q k^T * scale) v per (batch, head): libqim's ``qim_attention``.

    q: (B, S, H, 128), k, v: (B, T, H, 128) bf16 on the GPU, each with unit
    stride inside a token and any token stride (e.g. views into a fused QKV
    projection).  scale defaults to 1/sqrt(128).  Returns (B, S, H, 128) bf16.
    ``workspace``: from ``attention.workspace`` (allocated per call if None);
    with ``v=None`` it must already hold V^T, written by the QKV projection
    (``gemm.mx_matmul_qk_norm_rope(..., vt=workspace)``, T % 64 == 0).
    The block's attention core; the reference calls torch SDPA there
    (optimizations/quantized_decode.py:70-77)."""
    b, s, t, h, d, vp, ldv, ws = _common("attention", q, k, v, workspace)
    if out is None:
        out = torch.empty((b, s, h, d), device=q.device, dtype=torch.bfloat16)
    _native.call("qim_attention", _native.ptr(q), q.stride(1), _native.ptr(k), k.stride(1), vp, ldv,
                 _native.ptr(out), out.stride(1), _native.ptr(ws), ws.numel(), b, s, t, h, d,
                 float(scale if scale is not None else d ** -0.5), _native.stream(q.device))
    return out


def attention_mxfp8(q, k, v, scale=None, *, tiled=True, out=None, workspace=None):
    """``mxfp8.quantize(attention(q, k, v).reshape(B*S, H*128), tiled=tiled)``
    in one pass (libqim's ``qim_attention_mxfp8``): the same codes and scales,
    without the bf16 output.  The block's out-projection input; the reference
    runs SDPA and then its quantize kernel (optimizations/quantized_decode.py:
    70-96).  ``out``: a preallocated ``mxfp8.empty_quantized(B*S, H*128,
    device, tiled=tiled)``; ``workspace`` and ``v=None`` as for ``attention``."""
    b, s, t, h, d, vp, ldv, ws = _common("attention_mxfp8", q, k, v, workspace)
    if out is None:
        out = mxfp8.empty_quantized(b * s, h * d, q.device, tiled=tiled)
    _native.call("qim_attention_mxfp8", _native.ptr(q), q.stride(1), _native.ptr(k), k.stride(1), vp, ldv,
                 _native.ptr(out.values), _native.ptr(out.scales), int(tiled), _native.ptr(ws), ws.numel(),
                 b, s, t, h, d, float(scale if scale is not None else d ** -0.5), _native.stream(q.device))
    return out


def qk_norm_rope(q, k, weight_q, weight_k, freqs, eps_q=1e-6, eps_k=1e-6, heads=None):
    """Fused QK-RMSNorm + RoPE without a V pack (the MMDiT block's form).

    q, k: (B, S, H, D) bf16, or (B*S, >= H*D) row views into a fused QKV
    projection output (then ``heads`` gives H and the row stride is the token
    stride).  Returns contiguous (B, S, H, D) tensors."""
    if q.ndim == 4:
        b, s, h, d = q.shape
        ldt = q.stride(1)
        if (q.stride(3) != 1 or q.stride(2) != d or k.stride() != q.stride()
                or q.stride(0) != s * q.stride(1)):
            raise _native.Unsupported("qk_norm_rope", _native.QIM_ERR_LAYOUT, "q/k layout")
    else:
        rows, width = q.shape
        h = heads
        d = width // h
        b, s = 1, rows
        ldt = q.stride(0)
        if q.stride(1) != 1 or k.stride() != q.stride():
            raise _native.Unsupported("qk_norm_rope", _native.QIM_ERR_LAYOUT, "q/k layout")
    oq = torch.empty((b, s, h, d), device=q.device, dtype=torch.bfloat16)
    ok = torch.empty_like(oq)
    f = torch.view_as_real(freqs.contiguous())
    _native.call("qim_qk_norm_rope_pack", _native.ptr(q), _native.ptr(k), None, None, None,
                 _native.ptr(weight_q), _native.ptr(weight_k), _native.ptr(f), _native.ptr(oq),
                 _native.ptr(ok), None, b, s, 0, h, d, ldt, float(eps_q), float(eps_k),
                 _native.stream(q.device))
    return oq, ok
