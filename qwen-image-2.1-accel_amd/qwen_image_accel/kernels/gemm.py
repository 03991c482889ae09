"""MXFP8 GEMM with fused epilogues (the ``torch._scaled_mm`` call site).

Reference interface: src/qwen_image_accel/optimizations/mxfp8.py:32-36
``MXFP8Linear.matmul`` = ``torch._scaled_mm(A_q, W_q, scale_a, scale_b,
out_dtype=bf16)[:rows]``.  Here the product is libqim's ``qim_mxfp8_gemm``
(CDNA4 scaled MFMA, fp32 accumulation) and the epilogue that follows the GEMM
in the reference's block (bias, gated residual, SwiGLU, SwiGLU -> MXFP8) is
applied before the store.
"""
import torch

from qwen_image_accel import _native
from qwen_image_accel.kernels.mxfp8 import Quantized, empty_quantized

EPILOGUES = {
    "none": _native.EPI_NONE,
    "bias": _native.EPI_BIAS,
    "gated_residual": _native.EPI_GATED_RESIDUAL,
    "swiglu": _native.EPI_SWIGLU,
    "swiglu_quant": _native.EPI_SWIGLU_QUANT,
}


def mx_matmul_qk_norm_rope(activation, weight_fp8, weight_scale, weight_q, weight_k, freqs, heads, seq,
                           eps_q=1e-6, eps_k=1e-6, *, weight_tiled=False, out=None, vt=None):
    """The MMDiT block's QKV projection with QK-RMSNorm + RoPE in its epilogue.

    Returns the bf16 ``(rows, 3 * heads * 128)`` projection whose Q and K
    columns are ``rope(RMSNorm(.))`` per 128-wide head -- what
    ``kernels.attention.qk_norm_rope`` computes on the unfused output -- and
    whose V columns are the plain product.  ``freqs``: complex64 (seq, 64),
    row = output row % seq.  No reference counterpart as one call: it fuses
    kernels/attention.py:16-89 into optimizations/mxfp8.py:32-36.

    ``vt``: an attention workspace (``attention.workspace``; seq % 64 == 0,
    rows a multiple of seq): the V columns are written there as the
    attention core's V^T tiles instead of into the output, whose V columns
    are then left unwritten; pass ``v=None`` and this workspace to
    ``attention.attention`` / ``attention_mxfp8``."""
    a = activation
    w = weight_fp8 if weight_tiled else weight_rows(weight_fp8)
    n, k = w.shape
    if n != 3 * heads * 128 or a.values.shape[1] != k:
        raise ValueError(f"QKV weight must be (3 * {heads} * 128, K) with the activation's K")
    if freqs.dtype != torch.complex64 or freqs.shape != (seq, 64):
        raise ValueError("freqs must be complex64 (seq, 64)")
    m = a.rows
    if out is None:
        out = torch.empty((m, n), device=a.values.device, dtype=torch.bfloat16)
    if out.dtype != torch.bfloat16 or out.stride(-1) != 1 or out.shape != (m, n):
        raise ValueError("out must be a bf16 (rows, N) tensor with unit column stride")
    layouts = (_native.GEMM_A_TILED if a.tiled else 0) | (_native.GEMM_B_TILED if weight_tiled else 0)
    f = torch.view_as_real(freqs.contiguous())
    args = (_native.ptr(a.values), _native.ptr(a.scales), _native.ptr(w), _native.ptr(weight_scale), m, k, heads,
            layouts, _native.ptr(weight_q), _native.ptr(weight_k), _native.ptr(f), seq, float(eps_q), float(eps_k),
            _native.ptr(out), out.stride(0))
    if vt is None:
        _native.call("qim_mxfp8_gemm_qk_norm_rope", *args, _native.stream(out.device))
    else:
        if vt.numel() * vt.element_size() < m // seq * heads * seq * 256:
            raise ValueError("vt workspace too small")
        _native.call("qim_mxfp8_gemm_qk_norm_rope_vt", *args, _native.ptr(vt), _native.stream(out.device))
    return out


def weight_rows(weight_fp8):
    """The (N, K) row-major code matrix behind a weight given either as the
    reference's column-major (K, N) ``values.t()`` view or as (N, K)."""
    w = weight_fp8
    if not w.is_contiguous() and w.t().is_contiguous():
        w = w.t()
    if not w.is_contiguous():
        raise _native.Unsupported("mx_matmul", _native.QIM_ERR_LAYOUT, "weight codes must be dense")
    return w


def interleave_swiglu(gate_weight, up_weight, group=_native.SWIGLU_GROUP):
    """Stack gate (F, K) and up (F, K) weights into the (2F, K) row order the
    SwiGLU epilogues expect: groups of ``group`` gate rows, then the same up rows."""
    f, k = gate_weight.shape
    if up_weight.shape != (f, k) or f % group:
        raise ValueError(f"gate/up weights must both be (F, K) with F % {group} == 0")
    return torch.stack([gate_weight.reshape(f // group, group, k),
                        up_weight.reshape(f // group, group, k)], dim=1).reshape(2 * f, k)


_OUT_FORMATS = {torch.bfloat16: 0, torch.float32: _native.GEMM_OUT_F32, torch.float16: _native.GEMM_OUT_F16}


_WS_EPILOGUES = (_native.EPI_NONE, _native.EPI_BIAS, _native.EPI_GATED_RESIDUAL)


def mx_matmul(activation, weight_fp8, weight_scale, *, epilogue="none", bias=None, gate=None,
              residual=None, seq=None, out=None, weight_tiled=False, out_tiled=False, dtype=torch.bfloat16):
    """``activation @ weight.T`` in MXFP8 with a fused epilogue.

    activation: ``Quantized`` (Mp, K), row-major or tiled (``TiledQuantized``).
    weight_fp8: codes of the (N, K) weight (or its (K, N) column-major view), or
    with ``weight_tiled=True`` the (N, K) codes in the tiled layout;
    weight_scale: its swizzled scales.  Returns bf16 (rows, N) -- (rows, N/2)
    for "swiglu" -- or a ``Quantized`` (rows, N/2) for "swiglu_quant"
    (``TiledQuantized`` with ``out_tiled=True``).  ``gate`` is (B, 1, N) or
    (B, N) with ``seq`` rows per batch; ``residual`` is (rows, N).  ``dtype``:
    the output type of the plain epilogue ("none"): bf16, fp32 or fp16, as
    torch._scaled_mm's out_dtype (optimizations/mxfp8.py:34-35); the other
    epilogues write bf16."""
    epi = EPILOGUES[epilogue]
    if dtype not in _OUT_FORMATS:
        raise ValueError(f"the MXFP8 GEMM writes bf16, fp32 or fp16, not {dtype}")
    if dtype != torch.bfloat16 and epi != _native.EPI_NONE:
        raise ValueError(f"a {dtype} output is available with the plain epilogue only")
    a = activation
    w = weight_fp8 if weight_tiled else weight_rows(weight_fp8)
    if weight_tiled and not w.is_contiguous():
        raise _native.Unsupported("mx_matmul", _native.QIM_ERR_LAYOUT, "tiled weight codes must be dense")
    n, k = w.shape
    if out_tiled and epi != _native.EPI_SWIGLU_QUANT:
        raise ValueError("out_tiled applies to the quantized SwiGLU epilogue only")
    layouts = ((_native.GEMM_A_TILED if a.tiled else 0) | (_native.GEMM_B_TILED if weight_tiled else 0)
               | (_native.GEMM_OUT_TILED if out_tiled else 0) | _OUT_FORMATS[dtype])
    if a.values.shape[1] != k:
        raise ValueError(f"activation K={a.values.shape[1]} does not match weight K={k}")
    m = a.rows
    dev = a.values.device
    out_scales = None
    if epi == _native.EPI_SWIGLU_QUANT:
        result = empty_quantized(m, n // 2, dev, tiled=out_tiled)
        buf, ldo, out_scales = result.values, n // 2, result.scales
    else:
        width = n // 2 if epi == _native.EPI_SWIGLU else n
        if out is None:
            out = torch.empty((m, width), device=dev, dtype=dtype)
        if out.dtype != dtype or out.stride(-1) != 1 or out.shape != (m, width):
            raise ValueError(f"out must be a {dtype} (rows, N) tensor with unit column stride")
        buf, ldo, result = out, out.stride(0), out
    if epi == _native.EPI_GATED_RESIDUAL:
        gate = gate.reshape(-1, n)
        if residual.shape != (m, n) or not residual.is_contiguous() or not gate.is_contiguous():
            raise ValueError("gated residual needs a contiguous (rows, N) residual and (B, N) gate")
    args = (_native.ptr(a.values), _native.ptr(a.scales), _native.ptr(w), _native.ptr(weight_scale), m, n, k, epi,
            layouts, _native.ptr(bias), _native.ptr(gate), _native.ptr(residual), int(seq or m), _native.ptr(buf),
            ldo, _native.ptr(out_scales))
    # A tile grid whose last partial round is a few quarter tiles splits them
    # over K with a workspace from torch's caching allocator (stream-ordered,
    # so reusing it for the next call on the stream is safe).
    ws_bytes = _native.lib().qim_mxfp8_gemm_ws_bytes(m, n, k, epi) if epi in _WS_EPILOGUES else 0
    if ws_bytes > 0:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _native.call("qim_mxfp8_gemm_ws", *args, _native.ptr(ws), ws_bytes, _native.stream(dev))
    else:
        _native.call("qim_mxfp8_gemm_ex", *args, _native.stream(dev))
    return result
