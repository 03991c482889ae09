"""The reference's eager PyTorch path for the hot-path configurations, as
torch CPU ops in bf16.

TEST INFRASTRUCTURE ONLY: bench.py's ``cpu_baseline`` leg times these on the
host cores (the reference's own eager composition, which its kernels replace),
and tests/test_oracle.py holds them to the C oracle.  The product path never
imports this module.

Each function restates the eager composition the reference's kernels are
checked against, with the same op order and bf16 rounding at every op
boundary (torch does the rounding itself):
  - adaln: LayerNorm (eps, no affine) then (1 + scale), shift, gate, residual
    (kernels/layernorm.py:58-86 fallback; the MMDiT config-1 chain);
  - qk_rmsnorm_rope: Diffusers RMSNorm (WHL!diffusers/models/normalization.py:
    553-565) then apply_rotary_emb_qwen (WHL!transformer_qwenimage21.py:
    128-133), the reference of kernels/attention.py's check;
  - swiglu: F.silu(g) * v (WHL!transformer_qwenimage21.py:212);
  - gated_residual: h + gate * x (WHL!transformer_qwenimage21.py:641);
  - mx_quantize: the reference check's ref_quant (tests/gpu/check_mxfp8.py:
    20-30) and its 128x4 swizzle (:32-34);
  - mx_matmul: dequantize to fp32, matmul, + bias, bf16 (the tolerance
    reference of torch._scaled_mm, optimizations/mxfp8.py:32-36);
  - block: the config-5 block (optimizations/quantized_decode.py:117-135) with
    the attention stand-in o = v.
"""
import torch
import torch.nn.functional as F


def adaln(x, scale, shift=None, gate=None, res=None, eps=1e-6, add_one=True):
    """x, res: (B, S, D) bf16; scale, shift, gate: (B, 1, D) bf16."""
    y = F.layer_norm(x, (x.shape[-1],), eps=eps) * ((1 + scale) if add_one else scale)
    if shift is not None:
        y = y + shift
    if gate is not None:
        y = gate * y
    if res is not None:
        y = res + y
    return y


def rms_norm(x, weight, eps=1e-6):
    variance = x.to(torch.float32).pow(2).mean(-1, keepdim=True)
    return (x * torch.rsqrt(variance + eps)).to(weight.dtype) * weight


def rope(x, freqs):
    """x: (B, S, H, D); freqs: (S, D/2) complex64."""
    pairs = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
    return torch.view_as_real(pairs * freqs.unsqueeze(1)).flatten(3).type_as(x)


def qk_rmsnorm_rope(q, k, wq, wk, freqs, eps=1e-6):
    return rope(rms_norm(q, wq, eps), freqs), rope(rms_norm(k, wk, eps), freqs)


def swiglu(g, v):
    return F.silu(g) * v


def gated_residual(h, x, gate):
    return h + gate * x


def mx_quantize(x):
    """bf16 (M, K) -> (codes (Mp, K) uint8, swizzled E8M0 bytes)."""
    m, k = x.shape
    mp = (m + 127) // 128 * 128
    xp = torch.zeros(mp, k, dtype=torch.float32)
    xp[:m] = x.float()
    blocks = xp.view(mp, k // 32, 32)
    amax = blocks.abs().amax(-1)
    bits = amax.view(torch.int32)
    e = ((bits >> 23) & 0xFF) - 8 + ((bits & 0x7FFFFF) > 0x600000).int()
    e = torch.where(amax == 0, torch.zeros_like(e), e.clamp(0, 254))
    codes = (blocks * torch.exp2((127 - e).float())[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
    swz = e.to(torch.uint8).view(mp // 128, 4, 32, k // 128, 4).permute(0, 3, 2, 1, 4).reshape(-1)
    return codes.view(mp, k), swz


def mx_dequantize(codes, scales):
    mp, k = codes.shape
    e = scales.view(mp // 128, k // 128, 32, 4, 4).permute(0, 3, 2, 1, 4).reshape(mp, k // 32)
    vals = codes.view(torch.float8_e4m3fn).float().view(mp, k // 32, 32)
    return (vals * torch.exp2(e.float() - 127)[..., None]).view(mp, k)


def mx_matmul(a, w, rows, bias=None):
    """a, w: (codes, scales) of (Mp, K) and (N, K); -> bf16 (rows, N)."""
    y = mx_dequantize(*a)[:rows] @ mx_dequantize(*w).t()
    if bias is not None:
        y = y + bias.float()
    return y.to(torch.bfloat16)


def interleave_gate_up(gate, up, group=32):
    f, k = gate.shape
    return torch.stack([gate.reshape(f // group, group, k), up.reshape(f // group, group, k)], 1).reshape(2 * f, k)


def block(h, mod, freqs, wq, norm_q, norm_k, heads, eps=1e-6):
    """h: (B, S, D) bf16; mod: (B, 6, D) rows (shift1, scale1, gate1, shift2,
    scale2, gate2); wq: quantized weights {"qkv", "out", "gate_up", "down"}
    as (codes, scales) with gate/up interleaved; norm_q, norm_k: (128,)."""
    b, s, d = h.shape
    m = b * s
    shift1, scale1, g1, shift2, scale2, g2 = mod[:, :, None].unbind(1)
    gate1, gate2 = g1.tanh(), g2.tanh()
    x = adaln(h, scale1, shift1, eps=eps)
    qkv = mx_matmul(mx_quantize(x.reshape(m, d)), wq["qkv"], m).view(b, s, 3, heads, d // heads)
    q, k = qk_rmsnorm_rope(qkv[:, :, 0], qkv[:, :, 1], norm_q, norm_k, freqs, eps)  # q, k: the attention's inputs
    v = qkv[:, :, 2].reshape(m, d)                                                   # stand-in o = v
    h1 = gated_residual(h, mx_matmul(mx_quantize(v), wq["out"], m).view(b, s, d), gate1)
    x2 = adaln(h1, scale2, shift2, eps=eps)
    acc = mx_dequantize(*mx_quantize(x2.reshape(m, d)))[:m] @ mx_dequantize(*wq["gate_up"]).t()
    pairs = acc.to(torch.bfloat16).view(m, -1, 2, 32)
    act = swiglu(pairs[:, :, 0].reshape(m, -1), pairs[:, :, 1].reshape(m, -1))
    down = mx_matmul(mx_quantize(act), wq["down"], m).view(b, s, d)
    return gated_residual(h1, down, gate2), (q, k)
