"""Write the golden fixtures of the hot path: tests/golden/golden.npz.

The reference commits no golden vectors (its GPU checks are generative,
tests/gpu/check_*.py), so the fixtures are made here from seeded inputs with
two independent evaluations of the reference's eager semantics:

  * ``<op>_oracle``: the C oracle (oracle/qim_oracle.c), the checker the GPU
    tests use, with the exact rounding points of the reference;
  * ``<op>_eager``: the reference's eager PyTorch composition evaluated with
    torch's CPU library routines (F.layer_norm, F.silu, the complex multiply
    of apply_rotary_emb_qwen, the float8_e4m3fn cast of ref_quant in
    tests/gpu/check_mxfp8.py:20-30).

Inputs follow the reference checks' recipes: seeds 0, 1, 91, 717, 721, odd row
counts, padding, outliers x40 and magnitude sweeps.  Sizes are small (the file
is ~0.5 MB).  Re-run after changing the oracle:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def randn(g, shape, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def eager_quant(x):
    """tests/gpu/check_mxfp8.py:20-34 (ref_quant + swizzle) in torch CPU ops."""
    m, k = x.shape
    mp = (m + 127) // 128 * 128
    xp = torch.zeros(mp, k, dtype=torch.bfloat16)
    xp[:m] = x
    xv = xp.float().view(mp, k // 32, 32)
    amax = xv.abs().amax(-1)
    b = amax.view(torch.int32)
    e = ((b >> 23) & 0xFF) - 8 + ((b & 0x7FFFFF) > 6291456).int()
    e = torch.where(amax == 0, torch.zeros_like(e), e.clamp(0, 254))
    q = (xv * torch.exp2((127 - e).float())[..., None]).to(torch.float8_e4m3fn)
    sw = e.to(torch.uint8).view(mp // 128, 4, 32, k // 128, 4).permute(0, 3, 2, 1, 4).reshape(-1)
    return q.view(torch.uint8).view(mp, k).numpy(), sw.numpy()


def main():
    out = {}
    # MXFP8 quantize: odd rows, padding, outliers, a tiny row (check_mxfp8.py:38-50)
    g = torch.Generator().manual_seed(0)
    for m, k in ((77, 256), (130, 256), (1, 128)):
        x = randn(g, (m, k))
        x[:, ::64] *= 40
        if m > 100:
            x[m // 3] *= 1e-3
        q, s = O.mx_quantize(bits(x))
        eq, es = eager_quant(x)
        tag = f"quant_{m}x{k}"
        out[f"{tag}_x"] = bits(x)
        out[f"{tag}_q_oracle"], out[f"{tag}_s_oracle"] = q, s
        out[f"{tag}_q_eager"], out[f"{tag}_s_eager"] = eq, es

    # layer_norm_scale (check_layernorm_ops.py:13-22, seed 717) and config-1 chain
    g = torch.Generator().manual_seed(717)
    for mag in (0.001, 1.0, 20.0):
        x = randn(g, (2, 9, 512), mag)
        s = randn(g, (2, 1, 512))
        tag = f"ln_{mag:g}"
        out[f"{tag}_x"], out[f"{tag}_scale"] = bits(x), bits(s)
        out[f"{tag}_oracle"] = O.adaln(bits(x), bits(s))
        out[f"{tag}_eager"] = bits(F.layer_norm(x, (512,), eps=1e-6) * s)
    x, res = randn(g, (1, 16, 512)), randn(g, (1, 16, 512))
    shift, scale, gate = (randn(g, (1, 1, 512), 0.1) for _ in range(3))
    out["adaln_x"], out["adaln_res"] = bits(x), bits(res)
    out["adaln_shift"], out["adaln_scale"], out["adaln_gate"] = bits(shift), bits(scale), bits(gate)
    out["adaln_oracle"] = O.adaln(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True)
    out["adaln_eager"] = bits(res + gate * ((1 + scale) * F.layer_norm(x, (512,), eps=1e-6) + shift))
    q, s = O.adaln_quantize(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True)
    out["adaln_q_oracle"], out["adaln_s_oracle"] = q, s

    # gated residual and SwiGLU (check_fused.py seed 91)
    g = torch.Generator().manual_seed(91)
    h, x = randn(g, (2, 57, 256)), randn(g, (2, 57, 256))
    gt = randn(g, (2, 1, 256)).tanh()
    out["res_h"], out["res_x"], out["res_gate"] = bits(h), bits(x), bits(gt)
    out["res_oracle"] = O.residual(bits(h), bits(x), bits(gt))
    out["res_eager"] = bits(h + gt * x)
    a, v = randn(g, (77, 256), 3.0), randn(g, (77, 256))
    out["swiglu_g"], out["swiglu_v"] = bits(a), bits(v)
    out["swiglu_oracle"] = O.swiglu(bits(a), bits(v))
    out["swiglu_eager"] = bits(F.silu(a) * v)
    q, s = O.swiglu_quantize(bits(a), bits(v))
    out["swiglu_q_oracle"], out["swiglu_s_oracle"] = q, s

    # RMSNorm + RoPE + prefix pack (check_attention_ops.py seed 721)
    g = torch.Generator().manual_seed(721)
    B, S, P, H, D = 2, 9, 5, 2, 128
    q, k, v = (randn(g, (B, S, H, D)) for _ in range(3))
    ck, cv = randn(g, (B, P, H, D)), randn(g, (B, P, H, D))
    wq = (torch.rand(D, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    wk = (torch.rand(D, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    phase = torch.randn(S, D // 2, generator=g)
    freqs = torch.polar(torch.ones_like(phase), phase)
    f = torch.view_as_real(freqs).numpy()
    for n, t in (("q", q), ("k", k), ("v", v), ("ck", ck), ("cv", cv), ("wq", wq), ("wk", wk)):
        out[f"attn_{n}"] = bits(t)
    out["attn_freqs"] = f
    oq, ok, ov = O.norm_rope_pack(bits(q), bits(k), bits(v), bits(wq), bits(wk), f, bits(ck), bits(cv))
    out["attn_oq_oracle"], out["attn_ok_oracle"], out["attn_ov_oracle"] = oq, ok, ov

    def rms(x, w):
        var = x.float().pow(2).mean(-1, keepdim=True)
        return (x * torch.rsqrt(var + 1e-6)).to(torch.bfloat16) * w

    def rope(x):
        xr = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
        return torch.view_as_real(xr * freqs.unsqueeze(1)).flatten(3).type_as(x)

    out["attn_oq_eager"] = bits(rope(rms(q, wq)))
    out["attn_ok_eager"] = bits(torch.cat([ck, rope(rms(k, wk))], 1))
    out["rope_oq_oracle"], out["rope_ok_oracle"] = O.rope(bits(q), bits(k), f)
    out["rope_oq_eager"], out["rope_ok_eager"] = bits(rope(q)), bits(rope(k))

    # 3-axis RoPE table: 4 text tokens + one 6x6 image
    pos = O.rope_positions(4, 1, 6, 6)
    out["freqs_pos"], out["freqs_oracle"] = pos, O.rope_freqs(pos)

    # MXFP8 GEMM (+bias) on a small problem (seed 1)
    g = torch.Generator().manual_seed(1)
    a, w = randn(g, (100, 128)), randn(g, (256, 128), 0.02)
    bias = randn(g, (256,), 0.01)
    aq, as_ = O.mx_quantize(bits(a))
    wq8, ws8 = O.mx_quantize(bits(w))
    out["gemm_a"], out["gemm_w"], out["gemm_bias"] = bits(a), bits(w), bits(bias)
    acc = O.mx_gemm(aq, as_, wq8, ws8)[:100]
    out["gemm_acc_oracle"] = acc
    out["gemm_eager"] = (O.mx_dequantize(aq, as_, 100).astype(np.float64)
                         @ O.mx_dequantize(wq8, ws8).astype(np.float64).T).astype(np.float32)

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes,", len(out), "arrays")


if __name__ == "__main__":
    main()
