"""The MMDiT block (MMDiTBlock.forward: hidden 3072, 24 x
128 heads, FFN 12288, the attention core replaced by the stand-in o = v)
against the CPU oracle at its own sizes, M = 16640 (2048^2) and 4352
(1024^2), on sampled token rows.

The reference composes this block in optimizations/quantized_decode.py:
117-135.  Every step is local to a token row, so the oracle computes the
sampled rows only (oracle/block.py, rows=).  Each stage is checked on those
rows:
  - bit-exact where the HIP stage and the oracle start from the same input:
    the MXFP8 weights, LN1 -> MXFP8 (from h), the stand-in's MXFP8 (from the
    HIP V columns), LN2 -> MXFP8 (from the HIP h1);
  - rel-Frobenius <= 1e-2 where a GEMM feeds the stage, with the oracle fed
    the HIP stage's own input (QKV from the bit-exact x1; h1 from the HIP V;
    the SwiGLU -> MXFP8 activation from the HIP x2; h2 from the HIP
    activation and h1).
The residual stages are compared on their update (h1 - h, h2 - h1), so the
bar applies to the part the GEMM produced.

The whole block from h alone is held to 3e-2 instead: there the GEMMs'
accumulation differences (~2e-4 relative, the scaled MFMA's) reach three
requantizations (V, LN2's input h1, the SwiGLU activation), where they flip
the E4M3 code of the ~0.5 % of elements that sit that close to a rounding
boundary, each flip one code step (6-12 % of the element).  The oracle's own
block with 2.2e-4 relative noise added to its GEMM outputs moves by 2e-2 in
this measure (D 3072, F 12288, 64 rows); the kernels measure ~1.2e-2.
Rows: the first and last,
rows of the last 256-row tile row (the GEMM's quarter-tile tail at these
shapes) and random rows.
"""
import numpy as np
import pytest
import torch

from oracle import block as OB
from oracle import oracle as O
from qwen_image_accel.block import MMDiTBlock
from qwen_image_accel.kernels import mxfp8
from tests.helpers import (bf16_randn, bf16_values, bits, pack_quantized, quantized_rows, rel_fro,
                           unswizzle_scales)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def sample_rows(m, n=64, seed=0):
    rng = np.random.default_rng(seed)
    tail = np.arange(max(0, (m - 1) // 256 * 256), m)
    picks = [0, m - 1] + list(rng.choice(tail, min(8, tail.size), replace=False))
    rest = rng.choice(m, n, replace=False)
    return np.unique(np.concatenate([picks, rest]))[:n].astype(np.int64)


def update_err(new, old, ref_new):
    """rel-Frobenius of the residual update new - old against ref_new - old."""
    old = bf16_values(old).astype(np.float64)
    return rel_fro(bf16_values(new) - old, bf16_values(ref_new) - old)


def assert_quantized_rows_equal(hip, rows, ref_codes, ref_scales, what):
    """HIP Quantized rows vs an oracle quantization of exactly those rows."""
    codes, exps = quantized_rows(hip, rows)
    n, k = codes.shape
    ref_exps = unswizzle_scales(ref_scales, ref_codes.shape[0], k)[:n]
    assert np.array_equal(exps, ref_exps), f"{what}: scales differ"
    bad = codes != ref_codes[:n]
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} codes differ"


def assert_weight_equal(hip, ref, what):
    rm = mxfp8.as_row_major(hip)
    assert np.array_equal(rm.values.view(torch.uint8).cpu().numpy(), ref[0]), what
    assert np.array_equal(rm.scales.view(torch.uint8).cpu().numpy(), ref[1]), what


@pytest.mark.parametrize("b,s,dim,heads", [(1, 4352, 3072, 24), (1, 16640, 3072, 24), (1, 4352, 4096, 32)])
def test_block_config5_against_oracle(dev, b, s, dim, heads):
    """Config 5's block (D 3072, 24 heads) at 1024^2 and 2048^2, and the
    reference model's own width (D 4096 = 32 heads x 128, FFN 12288) at
    1024^2."""
    ffn = 12288
    side = int(round((s - 256) ** 0.5))
    say("block vs oracle", b, s, dim, heads, ffn)
    g = torch.Generator().manual_seed(42)
    blk = MMDiTBlock.random(g, dim=dim, heads=heads, ffn=ffn, device=dev)
    h = bf16_randn(g, (b, s, dim))
    mod = bf16_randn(g, (b, 6, dim), 0.1)
    f = O.rope_freqs(O.rope_positions(256, 1, side, side))
    freqs = torch.view_as_complex(torch.from_numpy(f))
    stages = {}
    out = blk.forward(h.to(dev), mod.to(dev), freqs.to(dev), stages=stages)
    torch.cuda.synchronize()

    m = b * s
    rows = sample_rows(m, seed=s)
    rt = torch.as_tensor(rows, device=dev)
    n = rows.size
    wb = {k: bits(v.cpu()) for k, v in blk.bf16_weights.items()}
    wq = OB.quantize_weights(wb)
    for name, hip in (("qkv", blk.w_qkv), ("out", blk.w_out), ("gate_up", blk.w_gate_up), ("down", blk.w_down)):
        assert_weight_equal(hip, wq[name], f"weight {name}")
    hb, mb = bits(h), bits(mod)
    bid = rows // s
    ref_out, st = OB.block_forward(hb, mb, f, wb, heads, rows=rows, wq=wq, return_stages=True)
    hs = hb.reshape(m, dim)[rows]
    shift1, scale1, g1, shift2, scale2, g2 = (mb[:, i] for i in range(6))
    gate1, gate2 = OB.tanh_bf16(g1), OB.tanh_bf16(g2)

    # LN1 -> MXFP8 from the same h: bit-exact.
    assert_quantized_rows_equal(stages["x1"], rows, *st["x1"], "x1")
    # QKV projection on the same x1 codes: V columns, and Q/K after norm + RoPE.
    qkv = bits(stages["qkv"][rt])
    err_v = rel_fro(bf16_values(qkv[:, 2 * dim:]), bf16_values(st["v"]))
    err_q = rel_fro(bf16_values(qkv[:, :dim]), bf16_values(st["q"]))
    err_k = rel_fro(bf16_values(qkv[:, dim:2 * dim]), bf16_values(st["k"]))
    # The stand-in's MXFP8 (from the HIP V columns): bit-exact.
    v_hip = np.ascontiguousarray(qkv[:, 2 * dim:])
    vq = O.mx_quantize(v_hip)
    assert_quantized_rows_equal(stages["o"], rows, *vq, "o")
    # h1 = h + tanh(g1) * (MXFP8(v) @ W_out), oracle fed the HIP V.
    h1 = bits(stages["h1"].reshape(m, dim)[rt])
    h1_ref = OB.gated_residual(hs, OB.gemm_bf16(*vq, wq["out"], n), bid, gate1)
    err_h1 = update_err(h1, hs, h1_ref)
    # LN2 -> MXFP8 from the same h1: bit-exact.
    x2q = OB.modulate_quantize(h1, bid, scale2, shift2, 1e-6)
    assert_quantized_rows_equal(stages["x2"], rows, *x2q, "x2")
    # SwiGLU -> MXFP8 out of the gate/up GEMM on the same x2 codes.
    accg, accu = OB.split_gate_up(O.mx_gemm(*x2q, *wq["gate_up"])[:n])
    aq_ref = O.swiglu_quantize(O.f32_to_bf16(accg), O.f32_to_bf16(accu))
    a_codes, a_exps = quantized_rows(stages["a"], rows)
    a_hip = pack_quantized(a_codes, a_exps)
    err_a = rel_fro(O.mx_dequantize(*a_hip, rows=n), O.mx_dequantize(*aq_ref, rows=n))
    # h2 = h1 + tanh(g2) * (a @ W_down), oracle fed the HIP activation.
    h2 = bits(out.reshape(m, dim)[rt])
    h2_ref = OB.gated_residual(h1, OB.gemm_bf16(*a_hip, wq["down"], n), bid, gate2)
    err_h2 = update_err(h2, h1, h2_ref)
    # The whole block from h alone.
    err_block = update_err(h2, hs, ref_out)
    errs = dict(v=err_v, q=err_q, k=err_k, h1=err_h1, a=err_a, h2=err_h2, block=err_block)
    print("[errs]", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert all(np.isfinite(list(errs.values())))
    for k, v in errs.items():
        assert v < (3e-2 if k == "block" else 1e-2), (k, v)
