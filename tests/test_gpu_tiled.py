"""Kernels that write or read the GEMM's tiled code layout, held bit-for-bit to
their row-major forms (the layout moves bytes, never values):

- quantize / layer_norm_scale_quantize / swiglu_quantize with ``tiled=True``
  write ``tile_codes`` of the row-major codes and the same scales;
- the GEMM with tiled A and/or B returns bit-identical outputs for every
  epilogue (same products in the same order; only DMA source addresses
  differ), and its quantized SwiGLU epilogue writes ``tile_codes`` of the
  row-major codes with ``out_tiled``;
- ``MXFP8Linear`` keeps its weight tiled, shows the reference's ``weight_fp8``
  view, and loads a reference state dict.

The row-major paths are themselves held to the oracle by test_gpu_kernels.py.
Shapes cover a padded row count with a 128-row last super-block (M = 300 ->
384, 4200 -> 4224) and the quarter-tile tail of the GEMM (272 tiles).
"""
import numpy as np
import pytest
import torch

from qwen_image_accel.kernels import epilogue, gemm, mxfp8
from qwen_image_accel.optimizations.mxfp8 import MXFP8Linear
from tests.helpers import bf16_randn

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def assert_tiled_form(tiled, rowmajor):
    assert tiled.tiled and not rowmajor.tiled
    assert tiled.rows == rowmajor.rows and tiled.shape == rowmajor.shape
    assert tiled.values.shape == rowmajor.values.shape
    assert np.array_equal(u8(tiled.values), u8(mxfp8.tile_codes(rowmajor.values)))
    assert np.array_equal(u8(tiled.scales), u8(rowmajor.scales))


@pytest.mark.parametrize("m,k", [(1, 128), (300, 384), (512, 3072), (4200, 256)])
def test_quantize_tiled(dev, m, k):
    say("quantize tiled", m, k)
    x = bf16_randn(torch.Generator().manual_seed(m + k), (m, k)).to(dev)
    assert_tiled_form(mxfp8.quantize(x, tiled=True), mxfp8.quantize(x))


@pytest.mark.parametrize("seq,d", [(300, 3072), (128, 256)])
def test_layer_norm_scale_quantize_tiled(dev, seq, d):
    say("adaln quantize tiled", seq, d)
    g = torch.Generator().manual_seed(seq)
    x = bf16_randn(g, (2, seq, d)).to(dev)
    scale, shift, gate = (bf16_randn(g, (2, 1, d), 0.1).to(dev) for _ in range(3))
    res = bf16_randn(g, (2, seq, d)).to(dev)
    norm = torch.nn.LayerNorm(d, eps=1e-6, elementwise_affine=False)
    kw = dict(shift=shift, gate=gate, residual=res, add_one=True)
    assert_tiled_form(epilogue.layer_norm_scale_quantize(x, scale, norm, tiled=True, **kw),
                      epilogue.layer_norm_scale_quantize(x, scale, norm, **kw))


def test_swiglu_quantize_tiled(dev):
    say("swiglu quantize tiled", 300, 512)
    gv = bf16_randn(torch.Generator().manual_seed(5), (300, 1024)).to(dev)
    gate, value = gv[:, :512], gv[:, 512:]
    assert_tiled_form(epilogue.swiglu_quantize(gate, value, tiled=True),
                      epilogue.swiglu_quantize(gate, value))


EPILOGUES = ["none", "bias", "gated_residual", "swiglu", "swiglu_quant"]


@pytest.mark.parametrize("m,n,k", [(300, 512, 256), (4352, 4096, 512), (4200, 4096, 384)])
def test_gemm_tiled_operands_bit_identical(dev, m, n, k):
    g = torch.Generator().manual_seed(m + n + k)
    a = bf16_randn(g, (m, k)).to(dev)
    w = bf16_randn(g, (n, k), 0.05).to(dev)
    aq, wq = mxfp8.quantize(a), mxfp8.quantize(w)
    at, wt = mxfp8.quantize(a, tiled=True), mxfp8.quantize(w, tiled=True)
    extra = {
        "bias": dict(bias=bf16_randn(g, (n,), 0.01).to(dev)),
        "gated_residual": dict(residual=bf16_randn(g, (m, n)).to(dev),
                               gate=bf16_randn(g, (2, 1, n)).tanh().to(dev), seq=(m + 1) // 2),
    }
    for epi in EPILOGUES:
        kw = extra.get(epi, {})
        say("gemm tiled", m, n, k, epi)
        want = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue=epi, **kw)
        for a_op, w_op, w_tiled in ((at, wq, False), (aq, wt, True), (at, wt, True)):
            got = gemm.mx_matmul(a_op, w_op.values, w_op.scales, epilogue=epi, weight_tiled=w_tiled, **kw)
            if epi == "swiglu_quant":
                assert not got.tiled
                assert np.array_equal(u8(got.values), u8(want.values))
                assert np.array_equal(u8(got.scales), u8(want.scales))
                got_t = gemm.mx_matmul(a_op, w_op.values, w_op.scales, epilogue=epi, weight_tiled=w_tiled,
                                       out_tiled=True)
                assert_tiled_form(got_t, want)
            else:
                assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (epi, a_op.tiled, w_tiled)


def test_mxfp8_linear_tiled_weight_and_reference_state_dict(dev):
    say("MXFP8Linear tiled weight")
    g = torch.Generator().manual_seed(11)
    lin = torch.nn.Linear(384, 512, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(512, 384, generator=g) * 0.02)
    lin = lin.to(dev, torch.bfloat16)
    mx = MXFP8Linear(lin)
    rowmajor = mxfp8.quantize(lin.weight.detach().contiguous())
    assert np.array_equal(u8(mx.weight_tiled), u8(mxfp8.tile_codes(rowmajor.values)))
    view = mx.weight_fp8
    assert view.shape == (384, 512) and view.t().is_contiguous()
    assert np.array_equal(u8(view.t()), u8(rowmajor.values))
    # A state dict in the reference's form (weight_fp8 = (K, N) view of row-major codes).
    fresh = MXFP8Linear(torch.nn.Linear(384, 512, bias=False).to(dev, torch.bfloat16))
    fresh.load_state_dict({"weight_fp8": rowmajor.values.t(), "weight_scale": rowmajor.scales})
    assert np.array_equal(u8(fresh.weight_tiled), u8(mx.weight_tiled))
    x = bf16_randn(g, (2, 100, 384)).to(dev)
    want = gemm.mx_matmul(mxfp8.quantize(x.reshape(200, 384)), rowmajor.values, rowmajor.scales)
    assert torch.equal(fresh(x).reshape(200, 512).view(torch.int16), want.view(torch.int16))
    assert torch.equal(mx(x).reshape(200, 512).view(torch.int16), want.view(torch.int16))


def test_mxfp8_linear_n_multiple_of_128_and_out_dtype(dev):
    """A 384-output linear (N % 256 == 128, converted as in the reference):
    forward equals the row-major GEMM on the same bytes; its state dict (the
    reference's keys) reloads byte for byte; matmul honours dtype."""
    say("MXFP8Linear N=384")
    g = torch.Generator().manual_seed(12)
    lin = torch.nn.Linear(256, 384, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(384, 256, generator=g) * 0.05)
    lin = lin.to(dev, torch.bfloat16)
    mx = MXFP8Linear(lin)
    x = bf16_randn(g, (3, 70, 256)).to(dev)
    rowmajor = mxfp8.quantize(lin.weight.detach().contiguous())
    a = mxfp8.quantize(x.reshape(210, 256))
    want = gemm.mx_matmul(a, rowmajor.values, rowmajor.scales)
    got = mx(x)
    assert got.shape == (3, 70, 384)
    assert torch.equal(got.reshape(210, 384).view(torch.int16), want.view(torch.int16))
    fresh = MXFP8Linear(torch.nn.Linear(256, 384, bias=False).to(dev, torch.bfloat16))
    fresh.load_state_dict({k: v.contiguous() for k, v in mx.state_dict().items()})
    assert np.array_equal(u8(fresh.weight_tiled), u8(mx.weight_tiled))
    y32 = mx.matmul(a, torch.float32)
    assert y32.dtype == torch.float32
    assert torch.equal(y32.to(torch.bfloat16).view(torch.int16), want.view(torch.int16))
