"""The MMDiT block (MMDiTBlock.forward) equals, bit for bit, the same block
composed of the unfused library ops: the GEMMs with plain bf16 outputs, then
qim_qk_norm_rope_pack, qim_attention + qim_mx_quantize, qim_gated_residual and
qim_swiglu_quantize as separate passes.  Each fused epilogue is held to its
unfused op by its own test, and each op to the oracle; this test checks the
wiring between them (which modulation row feeds which step, which residual
each gated add takes, the SwiGLU weight interleave), with the attention core
run as qim_attention + quantize, as qim_attention_mxfp8, or with V^T written
by the QKV projection (fused_attention).
"""
import pytest
import torch

from qwen_image_accel import rope
from qwen_image_accel.block import MMDiTBlock, _LayerNorm
from qwen_image_accel.kernels import attention, elementwise, gemm, mxfp8
from qwen_image_accel.kernels.epilogue import layer_norm_scale_quantize, swiglu_quantize
from tests.helpers import bf16_randn

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def unfused_block(blk, h, mod, freqs):
    b, s, d = h.shape
    hd = d // blk.heads
    shift1, scale1, g1, shift2, scale2, g2 = (mod[:, i:i + 1] for i in range(6))
    gate1 = elementwise.modulation_values(g1.contiguous(), (elementwise.MOD_TANH,))[0].unsqueeze(1)
    gate2 = elementwise.modulation_values(g2.contiguous(), (elementwise.MOD_TANH,))[0].unsqueeze(1)
    norm = _LayerNorm(d, blk.eps)

    def mm(x, w):
        return gemm.mx_matmul(x, w.values, w.scales, weight_tiled=True)

    x = layer_norm_scale_quantize(h, scale1.contiguous(), norm, shift=shift1.contiguous(), add_one=True, tiled=True)
    qkv = mm(x, blk.w_qkv).view(b, s, 3 * d)
    q, k = attention.qk_norm_rope(qkv[:, :, :d].unflatten(-1, (blk.heads, hd)),
                                  qkv[:, :, d:2 * d].unflatten(-1, (blk.heads, hd)),
                                  blk.norm_q, blk.norm_k, freqs, blk.eps, blk.eps)
    v = qkv[:, :, 2 * d:].unflatten(-1, (blk.heads, hd))
    o = attention.attention(q, k, v)
    h1 = elementwise.residual(h, mm(mxfp8.quantize(o.reshape(b * s, d), tiled=True), blk.w_out).view(b, s, d),
                              gate1)
    x2 = layer_norm_scale_quantize(h1, scale2.contiguous(), norm, shift=shift2.contiguous(), add_one=True,
                                   tiled=True)
    gu = mm(x2, blk.w_gate_up).view(b * s, -1, 2, 32)  # gate/up rows interleaved in groups of 32
    a = swiglu_quantize(gu[:, :, 0].reshape(b * s, -1), gu[:, :, 1].reshape(b * s, -1), tiled=True)
    return elementwise.residual(h1, mm(a, blk.w_down).view(b, s, d), gate2)


@pytest.mark.parametrize("b,side", [(1, 16), (2, 8)])
def test_block_equals_unfused_composition(dev, b, side):
    g = torch.Generator().manual_seed(100 + b)
    dim, heads, ffn = 512, 4, 1024
    s = 256 + side * side
    say("block", b, s, dim, heads, ffn)
    blk = MMDiTBlock.random(g, dim=dim, heads=heads, ffn=ffn, device=dev)
    h = bf16_randn(g, (b, s, dim)).to(dev)
    mod = bf16_randn(g, (b, 6, dim), 0.5).to(dev)
    freqs = rope.image_table(256, side, side, dev)
    ref = unfused_block(blk, h, mod, freqs)
    got = blk.forward(h, mod, freqs, attention_fn=attention.attention)
    got8 = blk.forward(h, mod, freqs, attention_mxfp8_fn=attention.attention_mxfp8)
    gotf = blk.forward(h, mod, freqs, fused_attention=True)
    torch.cuda.synchronize()
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got, ref)
    assert torch.equal(got8, ref)
    assert torch.equal(gotf, ref)
