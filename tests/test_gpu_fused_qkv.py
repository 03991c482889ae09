"""The QKV projection with QK-RMSNorm + RoPE fused into the GEMM epilogue
(qim_mxfp8_gemm_qk_norm_rope) equals, bit for bit, the unfused path: the GEMM
(bf16 output) followed by qim_qk_norm_rope_pack on its Q and K columns, V
unchanged.  Both sides use the same per-head arithmetic; the fused side reduces
a head row inside one wave (whole tiles) or across two waves through LDS
(quarter tiles of the partial last round: 612 tiles at M = 4352, H = 24), so
these shapes cover both, plus padding rows (M = 4200) and two batches (seq <
M, the RoPE row is row % seq).  The unfused path is held to the oracle by
test_gpu_kernels.py, and the fused output directly to the oracle's norm +
RoPE (oracle.norm_rope_pack) applied to the plain GEMM's bf16 Q/K columns.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qwen_image_accel.kernels import attention, gemm, mxfp8
from tests.helpers import bf16_randn, bits

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("m,heads,k,seq", [(300, 4, 256, 150), (4352, 24, 256, 2176), (4200, 24, 384, 4200)])
def test_qkv_gemm_with_qk_norm_rope_epilogue(dev, m, heads, k, seq):
    g = torch.Generator().manual_seed(m + heads + k)
    d = heads * 128
    a = bf16_randn(g, (m, k)).to(dev)
    w = bf16_randn(g, (3 * d, k), 0.05).to(dev)
    wq = (torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16).to(dev)
    wk = (torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16).to(dev)
    ang = torch.rand(seq, 64, generator=g, dtype=torch.float64) * 6.283185307179586
    freqs = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(dev)
    b = m // seq
    for tiled in (False, True):
        say("fused qkv", m, heads, k, seq, "tiled" if tiled else "row-major")
        aq = mxfp8.quantize(a, tiled=tiled)
        w8 = mxfp8.quantize(w, tiled=tiled)
        fused = gemm.mx_matmul_qk_norm_rope(aq, w8.values, w8.scales, wq, wk, freqs, heads, seq, 1e-6, 1e-5,
                                            weight_tiled=tiled)
        plain = gemm.mx_matmul(aq, w8.values, w8.scales, weight_tiled=tiled)
        qkv = plain.view(b, seq, 3 * d)
        q = qkv[:, :, :d].unflatten(-1, (heads, 128))
        kk = qkv[:, :, d:2 * d].unflatten(-1, (heads, 128))
        oq, ok = attention.qk_norm_rope(q, kk, wq, wk, freqs, 1e-6, 1e-5)
        torch.cuda.synchronize()
        as16 = lambda t: t.contiguous().view(torch.int16)  # noqa: E731
        assert torch.equal(as16(fused[:, :d]), as16(oq.reshape(m, d))), "Q"
        assert torch.equal(as16(fused[:, d:2 * d]), as16(ok.reshape(m, d))), "K"
        assert torch.equal(as16(fused[:, 2 * d:]), as16(plain[:, 2 * d:])), "V"
        # and the oracle's norm + RoPE of the plain GEMM's bf16 Q/K columns
        pb = bits(plain).reshape(b, seq, 3, heads, 128)
        rq, rk, _ = O.norm_rope_pack(pb[:, :, 0], pb[:, :, 1], pb[:, :, 0], bits(wq), bits(wk),
                                     torch.view_as_real(freqs).cpu().numpy(), epsq=1e-6, epsk=1e-5)
        fb = bits(fused).reshape(b, seq, 3, heads, 128)
        assert np.array_equal(fb[:, :, 0], rq), "Q vs oracle"
        assert np.array_equal(fb[:, :, 1], rk), "K vs oracle"


def test_qkv_gemm_rejects_odd_heads(dev):
    from qwen_image_accel import _native
    g = torch.Generator().manual_seed(1)
    aq = mxfp8.quantize(bf16_randn(g, (128, 128)).to(dev))
    w8 = mxfp8.quantize(bf16_randn(g, (3 * 3 * 128, 128)).to(dev))
    wq = torch.ones(128, dtype=torch.bfloat16, device=dev)
    freqs = torch.ones(128, 64, dtype=torch.complex64, device=dev)
    with pytest.raises(_native.Unsupported):
        gemm.mx_matmul_qk_norm_rope(aq, w8.values, w8.scales, wq, wq, freqs, 3, 128)


# 4352 x 24 heads: 612 tiles, whole tiles then quarter tiles (two waves per
# head); 2 x 320 rows: quarter tiles only, two batches.
@pytest.mark.parametrize("m,heads,k,seq", [(4352, 24, 256, 4352), (640, 4, 256, 320)])
def test_qkv_gemm_writes_attention_vt(dev, m, heads, k, seq):
    """qim_mxfp8_gemm_qk_norm_rope_vt: the V columns leave as the attention's
    V^T tiles.  Attention from those tiles (v = None) equals attention on the
    plain projection's V, bit for bit, and the Q/K columns are unchanged."""
    say("qkv vt", m, heads, k, seq)
    g = torch.Generator().manual_seed(m + heads)
    d = heads * 128
    a = bf16_randn(g, (m, k)).to(dev)
    w = bf16_randn(g, (3 * d, k), 0.05).to(dev)
    wq = (torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16).to(dev)
    wk = (torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16).to(dev)
    ang = torch.rand(seq, 64, generator=g, dtype=torch.float64) * 6.283185307179586
    freqs = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(dev)
    b = m // seq
    aq = mxfp8.quantize(a, tiled=True)
    w8 = mxfp8.quantize(w, tiled=True)
    plain = gemm.mx_matmul_qk_norm_rope(aq, w8.values, w8.scales, wq, wk, freqs, heads, seq, weight_tiled=True)
    ws = attention.workspace(b, seq, seq, heads, dev)
    ws.fill_(0xff)
    fused = gemm.mx_matmul_qk_norm_rope(aq, w8.values, w8.scales, wq, wk, freqs, heads, seq, weight_tiled=True,
                                        vt=ws)
    assert torch.equal(fused[:, :2 * d], plain[:, :2 * d])
    q, k_, v = (plain.view(b, seq, 3 * d)[:, :, i * d:(i + 1) * d].unflatten(-1, (heads, 128)) for i in range(3))
    ref = attention.attention(q, k_, v)
    got = attention.attention(q, k_, None, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
