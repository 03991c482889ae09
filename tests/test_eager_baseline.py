"""The eager torch-CPU restatement (oracle/eager_torch.py, bench.py's CPU
baseline) against the C oracle on the same seeded inputs (CPU only).

Bars: bit-exact where both sides round the same values once (the gated
residual, the MXFP8 bytes); the bf16 chain tolerance where torch reduces in
fp32 and the oracle in float64 (LayerNorm, RMSNorm); 1 ulp for SiLU (torch's
CPU exp against expf); rel-Frobenius for the GEMM (fp32 against float64
accumulation) and for the block (whose requantizations turn those last-bit
differences into a few E4M3 code steps).
"""
import numpy as np
import torch

from oracle import block as OB
from oracle import eager_torch as E
from oracle import oracle as O
from tests.helpers import bf16_close, bf16_close_chain, bf16_randn, bf16_values, bits, rel_fro


def test_adaln_config1_chain():
    g = torch.Generator().manual_seed(717)
    x, res = bf16_randn(g, (1, 256, 3072)), bf16_randn(g, (1, 256, 3072))
    shift, scale, gate = (bf16_randn(g, (1, 1, 3072), 0.1) for _ in range(3))
    got = E.adaln(x, scale, shift, gate, res)
    ref = O.adaln(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True)
    ok, worst = bf16_close_chain(bits(got), ref)
    assert ok, worst


def test_qk_rmsnorm_rope():
    g = torch.Generator().manual_seed(721)
    q, k = bf16_randn(g, (1, 300, 4, 128)), bf16_randn(g, (1, 300, 4, 128))
    wq, wk = ((torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16) for _ in range(2))
    f = O.rope_freqs(O.rope_positions(44, 1, 16, 16))
    oq, ok = E.qk_rmsnorm_rope(q, k, wq, wk, torch.view_as_complex(torch.from_numpy(f)))
    rq, rk, _ = O.norm_rope_pack(bits(q), bits(k), bits(q), bits(wq), bits(wk), f)
    for got, ref in ((oq, rq), (ok, rk)):
        good, worst = bf16_close_chain(bits(got), ref)
        assert good, worst


def test_swiglu_and_gated_residual():
    g = torch.Generator().manual_seed(91)
    a, v, h = bf16_randn(g, (64, 1024), 2.0), bf16_randn(g, (64, 1024)), bf16_randn(g, (64, 1024))
    gate = bf16_randn(g, (1, 1024)).tanh()
    assert bf16_close(bits(E.swiglu(a, v)), O.swiglu(bits(a), bits(v)))[0]
    got = E.gated_residual(h[None], v[None], gate[None])
    assert np.array_equal(bits(got)[0], O.residual(bits(h)[None], bits(v)[None], bits(gate))[0])


def test_mx_quantize_and_matmul():
    g = torch.Generator().manual_seed(0)
    x = bf16_randn(g, (200, 512))
    x[torch.rand(x.shape, generator=g) < 0.01] *= 20
    w = bf16_randn(g, (384, 512), 0.02)
    bias = bf16_randn(g, (384,), 0.01)
    qx, qw = E.mx_quantize(x), E.mx_quantize(w)
    ox, ow = O.mx_quantize(bits(x)), O.mx_quantize(bits(w))
    assert np.array_equal(qx[0].numpy(), ox[0]) and np.array_equal(qx[1].numpy(), ox[1])
    assert np.array_equal(qw[0].numpy(), ow[0]) and np.array_equal(qw[1].numpy(), ow[1])
    y = E.mx_matmul(qx, qw, 200, bias)
    ref = O.mx_gemm(*ox, *ow)[:200] + bf16_values(bits(bias))[None, :]
    assert rel_fro(bf16_values(bits(y)), ref) < 4e-3


def test_block_against_oracle_block():
    """The whole config-5 composition at a reduced size: the eager block
    against the oracle block (same weights and quantization), on the
    residual update h2 - h."""
    g = torch.Generator().manual_seed(42)
    b, s, d, heads, ffn = 1, 300, 512, 4, 1024
    w = {"qkv": bf16_randn(g, (3 * d, d), 0.05), "out": bf16_randn(g, (d, d), 0.05),
         "gate": bf16_randn(g, (ffn, d), 0.05), "up": bf16_randn(g, (ffn, d), 0.05),
         "down": bf16_randn(g, (d, ffn), 0.05)}
    nq, nk = ((torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16) for _ in range(2))
    h, mod = bf16_randn(g, (b, s, d)), bf16_randn(g, (b, 6, d), 0.3)
    f = O.rope_freqs(O.rope_positions(44, 1, 16, 16))
    wq = {"qkv": E.mx_quantize(w["qkv"]), "out": E.mx_quantize(w["out"]),
          "gate_up": E.mx_quantize(E.interleave_gate_up(w["gate"], w["up"])), "down": E.mx_quantize(w["down"])}
    out, _ = E.block(h, mod, torch.view_as_complex(torch.from_numpy(f)), wq, nq, nk, heads)
    wb = {k: bits(v) for k, v in w.items()}
    wb.update(norm_q=bits(nq), norm_k=bits(nk))
    ref = OB.block_forward(bits(h), bits(mod), f, wb, heads)
    hv = bf16_values(bits(h))
    assert rel_fro(bf16_values(bits(out)) - hv, bf16_values(ref) - hv) < 1e-2
