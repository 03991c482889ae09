"""HIP kernels against the committed golden fixtures (tests/golden/golden.npz):
bit-exact against the oracle's outputs for MXFP8 bytes, the gated residual,
RoPE, SwiGLU and the normalisations (float64 row statistics rounded once);
within the bf16 chain tolerance against eager torch-CPU outputs (own fp32
reductions); GEMM within rel-Frobenius 1e-2 of the dequantize-then-matmul."""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from qwen_image_accel.kernels import attention, bf16, elementwise, epilogue, gemm, layernorm, mxfp8
from tests.helpers import bf16_close, bf16_close_chain, bits, from_bits, rel_fro

pytestmark = pytest.mark.gpu
G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))


def t(name, dev):
    return from_bits(G[name], dev)


def u8(x):
    return x.view(torch.uint8).cpu().numpy()


class _LN:
    def __init__(self, d):
        self.normalized_shape, self.eps, self.elementwise_affine = (d,), 1e-6, False

    def __call__(self, x):
        return F.layer_norm(x, self.normalized_shape, eps=self.eps)


class _RMS:
    def __init__(self, w):
        self.weight, self.bias, self.eps = w, None, 1e-6


@pytest.mark.parametrize("tag", ["quant_77x256", "quant_130x256", "quant_1x128"])
def test_quantize(dev, tag):
    a = mxfp8.quantize(t(f"{tag}_x", dev))
    assert np.array_equal(u8(a.values), G[f"{tag}_q_eager"])
    assert np.array_equal(u8(a.scales), G[f"{tag}_s_eager"])


@pytest.mark.parametrize("mag", ["0.001", "1", "20"])
def test_layer_norm_scale(dev, mag):
    out = layernorm.layer_norm_scale(t(f"ln_{mag}_x", dev), t(f"ln_{mag}_scale", dev), _LN(512))
    assert np.array_equal(bits(out), G[f"ln_{mag}_oracle"])
    assert bf16_close_chain(bits(out), G[f"ln_{mag}_eager"])[0]


def test_adaln_chain_and_quantize(dev):
    x, s, sh, g, r = (t(f"adaln_{n}", dev) for n in ("x", "scale", "shift", "gate", "res"))
    out = layernorm.layer_norm_scale(x, s, _LN(512), shift=sh, gate=g, residual=r, add_one=True)
    assert np.array_equal(bits(out), G["adaln_oracle"])
    q = epilogue.layer_norm_scale_quantize(x, s, _LN(512), shift=sh, gate=g, residual=r, add_one=True)
    assert np.array_equal(u8(q.values), G["adaln_q_oracle"])
    assert np.array_equal(u8(q.scales), G["adaln_s_oracle"])


def test_residual(dev):
    out = elementwise.residual(t("res_h", dev), t("res_x", dev), t("res_gate", dev))
    assert np.array_equal(bits(out), G["res_eager"])


def test_swiglu(dev):
    """Bit-exact: the device SiLU equals the oracle's on every bf16 input
    (test_gpu_kernels.test_silu_exhaustive) and the product is one fp32
    multiply rounded once."""
    out = bf16.swiglu(t("swiglu_g", dev), t("swiglu_v", dev))
    assert np.array_equal(bits(out), G["swiglu_oracle"])
    q = epilogue.swiglu_quantize(t("swiglu_g", dev), t("swiglu_v", dev))
    assert np.array_equal(u8(q.values), G["swiglu_q_oracle"])
    assert np.array_equal(u8(q.scales), G["swiglu_s_oracle"])


def test_rope(dev):
    f = torch.view_as_complex(torch.from_numpy(G["attn_freqs"])).to(dev)
    oq, ok = elementwise.rope_qk(t("attn_q", dev), t("attn_k", dev), f)
    assert np.array_equal(bits(oq), G["rope_oq_oracle"]) and np.array_equal(bits(ok), G["rope_ok_oracle"])


def test_prepare_attention_inputs(dev):
    f = torch.view_as_complex(torch.from_numpy(G["attn_freqs"])).to(dev)
    a = lambda n: t(f"attn_{n}", dev)
    oq, ok, ov = attention.prepare_attention_inputs(a("q"), a("k"), a("v"), _RMS(a("wq")), _RMS(a("wk")), f,
                                                    a("ck"), a("cv"))
    assert np.array_equal(bits(ov), G["attn_ov_oracle"])
    assert np.array_equal(bits(oq), G["attn_oq_oracle"])
    assert np.array_equal(bits(ok), G["attn_ok_oracle"])


def test_gemm(dev):
    aq = mxfp8.quantize(t("gemm_a", dev))
    wq = mxfp8.quantize(t("gemm_w", dev))
    y = gemm.mx_matmul(aq, wq.values, wq.scales)
    assert rel_fro(y.float().cpu().numpy(), G["gemm_acc_oracle"]) < 1e-2
