"""The committed golden fixtures (tests/golden/golden.npz, made by
tests/golden/make_golden.py): the oracle still reproduces them bit for bit,
and its outputs agree with the eager torch-CPU evaluations stored beside them
(bit-exact for MXFP8 bytes and the gated residual, 1 bf16 ulp -- 2 for a rare
element of a two-rounding chain -- for the rest).  No GPU."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import bf16_close, bf16_close_chain, rel_fro

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))


@pytest.mark.parametrize("tag", ["quant_77x256", "quant_130x256", "quant_1x128"])
def test_quantize(tag):
    q, s = O.mx_quantize(G[f"{tag}_x"])
    assert np.array_equal(q, G[f"{tag}_q_oracle"]) and np.array_equal(s, G[f"{tag}_s_oracle"])
    assert np.array_equal(q, G[f"{tag}_q_eager"]) and np.array_equal(s, G[f"{tag}_s_eager"])


@pytest.mark.parametrize("mag", ["0.001", "1", "20"])
def test_layer_norm_scale(mag):
    t = f"ln_{mag}"
    out = O.adaln(G[f"{t}_x"], G[f"{t}_scale"])
    assert np.array_equal(out, G[f"{t}_oracle"])
    assert bf16_close_chain(out, G[f"{t}_eager"])[0]


def test_adaln_config1_chain():
    args = [G[f"adaln_{n}"] for n in ("x", "scale", "shift", "gate", "res")]
    out = O.adaln(*args, add_one=True)
    assert np.array_equal(out, G["adaln_oracle"])
    assert bf16_close_chain(out, G["adaln_eager"])[0]
    q, s = O.adaln_quantize(*args, add_one=True)
    assert np.array_equal(q, G["adaln_q_oracle"]) and np.array_equal(s, G["adaln_s_oracle"])


def test_residual():
    out = O.residual(G["res_h"], G["res_x"], G["res_gate"])
    assert np.array_equal(out, G["res_oracle"]) and np.array_equal(out, G["res_eager"])


def test_swiglu():
    out = O.swiglu(G["swiglu_g"], G["swiglu_v"])
    assert np.array_equal(out, G["swiglu_oracle"])
    assert bf16_close(out, G["swiglu_eager"])[0]
    q, s = O.swiglu_quantize(G["swiglu_g"], G["swiglu_v"])
    assert np.array_equal(q, G["swiglu_q_oracle"]) and np.array_equal(s, G["swiglu_s_oracle"])


def test_norm_rope_pack():
    a = lambda n: G[f"attn_{n}"]
    oq, ok, ov = O.norm_rope_pack(a("q"), a("k"), a("v"), a("wq"), a("wk"), a("freqs"), a("ck"), a("cv"))
    assert np.array_equal(oq, G["attn_oq_oracle"]) and np.array_equal(ok, G["attn_ok_oracle"])
    assert np.array_equal(ov, G["attn_ov_oracle"])
    assert np.array_equal(ov, np.concatenate([a("cv"), a("v")], 1))
    # RoPE cancellation amplifies a 1-ulp norm flip: compare in absolute terms
    for got, ref in ((oq, G["attn_oq_eager"]), (ok, G["attn_ok_eager"])):
        assert rel_fro(O.bf16_to_f32(got), O.bf16_to_f32(ref)) < 4e-3


def test_rope():
    a = lambda n: G[f"attn_{n}"]
    rq, rk = O.rope(a("q"), a("k"), a("freqs"))
    assert np.array_equal(rq, G["rope_oq_oracle"]) and np.array_equal(rk, G["rope_ok_oracle"])
    assert bf16_close(rq, G["rope_oq_eager"])[0] and bf16_close(rk, G["rope_ok_eager"])[0]


def test_rope_table():
    assert np.array_equal(O.rope_freqs(G["freqs_pos"]), G["freqs_oracle"])


def test_gemm():
    aq, as_ = O.mx_quantize(G["gemm_a"])
    wq, ws = O.mx_quantize(G["gemm_w"])
    acc = O.mx_gemm(aq, as_, wq, ws)[:100]
    assert np.array_equal(acc, G["gemm_acc_oracle"])
    assert rel_fro(acc, G["gemm_eager"]) < 1e-6
