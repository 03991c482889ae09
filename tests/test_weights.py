"""Weight-side MXFP8 formats (qwen_image_accel.weights), on the CPU: the scale
swizzle against the reference test's layout, the interleaved gate/up weight
against quantizing the interleaved bf16 weight (C oracle), and the
pre-quantized weight file round trip.  The GPU test runs the mxfp8 profile with
the interleaved gate/up GEMM and with weights loaded from a file."""
import copy

import numpy as np
import pytest
import torch

from oracle import oracle as O
from qwen_image_accel import pipeline, weights
from qwen_image_accel.kernels import gemm, mxfp8
from qwen_image_accel.optimizations import decode, mxfp8 as mx
from tests import fake_qwen21 as fq
from tests.helpers import bits, swizzle_permute


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def oracle_linear(w):
    """An MXFP8Linear holding the C oracle's quantization of bf16 weight w."""
    codes, scales = O.mx_quantize(bits(w))
    tiled = mxfp8.tile_codes(torch.from_numpy(codes).view(torch.float8_e4m3fn))
    return mx.MXFP8Linear.from_quantized(w.shape[1], w.shape[0], tiled, torch.from_numpy(scales))


def test_scale_swizzle_matches_reference_layout():
    g = torch.Generator().manual_seed(0)
    e = torch.randint(0, 256, (384, 16), generator=g, dtype=torch.uint8)
    flat = weights.swizzle_scales(e)
    assert np.array_equal(flat.numpy(), swizzle_permute(e.numpy()))
    assert torch.equal(weights.unswizzle_scales(flat, 384, 16 * 32), e)


@pytest.mark.parametrize("f,k", [(256, 256), (384, 512)])
def test_interleaved_gate_up_equals_quantized_interleave(f, k):
    """Rows (codes and scales) permuted from the two quantized weights are the
    bytes of quantizing the interleaved bf16 weight: no requantization."""
    g = torch.Generator().manual_seed(f + k)
    wg = (torch.randn(f, k, generator=g) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(f, k, generator=g) * 0.05).to(torch.bfloat16)
    wg[3, :64] *= 1000  # distinct scales per row and block
    codes, scales = weights.interleave_quantized(oracle_linear(wg), oracle_linear(wu))
    ref_codes, ref_scales = O.mx_quantize(bits(gemm.interleave_swiglu(wg, wu)))
    assert np.array_equal(u8(mxfp8.untile_codes(codes)), ref_codes)
    assert np.array_equal(u8(scales), ref_scales)


def test_fused_qkv_equals_quantized_concatenation():
    """Q, K, V weights stacked as one (3N, K) MXFP8 weight: the bytes of
    quantizing the stacked bf16 weight."""
    g = torch.Generator().manual_seed(9)
    ws = [(torch.randn(256, 384, generator=g) * 0.05).to(torch.bfloat16) for _ in range(3)]
    ws[1][7, 100:] *= 300
    attn = torch.nn.Module()
    attn.to_q, attn.to_k, attn.to_v = (oracle_linear(w) for w in ws)
    assert weights.fuse_qkv(attn)
    ref_codes, ref_scales = O.mx_quantize(bits(torch.cat(ws, 0)))
    assert np.array_equal(u8(mxfp8.untile_codes(attn._mx_qkv[0])), ref_codes)
    assert np.array_equal(u8(attn._mx_qkv[1]), ref_scales)


def test_fusions_skip_biased_projections():
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(256, 256, generator=g) * 0.05).to(torch.bfloat16)
    attn, mlp = torch.nn.Module(), torch.nn.Module()
    attn.to_q, attn.to_k, attn.to_v = oracle_linear(w), oracle_linear(w), oracle_linear(w)
    attn.to_k.bias = torch.zeros(256, dtype=torch.bfloat16)
    mlp.gate_layer, mlp.proj = oracle_linear(w), oracle_linear(w)
    mlp.proj.bias = torch.zeros(256, dtype=torch.bfloat16)
    assert not weights.fuse_qkv(attn) and getattr(attn, "_mx_qkv", None) is None
    assert not weights.fuse_gate_up(mlp) and getattr(mlp, "_mx_gate_up", None) is None
    with pytest.raises(ValueError, match="does not match"):
        mx.MXFP8Linear.from_quantized(256, 512, attn.to_q.weight_tiled, attn.to_q.weight_scale)


def _quantized_fake(seed=0):
    t = fq.make_transformer(dim=256, heads=2, ffn=512, seed=seed)
    for b in t.transformer_blocks:
        for name in ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0", "img_mlp.gate_layer",
                     "img_mlp.proj", "img_mlp.out"):
            parent, _, leaf = name.rpartition(".")
            lin = b.get_submodule(name)
            setattr(b.get_submodule(parent), leaf, oracle_linear(lin.weight.detach().to(torch.bfloat16)))
        assert weights.fuse_gate_up(b.img_mlp)
        assert weights.fuse_qkv(b.attn)
    return t


def test_save_and_load_prequantized_weights(tmp_path):
    src = _quantized_fake()
    path = str(tmp_path / "w.safetensors")
    names = weights.save_mxfp8(src, path)
    assert len(names) == 14
    dst = fq.make_transformer(dim=256, heads=2, ffn=512, seed=5)
    assert sorted(weights.load_mxfp8(dst, path)) == names
    a, b = dict(weights._modules(src)), dict(weights._modules(dst))
    for n in names:
        assert isinstance(b[n], mx.MXFP8Linear)
        assert np.array_equal(u8(a[n].weight_tiled), u8(b[n].weight_tiled))
        assert np.array_equal(u8(a[n].weight_scale), u8(b[n].weight_scale))
        assert b[n].weight_tiled.dtype == torch.float8_e4m3fn
    for i in range(2):
        ga, gb = src.transformer_blocks[i].img_mlp._mx_gate_up, dst.transformer_blocks[i].img_mlp._mx_gate_up
        assert np.array_equal(u8(ga[0]), u8(gb[0])) and np.array_equal(u8(ga[1]), u8(gb[1]))
        qa, qb = src.transformer_blocks[i].attn._mx_qkv, dst.transformer_blocks[i].attn._mx_qkv
        assert np.array_equal(u8(qa[0]), u8(qb[0])) and np.array_equal(u8(qa[1]), u8(qb[1]))


def test_load_rejects_other_files_and_shapes(tmp_path):
    from safetensors.torch import save_file
    bad = str(tmp_path / "bad.safetensors")
    save_file({"x": torch.zeros(4)}, bad, metadata={"format": "other"})
    with pytest.raises(ValueError, match="not a qim-mxfp8"):
        weights.load_mxfp8(fq.make_transformer(dim=256, heads=2, ffn=512), bad)
    path = str(tmp_path / "w.safetensors")
    weights.save_mxfp8(_quantized_fake(), path)
    with pytest.raises(ValueError, match="linear in this model"):
        weights.load_mxfp8(fq.make_transformer(dim=512, heads=4, ffn=1024), path)


# ----------------------------------------------------------------- GPU --

def _profile_out(dev, t, inputs):
    with torch.no_grad():
        cfg = pipeline.install_hot_path(t, "mxfp8", validate=False)
        out = t
        h, mod, freqs, cache = inputs
        x = h
        for b in out.transformer_blocks:
            x = b(hidden_states=x, modulation=mod, rotary_emb=freqs, layer_cache=cache, kv_cache_mode="cached")
    torch.cuda.synchronize()
    return cfg, x


@pytest.mark.gpu
def test_mxfp8_profile_fused_gate_up_and_prequantized_weights(dev, monkeypatch, tmp_path):
    """The mxfp8 profile's decode MLP as one interleaved gate/up GEMM with the
    SwiGLU -> MXFP8 epilogue, and its Q/K/V projections as one GEMM, equal,
    byte for byte, the separate GEMMs (+ swiglu_quantize); and a transformer
    whose weights load from a save_mxfp8 file (no quantization) gives the
    same output again."""
    print("[case] mxfp8 fused gate/up + prequantized weights", flush=True)
    monkeypatch.setenv("QW21_MXFP8_SKIP_BLOCKS", "")
    base = fq.make_transformer(dim=512, heads=4, ffn=1024, device=dev)
    inputs = fq.make_inputs(dim=512, heads=4, tokens=200, prefix=37, batch=1, device=dev)
    t_fused, t_plain, t_loaded = copy.deepcopy(base), copy.deepcopy(base), copy.deepcopy(base)
    cfg, fused = _profile_out(dev, t_fused, inputs)
    assert cfg["mxfp8_fused_gate_up"] == 2 and cfg["mxfp8_fused_qkv"] == 2
    with monkeypatch.context() as m:
        m.setattr(decode, "fuse_gate_up", lambda mlp: False)
        m.setattr(decode, "fuse_qkv", lambda attn: False)
        cfg_p, plain = _profile_out(dev, t_plain, inputs)
    assert cfg_p["mxfp8_fused_gate_up"] == 0 and cfg_p["mxfp8_fused_qkv"] == 0
    assert torch.equal(fused, plain)
    path = str(tmp_path / "w.safetensors")
    weights.save_mxfp8(t_fused, path)
    monkeypatch.setenv("QW21_MXFP8_WEIGHTS", path)
    cfg_l, loaded = _profile_out(dev, t_loaded, inputs)
    assert cfg_l["mxfp8_weights"] == path and cfg_l["mxfp8_linears"] == 14 and cfg_l["mxfp8_fused_gate_up"] == 2
    assert cfg_l["mxfp8_fused_qkv"] == 2
    assert torch.equal(loaded, fused)
