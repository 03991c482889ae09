"""The reference-facing boundary: profile registry, installers and the patched
cached-decode block (routing on the CPU, numerics on the GPU)."""
import copy

import numpy as np
import pytest
import torch

from qwen_image_accel import _native, pipeline, profiles
from qwen_image_accel.kernels import attention, bf16, elementwise, layernorm
from qwen_image_accel.optimizations import fusion, mxfp8, quantized_decode
from tests import fake_qwen21 as fq
from tests.helpers import rel_fro


# ---------------------------------------------------------------- profiles --

def test_profile_names_and_fields_match_reference():
    assert list(profiles.PROFILES) == ["baseline", "safe", "fused", "fused_sage", "mxfp8", "mxfp8_sage",
                                       "mxfp8_balanced", "mxfp8_balanced_sage", "compiled", "graph"]
    assert profiles.get_profile("fused").fused and not profiles.get_profile("fused").quantized
    assert profiles.get_profile("mxfp8").quantized
    assert profiles.get_profile("mxfp8_balanced").skip_blocks == "0,1,2,29,30,31"


@pytest.mark.parametrize("name,msg", [("fp8", "retired; use mxfp8"), ("nope", "Unknown Qwen optimization")])
def test_get_profile_rejects(name, msg):
    with pytest.raises(ValueError, match=msg):
        profiles.get_profile(name)


@pytest.mark.parametrize("name", ["fused_sage", "mxfp8_sage", "compiled", "graph"])
def test_out_of_scope_profiles_are_rejected(name):
    t = fq.make_transformer()
    with pytest.raises(NotImplementedError):
        pipeline.install_hot_path(t, name, validate=False)


def test_baseline_installs_nothing():
    t = fq.make_transformer()
    forwards = [b.forward for b in t.transformer_blocks]
    cfg = pipeline.install_hot_path(t, "baseline", validate=False)
    assert cfg == {"profile": "baseline", "approximate": False}
    assert [b.forward for b in t.transformer_blocks] == forwards
    with pytest.raises(RuntimeError, match="once"):
        pipeline.install_hot_path(t, "fused", validate=False)


def test_layer_selection():
    assert mxfp8.selected_layers("attention") == set(mxfp8.LAYER_GROUPS["attention"])
    assert mxfp8.selected_layers("attn.to_q, img_mlp.out") == {"attn.to_q", "img_mlp.out"}
    with pytest.raises(ValueError, match="Unknown MXFP8 layer"):
        mxfp8.selected_layers("attn.to_x")


def test_mxfp8linear_rejects_bias():
    with pytest.raises(ValueError, match="bias-free"):
        mxfp8.MXFP8Linear(torch.nn.Linear(256, 256, bias=True))


# ------------------------------------------- routing (CPU: eager fallbacks) --

def _cached(t, inputs):
    h, mod, freqs, cache = inputs
    out = h
    for b in t.transformer_blocks:
        out = b(hidden_states=out, modulation=mod, rotary_emb=freqs, layer_cache=cache, kv_cache_mode="cached")
    return out


def test_fused_decode_on_cpu_equals_eager_block():
    """On CPU tensors every kernel wrapper takes the reference's eager fallback,
    so the patched block must equal the native block bit for bit."""
    t = fq.make_transformer()
    ref_t = copy.deepcopy(t)
    inputs = fq.make_inputs()
    with torch.no_grad():
        want = _cached(ref_t, inputs)
        cfg = pipeline.install_hot_path(t, "fused", validate=False)
        got = _cached(t, inputs)
    assert cfg["fused_norm_rope_kv_pack"] and isinstance(t.transformer_blocks[0].attn.processor,
                                                          fusion.FusedRopeProcessor)
    assert torch.equal(got, want)


def test_prefill_keeps_native_forward():
    t = fq.make_transformer()
    ref_t = copy.deepcopy(t)
    h, mod, freqs, cache = fq.make_inputs()
    with torch.no_grad():
        want = ref_t.transformer_blocks[0](hidden_states=h, modulation=mod[:-1], rotary_emb=freqs)
        pipeline.install_hot_path(t, "fused", validate=False)
        got = t.transformer_blocks[0](hidden_states=h, modulation=mod[:-1], rotary_emb=freqs)
    assert torch.equal(got, want)


# ------------------------------------------------------- numerics (GPU) --

def _run_profile(dev, profile):
    t = fq.make_transformer(dim=512, heads=4, ffn=1024, device=dev)
    ref_t = copy.deepcopy(t)
    inputs = fq.make_inputs(dim=512, heads=4, tokens=200, prefix=37, batch=1, device=dev)
    before = dict(_native.calls)
    with torch.no_grad():
        want = _cached(ref_t, inputs)
        cfg = pipeline.install_hot_path(t, profile, validate=False)
        got = _cached(t, inputs)
    torch.cuda.synchronize()
    used = {k for k, v in _native.calls.items() if v > before.get(k, 0)}
    return cfg, used, rel_fro(got.float().cpu().numpy(), want.float().cpu().numpy())


@pytest.mark.gpu
def test_fused_profile_matches_native_block(dev):
    """The BF16 fused block differs from the native one only by reduction order
    (LayerNorm / RMSNorm statistics)."""
    print("[case] boundary fused", flush=True)
    cfg, used, err = _run_profile(dev, "fused")
    assert {"qim_adaln", "qim_gated_residual", "qim_qk_norm_rope_pack", "qim_swiglu"} <= used, used
    assert err < 5e-3, err


@pytest.mark.gpu
def test_mxfp8_profile_matches_native_block(dev, monkeypatch):
    """The composed MXFP8 block vs the native bf16 block: the difference is the
    MXFP8 quantization (the reference reports ~1.7% velocity rel-RMSE for
    mxfp8, docs/benchmarks/measurements.json teacher_forced)."""
    print("[case] boundary mxfp8", flush=True)
    monkeypatch.setenv("QW21_MXFP8_SKIP_BLOCKS", "")
    cfg, used, err = _run_profile(dev, "mxfp8")
    assert cfg["mxfp8_linears"] == 14 and cfg["mxfp8_fused_gate_up"] == 2
    # SwiGLU -> MXFP8 runs in the interleaved gate/up GEMM's epilogue (weights.fuse_gate_up)
    assert {"qim_adaln_quantize", "qim_mx_quantize_tiled"} <= used, used
    assert used & {"qim_mxfp8_gemm_ex", "qim_mxfp8_gemm_ws"}, used
    assert "qim_swiglu_quantize_tiled" not in used, used
    assert err < 5e-2, err


@pytest.mark.gpu
def test_mxfp8_default_skip_blocks(dev):
    """Blocks 0 and 31 stay BF16 by default (optimizations/mxfp8.py:74): of the
    two stand-in blocks only block 1's seven linears are converted."""
    cfg, used, err = _run_profile(dev, "mxfp8")
    assert cfg["mxfp8_linears"] == 7 and cfg["mxfp8_skipped_blocks"] == "0,31"
    assert err < 5e-2, err


def test_attention_backend_env_is_validated(monkeypatch):
    from qwen_image_accel.optimizations import attention_call
    monkeypatch.setenv("QW21_ATTENTION_BACKEND", "flash")
    x = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="QW21_ATTENTION_BACKEND"):
        attention_call.attention(x, x, x)


@pytest.mark.gpu
def test_mxfp8_profile_with_qim_attention_backend(dev, monkeypatch):
    """QW21_ATTENTION_BACKEND=qim: the decode attention runs on this build's
    core, which also writes the MXFP8 out-projection's input
    (qim_attention_mxfp8); the block output stays within the attention bar of
    the default path."""
    print("[case] boundary mxfp8 + qim attention", flush=True)
    monkeypatch.setenv("QW21_MXFP8_SKIP_BLOCKS", "")
    _, used0, _ = _run_profile(dev, "mxfp8")
    assert "qim_attention" not in used0
    t = fq.make_transformer(dim=512, heads=4, ffn=1024, device=dev)
    ref_t = copy.deepcopy(t)
    inputs = fq.make_inputs(dim=512, heads=4, tokens=200, prefix=37, batch=1, device=dev)
    with torch.no_grad():
        pipeline.install_hot_path(ref_t, "mxfp8", validate=False)
        want = _cached(ref_t, inputs)
        monkeypatch.setenv("QW21_ATTENTION_BACKEND", "qim")
        before = dict(_native.calls)
        pipeline.install_hot_path(t, "mxfp8", validate=False)
        got = _cached(t, inputs)
    torch.cuda.synchronize()
    # the out-projection is MXFP8: the core writes its input (qim_attention_mxfp8)
    assert _native.calls.get("qim_attention_mxfp8", 0) > before.get("qim_attention_mxfp8", 0)
    assert rel_fro(got.float().cpu().numpy(), want.float().cpu().numpy()) < 1e-2


def test_qim_attention_backend_applies_only_where_it_can(monkeypatch):
    """QW21_ATTENTION_BACKEND=qim routes only unmasked bf16 CUDA calls with head
    dim 128 and packed heads; everything else keeps the reference's dispatch."""
    from qwen_image_accel.optimizations import attention_call
    x = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    monkeypatch.delenv("QW21_ATTENTION_BACKEND", raising=False)
    assert not attention_call.qim_backend(x, x, x)
    monkeypatch.setenv("QW21_ATTENTION_BACKEND", "qim")
    assert not attention_call.qim_backend(x, x, x)                      # CPU tensors
    assert not attention_call._qim_applies(x.float(), x.float(), x.float(), None)
    assert not attention_call._qim_applies(x, x, x, torch.ones(1, 1, 4, 4, dtype=torch.bool))
    y = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    assert not attention_call._qim_applies(y, y, y, None)                # head dim 64
    out = attention_call.attention(x, x, x)                              # falls back to SDPA on the CPU
    assert out.shape == x.shape and out.dtype == x.dtype


# ----------------------------------------------- MXFP8Linear state dicts --

def _quantized_linear(k, n, seed=0):
    """An MXFP8Linear over random code and scale bytes (no GPU needed)."""
    from qwen_image_accel.kernels.mxfp8 import padded_rows, tile_codes
    g = torch.Generator().manual_seed(seed)
    rows = padded_rows(n)
    codes = torch.randint(0, 256, (rows, k), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
    scales = torch.randint(100, 140, (rows * k // 32,), generator=g, dtype=torch.uint8)
    return mxfp8.MXFP8Linear.from_quantized(k, n, tile_codes(codes), scales), codes


@pytest.mark.parametrize("k,n", [(256, 256), (384, 640), (256, 100 * 128)])
def test_mxfp8linear_state_dict_uses_reference_keys(k, n):
    """state_dict() holds the reference's weight_fp8 -- the (K, padded N)
    transpose view of row-major codes -- and weight_scale; it loads back into
    a fresh module byte for byte, also as a contiguous (K, N) copy (as a
    safetensors round trip returns it; K = N included, where a transposed
    load would go unnoticed by shape); a wrong shape is refused."""
    m, codes = _quantized_linear(k, n)
    sd = m.state_dict()
    assert set(sd) == {"weight_fp8", "weight_scale"}
    assert sd["weight_fp8"].shape == (k, codes.shape[0])
    assert torch.equal(sd["weight_fp8"].t().view(torch.uint8), codes.view(torch.uint8))
    for form in (sd["weight_fp8"], sd["weight_fp8"].contiguous()):
        fresh, _ = _quantized_linear(k, n, seed=1)
        fresh.load_state_dict({"weight_fp8": form, "weight_scale": sd["weight_scale"]})
        assert torch.equal(fresh.weight_tiled.view(torch.uint8), m.weight_tiled.view(torch.uint8))
        assert torch.equal(fresh.weight_scale.view(torch.uint8), m.weight_scale.view(torch.uint8))
    fresh, _ = _quantized_linear(k, n, seed=1)
    with pytest.raises(ValueError, match="weight_fp8"):
        fresh.load_state_dict({"weight_fp8": sd["weight_fp8"][:, :128], "weight_scale": sd["weight_scale"]})


def test_conversion_plan_takes_multiples_of_128():
    """The reference converts a linear when K and N are multiples of 128
    (optimizations/mxfp8.py:15-16): a 384-wide projection is planned, a
    320-wide one is not; skipped blocks and the layer selection apply."""
    t = fq.make_transformer(n_blocks=3, dim=256, heads=2, ffn=512)
    t.transformer_blocks[1].img_mlp.proj = torch.nn.Linear(256, 384, bias=False)
    t.transformer_blocks[2].img_mlp.proj = torch.nn.Linear(256, 320, bias=False)
    plan = mxfp8.conversion_plan(t, skip_blocks="0", layers="img_mlp.proj,attn.to_q")
    assert [(i, p) for i, p, _ in plan] == [(1, "attn.to_q"), (1, "img_mlp.proj"), (2, "attn.to_q")]
    assert mxfp8.skipped_blocks("") == set() and mxfp8.skipped_blocks(" 3, 5") == {3, 5}
