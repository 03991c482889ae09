"""Install a profile's hot-path kernels into a Qwen-Image-2.1 pipeline.

Reference interface: src/qwen_image_accel/pipeline.py -- ``configure_pipeline``
(:109-198), ``_validate_fused_runtime`` (:94-106).  This build keeps the
install points of the hot path (:131-172): MXFP8 conversion of the block
linears for quantized profiles, then the composed (``mxfp8``) or BF16
(``fused``) cached-decode block, then the Q/K RMSNorm and SwiGLU hooks.  The
product-level parts of the reference's configure step -- text-encoder
placement, VAE tiling policy, step cache, CUDA-graph and compile policies,
SageAttention2 -- are outside this build and are not installed.
"""
import os

import torch

from qwen_image_accel.profiles import get_profile


def validate_runtime(transformer):
    """Reject inputs the HIP kernels were not built for, before changing anything
    (the reference's guard checks torch/CUDA/Triton/SM120; this one checks for
    a gfx950 device and a bf16 transformer)."""
    dtype = getattr(transformer, "dtype", torch.bfloat16)
    if dtype != torch.bfloat16:
        raise ValueError("The fused/mxfp8 profiles require a BF16 transformer")
    if not torch.cuda.is_available():
        raise RuntimeError("The fused/mxfp8 profiles need a ROCm GPU; use QW21_PROFILE=safe")
    arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"libqim is built for gfx950 (MI355X); this device is {arch!r}")
    from qwen_image_accel import _native
    _native.lib()  # fail loudly if the kernels are missing


def install_hot_path(transformer, profile="fused", *, validate=True):
    """The hot-path install points of configure_pipeline (pipeline.py:131-172),
    applied to a transformer.  Returns the configuration record."""
    selected = get_profile(profile)
    if getattr(transformer, "_qw_hot_path", None) is not None:
        raise RuntimeError("Configure a fresh transformer once; profiles cannot be switched in place")
    if selected.sage:
        raise NotImplementedError(f"profile {profile!r} needs SageAttention2, whose attention core is "
                                  "outside this build; use 'fused' or 'mxfp8'")
    if selected.compile or selected.graph:
        raise NotImplementedError(f"profile {profile!r} is an execution policy outside this build")
    config = {"profile": profile, "approximate": False}
    if not selected.fused:
        transformer._qw_hot_path = config
        return config
    if validate:
        validate_runtime(transformer)
    if selected.quantized:
        from qwen_image_accel.optimizations.mxfp8 import quantize_transformer
        skip = os.environ.get("QW21_MXFP8_SKIP_BLOCKS", selected.skip_blocks or "0,31")
        layers = os.environ.get("QW21_MXFP8_LAYERS", "all")
        weights = os.environ.get("QW21_MXFP8_WEIGHTS", "")
        if weights:   # pre-quantized weights (weights.save_mxfp8): no quantization at startup
            from qwen_image_accel.weights import load_mxfp8
            config["mxfp8_linears"] = len(load_mxfp8(transformer, weights))
            config["mxfp8_weights"] = weights
        else:
            config["mxfp8_linears"] = len(quantize_transformer(transformer, skip, layers))
        config["mxfp8_skipped_blocks"] = skip
        config["mxfp8_layer_selection"] = layers
        config["approximate"] = True
        from qwen_image_accel.optimizations.quantized_decode import install_mx_fused_decode
        install_mx_fused_decode(transformer)
        config["mxfp8_fused_gate_up"] = sum(getattr(b.img_mlp, "_mx_gate_up", None) is not None
                                            for b in transformer.transformer_blocks)
        config["mxfp8_fused_qkv"] = sum(getattr(b.attn, "_mx_qkv", None) is not None
                                        for b in transformer.transformer_blocks)
    else:
        from qwen_image_accel.optimizations.fusion import install_fused_decode
        install_fused_decode(transformer)
    from qwen_image_accel.kernels.bf16 import install_qk_norm, install_swiglu
    install_qk_norm(transformer)
    if not selected.quantized:
        install_swiglu(transformer)   # the composed path installs its own
    config.update(fused_qk_rmsnorm=True, fused_swiglu=True, fused_norm_rope_kv_pack=True,
                  fused_layernorm_scale=True, runtime_token_counts=True)
    transformer._qw_hot_path = config
    return config


def configure_pipeline(pipe, profile="fused"):
    """configure_pipeline(pipe, profile) restricted to the hot path: the
    transformer goes to the GPU and gets the profile's kernels."""
    selected = get_profile(profile)
    if hasattr(pipe, "_qw_optimization"):
        raise RuntimeError("Configure a fresh pipeline once; profiles cannot be switched in place")
    if selected.fused:
        validate_runtime(pipe.transformer)
    pipe.transformer.to("cuda")
    config = install_hot_path(pipe.transformer, profile, validate=False)
    pipe._qw_optimization = config
    return config
