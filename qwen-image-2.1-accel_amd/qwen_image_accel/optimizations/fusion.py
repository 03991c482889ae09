"""Selective BF16 fusion of the cached-decode block (the ``fused`` profile).

Reference interface: src/qwen_image_accel/optimizations/fusion.py --
``FusedRopeProcessor`` (:12-35) and ``install_fused_decode`` (:38-60).  The
block keeps its bf16 GEMMs; LayerNorm x scale, the Q/K RMSNorm + RoPE +
prefix pack and the gated residuals run in this build's kernels.  The stages
are optimizations/decode.py's, shared with the mxfp8 profile.
"""
from qwen_image_accel.optimizations.decode import FusedRopeProcessor, install_cached_decode


def install_fused_decode(transformer):
    """Install the bf16 cached-decode block; prefill keeps the native forward."""
    install_cached_decode(transformer, quantized=False)


__all__ = ["FusedRopeProcessor", "install_fused_decode"]
