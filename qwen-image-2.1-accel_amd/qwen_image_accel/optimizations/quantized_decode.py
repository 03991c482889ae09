"""The composed cached-decode block: fused BF16 kernels + MXFP8 GEMMs (``mxfp8``).

Reference interface: src/qwen_image_accel/optimizations/quantized_decode.py --
``MXFusedProcessor`` (:31-78) and ``install_mx_fused_decode`` (:108-137).
Q/K/V share one quantized activation, as do the SwiGLU gate and value
projections; the LayerNorm emits it directly when every consumer is MXFP8.
Beyond the reference: the Q/K/V weights are stacked into one GEMM and the
gate/up weights interleaved so that one GEMM's epilogue writes the down
projection's MXFP8 input (weights.fuse_qkv / fuse_gate_up).  The stages are
optimizations/decode.py's, shared with the fused profile.
"""
from qwen_image_accel.optimizations.decode import MXFusedProcessor, QuantizedSwiGLU, install_cached_decode


def install_mx_fused_decode(transformer, sage=False):
    """Install the composed cached-decode block; prefill keeps the native forward."""
    if sage:
        raise NotImplementedError("SageAttention2 decode is outside this build; use the mxfp8 profile")
    install_cached_decode(transformer, quantized=True)


__all__ = ["MXFusedProcessor", "QuantizedSwiGLU", "install_mx_fused_decode"]
