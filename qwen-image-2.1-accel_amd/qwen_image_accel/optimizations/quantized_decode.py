"""The composed cached-decode block: fused BF16 kernels + MXFP8 GEMMs (``mxfp8``).

Reference interface: src/qwen_image_accel/optimizations/quantized_decode.py --
``MXFusedProcessor`` (:31-78), ``_mx_mlp_forward`` (:81-96), ``_normalized``
(:99-105), ``install_mx_fused_decode`` (:108-137).  Q/K/V share one quantized
activation and the SwiGLU gate/value projections share another; LayerNorm and
SwiGLU emit MXFP8 directly when every consumer is an MXFP8 linear.  Those
shared activations are consumed only by this build's GEMM, so they are written
in its tiled code layout.
"""
import types

from qwen_image_accel.kernels.bf16 import swiglu
from qwen_image_accel.kernels.elementwise import residual
from qwen_image_accel.kernels.gemm import mx_matmul
from qwen_image_accel.kernels.epilogue import layer_norm_scale_quantize, swiglu_quantize
from qwen_image_accel.kernels.layernorm import layer_norm_scale
from qwen_image_accel.kernels.mxfp8 import Quantized, quantize
from qwen_image_accel.optimizations.fusion import _attend, modulation_values
from qwen_image_accel.optimizations.mxfp8 import MXFP8Linear
from qwen_image_accel.weights import fuse_gate_up, fuse_qkv


class MXFusedProcessor:
    """Cached-decode attention with one shared Q/K/V activation quantization.

    ``sage=True`` names SageAttention2, which this build does not provide."""

    def __init__(self, native=None, sage=False):
        if sage:
            raise NotImplementedError("SageAttention2 decode is outside this build; use the mxfp8 profile")
        self.native = native
        self.sage = False

    def __call__(self, attn, hidden_states, attention_mask=None, rotary_emb=None,
                 layer_cache=None, kv_cache_mode=None, cache_write_slice=None,
                 segments=None, key_valid=None):
        if kv_cache_mode != "cached":
            return self.native(attn, hidden_states, attention_mask, rotary_emb, layer_cache,
                               kv_cache_mode, cache_write_slice, segments, key_valid)
        projections = (attn.to_q, attn.to_k, attn.to_v)
        qkv = getattr(attn, "_mx_qkv", None)
        if qkv is not None and (isinstance(hidden_states, Quantized) or hidden_states.is_contiguous()):
            # One GEMM for the three projections (weights.fuse_qkv); Q, K, V are
            # column blocks of its output, which the norm + RoPE + pack reads in place.
            shared = hidden_states if isinstance(hidden_states, Quantized) else \
                quantize(hidden_states.reshape(-1, hidden_states.shape[-1]), tiled=True)
            lead = hidden_states.shape[:-1]
            out = mx_matmul(shared, qkv[0], qkv[1], weight_tiled=True).view(*lead, -1)
            d = out.shape[-1] // 3
            q, k, v = (out[..., i * d:(i + 1) * d].unflatten(-1, (attn.heads, -1)) for i in range(3))
        elif isinstance(hidden_states, Quantized):
            # The block's LayerNorm already emitted FP8; no BF16 tensor exists.
            lead = hidden_states.shape[:-1]
            q, k, v = (p.matmul(hidden_states).view(*lead, attn.heads, -1) for p in projections)
        elif all(isinstance(p, MXFP8Linear) for p in projections) and hidden_states.is_contiguous():
            shared = quantize(hidden_states.reshape(-1, hidden_states.shape[-1]), tiled=True)
            lead = hidden_states.shape[:-1]
            q, k, v = (p.matmul(shared).view(*lead, attn.heads, -1) for p in projections)
        else:
            q, k, v = (p(hidden_states).unflatten(-1, (attn.heads, -1)) for p in projections)
        return _attend(self, attn, q, k, v, attention_mask, rotary_emb, layer_cache)


def _mx_mlp_forward(self, hidden_states):
    """SwiGLU whose gate and value projections share one quantized activation.

    With the interleaved gate/up weight (``weights.fuse_gate_up``) and an MXFP8
    down projection, one GEMM computes both projections and its epilogue writes
    the down projection's MXFP8 input (the same bytes as the two GEMMs +
    ``swiglu_quantize``)."""
    lead = hidden_states.shape[:-1]
    if isinstance(hidden_states, Quantized):
        shared = hidden_states
    elif (isinstance(self.gate_layer, MXFP8Linear) and isinstance(self.proj, MXFP8Linear)
            and hidden_states.is_contiguous()):
        shared = quantize(hidden_states.reshape(-1, hidden_states.shape[-1]), tiled=True)
    else:
        return self.out(swiglu(self.gate_layer(hidden_states), self.proj(hidden_states)))
    gate_up = getattr(self, "_mx_gate_up", None)
    if gate_up is not None and isinstance(self.out, MXFP8Linear):
        activated = mx_matmul(shared, gate_up[0], gate_up[1], epilogue="swiglu_quant", weight_tiled=True,
                              out_tiled=True)
        return self.out.matmul(activated).view(*lead, -1)
    gate, value = self.gate_layer.matmul(shared), self.proj.matmul(shared)
    if isinstance(self.out, MXFP8Linear):
        activated = swiglu_quantize(gate, value, tiled=True)
        if activated is not None:
            return self.out.matmul(activated).view(*lead, -1)
    return self.out(swiglu(gate, value)).view(*lead, -1)


def _normalized(hidden_states, scale, norm, *consumers):
    """FP8 straight out of the LayerNorm when every consumer is an MXFP8 linear."""
    if all(isinstance(consumer, MXFP8Linear) for consumer in consumers):
        fused = layer_norm_scale_quantize(hidden_states, scale, norm, tiled=True)
        if fused is not None:
            return fused
    return layer_norm_scale(hidden_states, scale, norm)


def install_mx_fused_decode(transformer, sage=False):
    """Install the composed decode path.  Prefill keeps the native block forward."""
    cache = {"modulation": None, "values": None}
    transformer._qw_modulation_cache = cache
    for block in transformer.transformer_blocks:
        eager = block.forward
        block.attn.set_processor(MXFusedProcessor(block.attn.processor, sage=sage))
        block.img_mlp.forward = types.MethodType(_mx_mlp_forward, block.img_mlp)
        if getattr(block.img_mlp, "_mx_gate_up", None) is None:
            fuse_gate_up(block.img_mlp)
        if getattr(block.attn, "_mx_qkv", None) is None:
            fuse_qkv(block.attn)

        def forward(*args, _block=block, _eager=eager, **kwargs):
            if kwargs.get("kv_cache_mode") != "cached":
                return _eager(*args, **kwargs)
            h, modulation = kwargs["hidden_states"], kwargs["modulation"]
            s1, g1, s2, g2 = modulation_values(cache, modulation)
            attn_kwargs = {k: v for k, v in kwargs.items()
                           if k not in {"hidden_states", "modulation", "target_token_mask"}}
            attn = _block.attn
            x = _normalized(h, s1, _block.img_norm1, attn.to_q, attn.to_k, attn.to_v)
            h = residual(h, attn(hidden_states=x, **attn_kwargs), g1)
            mlp = _block.img_mlp
            x = _normalized(h, s2, _block.img_norm2, mlp.gate_layer, mlp.proj)
            return residual(h, mlp(x), g2)
        block.forward = forward
