"""The cached-decode block of the ``fused`` and ``mxfp8`` profiles.

Reference interface: optimizations/fusion.py (``install_fused_decode``
:38-60, ``FusedRopeProcessor`` :12-35) and optimizations/quantized_decode.py
(``install_mx_fused_decode`` :108-137, ``MXFusedProcessor`` :31-78, the MLP
:81-96, the normalisation :99-105); the eager block they replace is
WHL!diffusers/models/transformers/transformer_qwenimage21.py:615-649.

One installer serves both profiles.  For every block it decides, once, how
each stage of a cached decode step runs -- from the profile and from what the
block holds after conversion (which linears are ``MXFP8Linear``, whether the
stacked Q/K/V and interleaved gate/up weights were built):

    stage      fused (bf16)                     mxfp8
    norm1/2    layer_norm_scale                 layer_norm_scale_quantize when every
                                                consumer is MXFP8 (one shared activation)
    qkv        to_q / to_k / to_v               one stacked GEMM, or three GEMMs on the
                                                shared activation
    prepare    prepare_attention_inputs (fused RMSNorm + RoPE + prefix pack), else the
               eager RMSNorm, RoPE and concatenation
    attention  Diffusers' dispatch, or this build's core (QW21_ATTENTION_BACKEND=qim),
               which also writes an MXFP8 out-projection's input
    mlp        img_mlp (SwiGLU hook)            gate/up GEMM with the SwiGLU -> MXFP8
                                                epilogue, or two GEMMs + swiglu_quantize
    residual   residual(h, branch, tanh g)

Prefill (any ``kv_cache_mode`` other than "cached") runs the block's own
forward and the attention processor it replaced.
"""
import torch

from qwen_image_accel.kernels.attention import attention_mxfp8, prepare_attention_inputs
from qwen_image_accel.kernels.bf16 import swiglu
from qwen_image_accel.kernels.elementwise import residual, rope_qk
from qwen_image_accel.kernels.epilogue import layer_norm_scale_quantize, swiglu_quantize
from qwen_image_accel.kernels.gemm import mx_matmul
from qwen_image_accel.kernels.layernorm import layer_norm_scale
from qwen_image_accel.kernels.mxfp8 import Quantized, quantize
from qwen_image_accel.optimizations.attention_call import attention, qim_backend
from qwen_image_accel.optimizations.mxfp8 import MXFP8Linear
from qwen_image_accel.weights import fuse_gate_up, fuse_qkv

# Keyword arguments of a block call that the attention module does not take.
BLOCK_ONLY = frozenset({"hidden_states", "modulation", "target_token_mask"})


class StepTerms:
    """The per-step modulation terms (1 + s1, tanh g1, 1 + s2, tanh g2), each
    (B, 1, D), from a cached step's (B + 1, 4D) modulation (its last row is
    the cached prefix's).  Computed once per modulation tensor; the state is
    the dict ``transformer._qw_modulation_cache`` (key "modulation": the
    tensor they belong to, so setting it to None forces a recompute)."""

    def __init__(self, transformer):
        self.state = {"modulation": None, "values": None}
        transformer._qw_modulation_cache = self.state

    def __call__(self, modulation):
        if self.state["modulation"] is not modulation:
            s1, g1, s2, g2 = modulation[:-1, None].unflatten(-1, (4, -1)).unbind(-2)
            self.state["values"] = (1 + s1, g1.tanh(), 1 + s2, g2.tanh())
            self.state["modulation"] = modulation
        return self.state["values"]


def all_mxfp8(*linears):
    return all(isinstance(m, MXFP8Linear) for m in linears)


def shared_activation(x, consumers):
    """One MXFP8 activation for several MXFP8 consumers: x itself when a norm
    already emitted it, x quantized once when it is a contiguous bf16 tensor
    and every consumer is MXFP8, else None (the consumers run on bf16)."""
    if isinstance(x, Quantized):
        return x
    if all_mxfp8(*consumers) and x.is_contiguous():
        return quantize(x.reshape(-1, x.shape[-1]), tiled=True)
    return None


# ------------------------------------------------------------ attention --

def project_qkv(attn, x, quantized):
    """(q, k, v), each (B, S, heads, head_dim)."""
    linears = (attn.to_q, attn.to_k, attn.to_v)
    shared = shared_activation(x, linears) if quantized else None
    if shared is None:
        return tuple(p(x).unflatten(-1, (attn.heads, -1)) for p in linears)
    lead = shared.shape[:-1]
    stacked = getattr(attn, "_mx_qkv", None)
    if stacked is None:
        return tuple(p.matmul(shared).view(*lead, attn.heads, -1) for p in linears)
    # One GEMM over the stacked weight; q, k, v are column blocks of its output
    # (one token stride), which the fused norm + RoPE + pack reads in place.
    return mx_matmul(shared, *stacked, weight_tiled=True).view(*lead, 3, attn.heads, -1).unbind(-3)


def _eager_rope(q, k, freqs):
    if q.is_cuda and q.dtype == torch.bfloat16 and q.is_contiguous() and k.is_contiguous():
        return rope_qk(q, k, freqs)

    def rotate(x):  # apply_rotary_emb_qwen(use_real=False)
        pairs = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
        return torch.view_as_real(pairs * freqs.unsqueeze(1)).flatten(3).type_as(x)
    return rotate(q), rotate(k)


def attention_inputs(attn, q, k, v, freqs, layer_cache):
    """Q/K RMSNorm + RoPE, and the cached prefix K/V in front of k and v."""
    prefix_k, prefix_v = layer_cache.get()
    fused = prepare_attention_inputs(q, k, v, attn.norm_q, attn.norm_k, freqs, prefix_k, prefix_v)
    if fused is not None:
        return fused
    q, k = attn.norm_q(q).to(v.dtype), attn.norm_k(k).to(v.dtype)
    if freqs is not None:
        q, k = _eager_rope(q, k, freqs)
    return q, torch.cat([prefix_k, k], dim=1), torch.cat([prefix_v, v], dim=1)


def attend_and_project(attn, q, k, v, mask, native):
    out_proj, dropout = attn.to_out[0], attn.to_out[1]
    if isinstance(out_proj, MXFP8Linear) and qim_backend(q, k, v, mask):
        # This build's attention core writes the MXFP8 out-projection's input
        # itself: the bytes MXFP8Linear.forward would quantize from its output.
        return dropout(out_proj.matmul(attention_mxfp8(q, k, v)).view(*q.shape[:2], -1))
    o = attention(q, k, v, mask, native)
    return dropout(out_proj(o.flatten(2, 3).to(q.dtype)))


class CachedDecodeProcessor:
    """Attention processor of the cached decode step: projections, fused
    norm + RoPE + prefix pack, attention core, out projection.  Other
    ``kv_cache_mode`` values go to ``native``, the processor it replaced."""

    quantized = False

    def __init__(self, native=None):
        self.native = native

    def __call__(self, attn, hidden_states, attention_mask=None, rotary_emb=None, layer_cache=None,
                 kv_cache_mode=None, cache_write_slice=None, segments=None, key_valid=None):
        if kv_cache_mode != "cached":
            return self.native(attn, hidden_states, attention_mask, rotary_emb, layer_cache, kv_cache_mode,
                               cache_write_slice, segments, key_valid)
        q, k, v = project_qkv(attn, hidden_states, self.quantized)
        q, k, v = attention_inputs(attn, q, k, v, rotary_emb, layer_cache)
        return attend_and_project(attn, q, k, v, attention_mask, self.native)


class FusedRopeProcessor(CachedDecodeProcessor):
    """The ``fused`` profile's processor: bf16 projections."""


class MXFusedProcessor(CachedDecodeProcessor):
    """The ``mxfp8`` profile's processor: MXFP8 projections on one shared
    activation.  ``sage=True`` (SageAttention2) is outside this build."""

    quantized = True

    def __init__(self, native=None, sage=False):
        if sage:
            raise NotImplementedError("SageAttention2 decode is outside this build; use the mxfp8 profile")
        super().__init__(native)
        self.sage = False


# ------------------------------------------------------------------ MLP --

class QuantizedSwiGLU:
    """``img_mlp.forward`` of the mxfp8 profile: gate and value projections on
    one shared MXFP8 activation, SwiGLU straight to the down projection's
    MXFP8 input (in the interleaved gate/up GEMM's epilogue when that weight
    exists)."""

    def __init__(self, mlp):
        self.mlp = mlp

    def __call__(self, x):
        mlp = self.mlp
        shared = shared_activation(x, (mlp.gate_layer, mlp.proj))
        if shared is None:
            return mlp.out(swiglu(mlp.gate_layer(x), mlp.proj(x)))
        lead = shared.shape[:-1]
        to_mxfp8 = isinstance(mlp.out, MXFP8Linear)
        gate_up = getattr(mlp, "_mx_gate_up", None)
        if gate_up is not None and to_mxfp8:
            act = mx_matmul(shared, *gate_up, epilogue="swiglu_quant", weight_tiled=True, out_tiled=True)
            return mlp.out.matmul(act).view(*lead, -1)
        gate, value = mlp.gate_layer.matmul(shared), mlp.proj.matmul(shared)
        act = swiglu_quantize(gate, value, tiled=True) if to_mxfp8 else None
        if act is None:
            return mlp.out(swiglu(gate, value)).view(*lead, -1)
        return mlp.out.matmul(act).view(*lead, -1)


# ---------------------------------------------------------------- block --

class DecodeBlock:
    """A block's forward: cached decode through the stages above, anything
    else through the block's own forward."""

    def __init__(self, block, terms, quantized):
        self.block, self.eager, self.terms, self.quantized = block, block.forward, terms, quantized

    def normalize(self, h, scale, norm, consumers):
        if self.quantized and all_mxfp8(*consumers):
            x = layer_norm_scale_quantize(h, scale, norm, tiled=True)
            if x is not None:
                return x
        return layer_norm_scale(h, scale, norm)

    def __call__(self, *args, **kwargs):
        if kwargs.get("kv_cache_mode") != "cached":
            return self.eager(*args, **kwargs)
        blk = self.block
        h = kwargs["hidden_states"]
        scale1, gate1, scale2, gate2 = self.terms(kwargs["modulation"])
        attn_kwargs = {name: value for name, value in kwargs.items() if name not in BLOCK_ONLY}
        x = self.normalize(h, scale1, blk.img_norm1, (blk.attn.to_q, blk.attn.to_k, blk.attn.to_v))
        h = residual(h, blk.attn(hidden_states=x, **attn_kwargs), gate1)
        x = self.normalize(h, scale2, blk.img_norm2, (blk.img_mlp.gate_layer, blk.img_mlp.proj))
        return residual(h, blk.img_mlp(x), gate2)


def install_cached_decode(transformer, quantized):
    """Install the cached-decode block on every block of ``transformer``
    (``quantized``: the mxfp8 profile's stages, after quantize_transformer)."""
    terms = StepTerms(transformer)
    processor = MXFusedProcessor if quantized else FusedRopeProcessor
    for block in transformer.transformer_blocks:
        block.attn.set_processor(processor(block.attn.processor))
        if quantized:
            if getattr(block.img_mlp, "_mx_gate_up", None) is None:
                fuse_gate_up(block.img_mlp)
            if getattr(block.attn, "_mx_qkv", None) is None:
                fuse_qkv(block.attn)
            block.img_mlp.forward = QuantizedSwiGLU(block.img_mlp)
        block.forward = DecodeBlock(block, terms, quantized)
