"""Selective BF16 fusion of the cached-decode block (the ``fused`` profile).

Reference interface: src/qwen_image_accel/optimizations/fusion.py --
``FusedRopeProcessor`` (:12-35) and ``install_fused_decode`` (:38-60).  The
block keeps its native GEMMs and attention; LayerNorm x scale, Q/K RMSNorm +
RoPE + prefix K/V pack and the gated residuals run in this build's kernels.
Prefill (any ``kv_cache_mode`` other than "cached") keeps the native forward.
"""
import torch

from qwen_image_accel.kernels.attention import prepare_attention_inputs
from qwen_image_accel.kernels.elementwise import residual, rope_qk
from qwen_image_accel.kernels.layernorm import layer_norm_scale
from qwen_image_accel.optimizations.attention_call import attention, qim_backend


class FusedRopeProcessor:
    """Cached-decode attention: native Q/K/V projections, fused norm + RoPE + pack.

    ``native`` is the processor it replaces; it still serves prefill."""

    def __init__(self, native=None):
        self.native = native

    def __call__(self, attn, hidden_states, attention_mask=None, rotary_emb=None,
                 layer_cache=None, kv_cache_mode=None, cache_write_slice=None,
                 segments=None, key_valid=None):
        if kv_cache_mode != "cached":
            return self.native(attn, hidden_states, attention_mask, rotary_emb, layer_cache,
                               kv_cache_mode, cache_write_slice, segments, key_valid)
        q = attn.to_q(hidden_states).unflatten(-1, (attn.heads, -1))
        k = attn.to_k(hidden_states).unflatten(-1, (attn.heads, -1))
        v = attn.to_v(hidden_states).unflatten(-1, (attn.heads, -1))
        return _attend(self, attn, q, k, v, attention_mask, rotary_emb, layer_cache)


def _attend(processor, attn, q, k, v, attention_mask, rotary_emb, layer_cache):
    """Shared tail of the cached processors: norm + RoPE + pack, attention, out proj."""
    cached_k, cached_v = layer_cache.get()
    prepared = prepare_attention_inputs(q, k, v, attn.norm_q, attn.norm_k, rotary_emb, cached_k, cached_v)
    if prepared is not None:
        q, k, v = prepared
    else:
        q, k = attn.norm_q(q).to(v.dtype), attn.norm_k(k).to(v.dtype)
        if rotary_emb is not None:
            q, k = _rope(q, k, rotary_emb)
        k, v = torch.cat([cached_k, k], dim=1), torch.cat([cached_v, v], dim=1)
    out_proj = attn.to_out[0]
    if getattr(out_proj, "weight_tiled", None) is not None and qim_backend(q, k, v, attention_mask):
        # MXFP8 out-projection after this build's attention core: the core
        # writes the projection's MXFP8 input itself (qim_attention_mxfp8),
        # the same bytes MXFP8Linear.forward would quantize.
        from qwen_image_accel.kernels.attention import attention_mxfp8
        lead = q.shape[:2]
        return attn.to_out[1](out_proj.matmul(attention_mxfp8(q, k, v)).view(*lead, -1))
    result = attention(q, k, v, attention_mask, getattr(processor, "native", None))
    return attn.to_out[1](out_proj(result.flatten(2, 3).to(q.dtype)))


def _rope(q, k, freqs):
    if q.is_cuda and q.dtype == torch.bfloat16 and q.is_contiguous() and k.is_contiguous():
        return rope_qk(q, k, freqs)
    def one(x):  # apply_rotary_emb_qwen(use_real=False), the eager definition
        xr = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
        return torch.view_as_real(xr * freqs.unsqueeze(1)).flatten(3).type_as(x)
    return one(q), one(k)


def modulation_values(cache, modulation):
    """(1 + s1, tanh g1, 1 + s2, tanh g2) as (B, 1, D), computed once per step
    and keyed by the modulation tensor's identity (fusion.py:48-53).  The
    trailing modulation row belongs to the cached prefix, not the target."""
    if cache["modulation"] is not modulation:
        s1, g1, s2, g2 = modulation[:-1].chunk(4, dim=-1)
        cache["modulation"] = modulation
        cache["values"] = (1 + s1[:, None], g1[:, None].tanh(), 1 + s2[:, None], g2[:, None].tanh())
    return cache["values"]


def install_fused_decode(transformer):
    cache = {"modulation": None, "values": None}
    transformer._qw_modulation_cache = cache
    for block in transformer.transformer_blocks:
        eager = block.forward
        block.attn.set_processor(FusedRopeProcessor(block.attn.processor))

        def forward(*args, _block=block, _eager=eager, **kwargs):
            if kwargs.get("kv_cache_mode") != "cached":
                return _eager(*args, **kwargs)
            h, modulation = kwargs["hidden_states"], kwargs["modulation"]
            s1, g1, s2, g2 = modulation_values(cache, modulation)
            x = layer_norm_scale(h, s1, _block.img_norm1)
            attn_kwargs = {k: v for k, v in kwargs.items()
                           if k not in {"hidden_states", "modulation", "target_token_mask"}}
            h = residual(h, _block.attn(hidden_states=x, **attn_kwargs), g1)
            x = layer_norm_scale(h, s2, _block.img_norm2)
            return residual(h, _block.img_mlp(x), g2)
        block.forward = forward
