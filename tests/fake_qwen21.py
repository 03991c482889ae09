"""A tiny stand-in for Diffusers' QwenImage21 transformer, enough to exercise
the profile installers (Diffusers is not installed here).

It follows the eager semantics of the block the reference patches
(WHL!diffusers/models/transformers/transformer_qwenimage21.py:604-649:
LayerNorm without affine, scale/gate modulation, RMSNorm on Q/K, complex RoPE,
prefix K/V cache, SwiGLU MLP) and the call protocol the installers rely on:
``block.forward(hidden_states=..., modulation=..., rotary_emb=...,
kv_cache_mode=..., layer_cache=...)``, ``attn.processor`` /
``attn.set_processor``, ``layer_cache.get()``.  In cached decode the
modulation carries one trailing row for the prefix, which the target rows do
not use (optimizations/fusion.py:48-53; pipeline.py:76-86).
"""
import types

import torch
import torch.nn.functional as F
from torch import nn


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))
        self.bias = None

    def forward(self, x):
        var = x.to(torch.float32).pow(2).mean(-1, keepdim=True)
        x = x * torch.rsqrt(var + self.eps)
        if self.weight.dtype in (torch.float16, torch.bfloat16):
            x = x.to(self.weight.dtype)
        return x * self.weight


def apply_rotary(x, freqs):
    xr = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
    return torch.view_as_real(xr * freqs.unsqueeze(1)).flatten(3).type_as(x)


class NativeProcessor:
    """The eager attention processor (prefill and cached decode)."""

    def __call__(self, attn, hidden_states, attention_mask=None, rotary_emb=None, layer_cache=None,
                 kv_cache_mode=None, cache_write_slice=None, segments=None, key_valid=None):
        q = attn.to_q(hidden_states).unflatten(-1, (attn.heads, -1))
        k = attn.to_k(hidden_states).unflatten(-1, (attn.heads, -1))
        v = attn.to_v(hidden_states).unflatten(-1, (attn.heads, -1))
        q, k = attn.norm_q(q).to(v.dtype), attn.norm_k(k).to(v.dtype)
        if rotary_emb is not None:
            q, k = apply_rotary(q, rotary_emb), apply_rotary(k, rotary_emb)
        if kv_cache_mode == "cached":
            ck, cv = layer_cache.get()
            k, v = torch.cat([ck, k], 1), torch.cat([cv, v], 1)
        o = F.scaled_dot_product_attention(q.transpose(1, 2).float(), k.transpose(1, 2).float(),
                                           v.transpose(1, 2).float()).transpose(1, 2).to(q.dtype)
        return attn.to_out[1](attn.to_out[0](o.flatten(2, 3)))


class Attention(nn.Module):
    def __init__(self, dim, heads):
        super().__init__()
        self.heads = heads
        hd = dim // heads
        self.to_q, self.to_k, self.to_v = (nn.Linear(dim, dim, bias=False) for _ in range(3))
        self.to_out = nn.ModuleList([nn.Linear(dim, dim, bias=False), nn.Dropout(0.0)])
        self.norm_q, self.norm_k = RMSNorm(hd), RMSNorm(hd)
        self.processor = NativeProcessor()

    def set_processor(self, p):
        self.processor = p

    def forward(self, hidden_states, **kw):
        return self.processor(self, hidden_states, **kw)


class SwiGLU(nn.Module):
    def __init__(self, dim, hidden):
        super().__init__()
        self.proj = nn.Linear(dim, hidden, bias=False)
        self.out = nn.Linear(hidden, dim, bias=False)
        self.gate_layer = nn.Linear(dim, hidden, bias=False)

    def forward(self, x):
        return self.out(F.silu(self.gate_layer(x)) * self.proj(x))


class Block(nn.Module):
    def __init__(self, dim, heads, ffn):
        super().__init__()
        self.img_norm1 = nn.LayerNorm(dim, elementwise_affine=False, eps=1e-6)
        self.attn = Attention(dim, heads)
        self.img_norm2 = nn.LayerNorm(dim, elementwise_affine=False, eps=1e-6)
        self.img_mlp = SwiGLU(dim, ffn)

    def forward(self, hidden_states, modulation, rotary_emb=None, attention_mask=None,
                target_token_mask=None, layer_cache=None, kv_cache_mode=None, cache_write_slice=None,
                segments=None, key_valid=None):
        if kv_cache_mode == "cached":
            modulation = modulation[:-1]
        mod1, mod2 = modulation[:, None].chunk(2, dim=-1)
        s1, g1 = mod1.chunk(2, dim=-1)
        s2, g2 = mod2.chunk(2, dim=-1)
        x = self.img_norm1(hidden_states) * (1 + s1)
        o = self.attn(hidden_states=x, attention_mask=attention_mask, rotary_emb=rotary_emb,
                      layer_cache=layer_cache, kv_cache_mode=kv_cache_mode)
        hidden_states = hidden_states + g1.tanh() * o
        x = self.img_norm2(hidden_states) * (1 + s2)
        return hidden_states + g2.tanh() * self.img_mlp(x)


class LayerCache:
    def __init__(self, k, v):
        self.k, self.v = k, v

    def get(self):
        return self.k, self.v


def make_transformer(n_blocks=2, dim=256, heads=2, ffn=512, dtype=torch.bfloat16, device="cpu", seed=0):
    torch.manual_seed(seed)
    blocks = nn.ModuleList([Block(dim, heads, ffn) for _ in range(n_blocks)])
    for b in blocks:
        for m in b.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, std=0.02)
        with torch.no_grad():
            b.attn.norm_q.weight.uniform_(0.8, 1.2)
            b.attn.norm_k.weight.uniform_(0.8, 1.2)
    t = types.SimpleNamespace(transformer_blocks=blocks.to(device=device, dtype=dtype), dtype=dtype)
    return t


def make_inputs(dim=256, heads=2, tokens=64, prefix=16, batch=1, dtype=torch.bfloat16, device="cpu", seed=1):
    g = torch.Generator().manual_seed(seed)
    hd = dim // heads
    h = torch.randn(batch, tokens, dim, generator=g).to(dtype)
    modulation = (torch.randn(batch + 1, 4 * dim, generator=g) * 0.1).to(dtype)
    phase = torch.randn(tokens, hd // 2, generator=g)
    freqs = torch.polar(torch.ones_like(phase), phase)
    ck = torch.randn(batch, prefix, heads, hd, generator=g).to(dtype)
    cv = torch.randn(batch, prefix, heads, hd, generator=g).to(dtype)
    to = lambda x: x.to(device)
    return to(h), to(modulation), to(freqs), LayerCache(to(ck), to(cv))


# ------------------------------------------------- stand-in pipeline --

class FlowEulerScheduler:
    """Euler steps of a flow-matching sampler over noise levels 1 -> 0:
    x <- x + (sigma[i+1] - sigma[i]) * v, in fp32, stored in the latent dtype."""

    def __init__(self, steps):
        self.sigmas = torch.linspace(1.0, 0.0, steps + 1)

    def step(self, velocity, index, sample):
        dt = float(self.sigmas[index + 1] - self.sigmas[index])
        return ((sample.float() + dt * velocity.float()).to(sample.dtype),)


class StandInTransformer(nn.Module):
    """The blocks as a denoiser: the latent enters as the hidden states, the
    step's modulation is a fixed base scaled by (1 + sigma), every block runs
    in cached decode against the shared prefix K/V, and the velocity is what
    the blocks add to the hidden states.  The base's gate terms are 10x those
    of make_inputs, so that each block adds O(0.1) to the O(1) stream and the
    velocity sits well above the bf16 rounding of the hidden states."""

    def __init__(self, t, inputs):
        super().__init__()
        self.transformer_blocks = t.transformer_blocks
        self.dtype = t.dtype
        _, mod, freqs, cache = inputs
        d = mod.shape[-1] // 4
        mod = mod.float().clone()
        mod[:, d:2 * d] *= 10
        mod[:, 3 * d:] *= 10
        # buffers, so that .to(device) moves them with the blocks
        self.register_buffer("mod", mod.to(t.dtype))
        self.register_buffer("freqs", freqs)
        self.register_buffer("cache_k", cache.k)
        self.register_buffer("cache_v", cache.v)

    def forward(self, hidden_states, sigma):
        h = hidden_states
        mod = (self.mod.float() * (1.0 + sigma)).to(self.mod.dtype)
        cache = LayerCache(self.cache_k, self.cache_v)
        for b in self.transformer_blocks:
            h = b(hidden_states=h, modulation=mod, rotary_emb=self.freqs, layer_cache=cache, kv_cache_mode="cached")
        return (h - hidden_states,)


class StandInPipeline:
    """transformer + scheduler + a denoising loop: the parts of a Diffusers
    pipeline that teacher-forced replay touches."""

    def __init__(self, transformer, steps):
        self.transformer = transformer
        self.scheduler = FlowEulerScheduler(steps)
        self.steps = steps

    def __call__(self, latents):
        for i in range(self.steps):
            v = self.transformer(latents, float(self.scheduler.sigmas[i]))[0]
            latents = self.scheduler.step(v, i, latents)[0]
        return latents


def make_pipeline(steps=6, n_blocks=2, dim=256, heads=2, ffn=512, tokens=64, prefix=16, device="cpu"):
    """A fresh stand-in pipeline (same weights and inputs for every call) and
    its starting latent."""
    t = make_transformer(n_blocks=n_blocks, dim=dim, heads=heads, ffn=ffn, device=device)
    inputs = make_inputs(dim=dim, heads=heads, tokens=tokens, prefix=prefix, device=device)
    return StandInPipeline(StandInTransformer(t, inputs), steps), inputs[0]
