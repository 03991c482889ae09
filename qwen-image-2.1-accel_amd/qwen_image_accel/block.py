"""One MMDiT transformer block on the MXFP8 path, minus the attention core.

This is the block composition the reference's ``install_mx_fused_decode``
installs (src/qwen_image_accel/optimizations/quantized_decode.py:108-137;
eager definition WHL!diffusers/models/transformers/transformer_qwenimage21.py:
615-649), in the MMDiT form of the benchmark configuration (shift + scale + gate
modulation, fused QKV projection, hidden 3072, 24 heads x 128, FFN 12288):

    x   = MXFP8(LN(h) * (1 + scale1) + shift1)             qim_adaln_quantize
    qkv = x @ W_qkv; q,k = rope(RMSNorm(q)), rope(RMSNorm(k))
                                                            qim_mxfp8_gemm_qk_norm_rope
    o   = attention(q, k, v)        -- qim_attention (attention_fn); stand-in o = v
    h   = h + tanh(g1) * (MXFP8(o) @ W_out)                 qim_mx_quantize + GEMM epilogue
          (fused_attention: V leaves the QKV GEMM as the attention's V^T
          tiles, qim_mxfp8_gemm_qk_norm_rope_vt, and MXFP8(attention(q, k,
          v)) is one pass, qim_attention_mxfp8)
    x   = MXFP8(LN(h) * (1 + scale2) + shift2)             qim_adaln_quantize
    a   = MXFP8(silu(x @ W_gate) * (x @ W_up))              GEMM, SwiGLU->MXFP8 epilogue
    h   = h + tanh(g2) * (a @ W_down)                       GEMM, gated-residual epilogue

Eight launches, all of this library: the modulation terms and the seven
above (QK-RMSNorm + RoPE run in the QKV GEMM's epilogue, head by head: each
wave of the GEMM holds whole 128-wide head rows); every MXFP8 operand (weights
and activations) is in the GEMM's tiled code layout, written that way by its
producer; every bf16 rounding point of the eager block is kept (the
activation quantizations share one FP8 tensor per consumer group, as in
quantized_decode.py:50-53, 81-96).  The modulation precompute (1 + s and
tanh(g) of the six modulation rows, one launch of qim_modulation_values) is
the reference's per-step precompute (optimizations/fusion.py:48-53).
"""
from dataclasses import dataclass

import torch

from qwen_image_accel.kernels import attention, elementwise, gemm, mxfp8
from qwen_image_accel.kernels.epilogue import layer_norm_scale_quantize


class _LayerNorm:
    """The block's affine-free LayerNorm (eps 1e-6) as the kernels' ``norm`` argument."""

    def __init__(self, dim, eps=1e-6):
        self.normalized_shape = (dim,)
        self.eps = eps
        self.elementwise_affine = False

    def __call__(self, x):
        return torch.nn.functional.layer_norm(x, self.normalized_shape, eps=self.eps)


def modulation_terms(modulation):
    """(shift1, 1 + scale1, tanh(gate1), shift2, 1 + scale2, tanh(gate2)), each
    (B, 1, D) bf16, from the (B, 6, D) modulation rows in one launch
    (qim_modulation_values): the reference's per-step precompute
    (optimizations/fusion.py:48-53) in the MMDiT layout."""
    k = elementwise
    mv = k.modulation_values(modulation.contiguous(), (k.MOD_COPY, k.MOD_ONE_PLUS, k.MOD_TANH) * 2)
    return tuple(mv[i].unsqueeze(1) for i in range(6))  # each (B, 1, D), contiguous


@dataclass
class MMDiTBlock:
    dim: int
    heads: int
    ffn: int
    w_qkv: mxfp8.Quantized      # (3*dim, dim), tiled codes
    w_out: mxfp8.Quantized      # (dim, dim), tiled codes
    w_gate_up: mxfp8.Quantized  # (2*ffn, dim), gate/up rows interleaved, tiled codes
    w_down: mxfp8.Quantized     # (dim, ffn), tiled codes
    norm_q: torch.Tensor        # (head_dim,) bf16
    norm_k: torch.Tensor
    bf16_weights: dict          # the unquantized bf16 weights (kept for checking)
    eps: float = 1e-6

    @staticmethod
    def from_weights(w_qkv, w_out, w_gate, w_up, w_down, norm_q, norm_k, heads):
        """Quantize bf16 weights once (like MXFP8Linear.__init__)."""
        dim = w_out.shape[0]
        ffn = w_gate.shape[0]
        gu = gemm.interleave_swiglu(w_gate, w_up)
        def q(w):
            return mxfp8.quantize(w, tiled=True)
        return MMDiTBlock(dim, heads, ffn, q(w_qkv), q(w_out), q(gu), q(w_down), norm_q, norm_k,
                          dict(qkv=w_qkv, out=w_out, gate=w_gate, up=w_up, down=w_down,
                               norm_q=norm_q, norm_k=norm_k))

    @staticmethod
    def random(gen, dim=3072, heads=24, ffn=12288, device="cuda", std=0.02):
        """Random-init bf16 weights ~N(0, std^2) from a CPU generator."""
        def w(*shape):
            return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16).to(device)
        hd = dim // heads
        nq = (torch.rand(hd, generator=gen) * 0.4 + 0.8).to(torch.bfloat16).to(device)
        nk = (torch.rand(hd, generator=gen) * 0.4 + 0.8).to(torch.bfloat16).to(device)
        return MMDiTBlock.from_weights(w(3 * dim, dim), w(dim, dim), w(ffn, dim), w(ffn, dim),
                                       w(dim, ffn), nq, nk, heads)

    def forward(self, h, modulation, freqs, attention_fn=None, attention_mxfp8_fn=None, fused_attention=False,
                stages=None):
        """h: (B, S, dim) bf16; modulation: (B, 6, dim) bf16 rows
        (shift1, scale1, gate1, shift2, scale2, gate2); freqs: (S, head_dim/2)
        complex64.  ``attention_fn(q, k, v) -> (B, S, dim)`` defaults to the
        stand-in that returns v.  ``attention_mxfp8_fn(q, k, v)`` (e.g.
        ``attention.attention_mxfp8``), when given, returns the attention
        output already quantized in the tiled layout (the same bytes as
        quantizing attention_fn's output) and replaces both.
        ``fused_attention=True`` runs the library's attention core with both
        of its fusions: the QKV projection writes V straight into the
        attention's V^T tiles (S % 64 == 0) and the attention writes the
        out-projection's MXFP8 input -- the same bytes as
        ``attention_fn=attention.attention``.  ``stages``: a dict that
        receives the intermediate results (x1, qkv, o, h1, x2, a) for
        checking; nothing is copied."""
        b, s, d = h.shape
        shift1, scale1, gate1, shift2, scale2, gate2 = modulation_terms(modulation)
        norm = _LayerNorm(d, self.eps)
        hd = d // self.heads

        x = layer_norm_scale_quantize(h, scale1, norm, shift=shift1, add_one=False, tiled=True)
        ws = None
        if fused_attention:
            if s % 64:
                raise ValueError(f"fused_attention needs S % 64 == 0 (S = {s})")
            ws = attention.workspace(b, s, s, self.heads, h.device)
        qkv = gemm.mx_matmul_qk_norm_rope(x, self.w_qkv.values, self.w_qkv.scales, self.norm_q, self.norm_k,
                                          freqs, self.heads, s, self.eps, self.eps, weight_tiled=True, vt=ws)
        qkv4 = qkv.view(b, s, 3 * d)
        q = qkv4[:, :, :d].unflatten(-1, (self.heads, hd))                      # normalised + rotated
        k = qkv4[:, :, d:2 * d].unflatten(-1, (self.heads, hd))
        v = qkv4[:, :, 2 * d:].unflatten(-1, (self.heads, hd))
        if fused_attention:
            oq = attention.attention_mxfp8(q, k, None, workspace=ws)   # V^T already in ws
        elif attention_mxfp8_fn is not None:
            oq = attention_mxfp8_fn(q, k, v)
        else:
            o = qkv[:, 2 * d:] if attention_fn is None else attention_fn(q, k, v).reshape(b * s, d)  # stand-in: v
            oq = mxfp8.quantize(o, tiled=True)
        h1 = self._mm(oq, self.w_out, epilogue="gated_residual", gate=gate1,
                      residual=h.reshape(b * s, d), seq=s)
        h1 = h1.view(b, s, d)
        x2 = layer_norm_scale_quantize(h1, scale2, norm, shift=shift2, add_one=False, tiled=True)
        a = self._mm(x2, self.w_gate_up, epilogue="swiglu_quant", out_tiled=True)
        if stages is not None:
            stages.update(x1=x, qkv=qkv, o=oq, h1=h1, x2=x2, a=a)
        h2 = self._mm(a, self.w_down, epilogue="gated_residual", gate=gate2,
                      residual=h1.reshape(b * s, d), seq=s)
        return h2.view(b, s, d)

    @staticmethod
    def _mm(x, w, **epilogue):
        return gemm.mx_matmul(x, w.values, w.scales, weight_tiled=True, **epilogue)

    def flops(self, tokens):
        """GEMM flops of one forward over `tokens` rows (2*M*N*K each)."""
        d, f = self.dim, self.ffn
        return 2 * tokens * (3 * d * d + d * d + 2 * f * d + d * f)
