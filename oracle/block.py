"""Oracle composition of one MMDiT block minus the attention core.

TEST INFRASTRUCTURE ONLY (imported by tests/, smoke() and bench.py's
cpu_baseline leg).  Composes the oracle's functions in the block order of the
reference's MXFP8 decode path (src/qwen_image_accel/optimizations/
quantized_decode.py:117-135; eager block WHL!transformer_qwenimage21.py:
615-649) with the MMDiT shift/scale/gate modulation and the attention stand-in
o = v.  All tensors are numpy bf16 bit patterns (uint16).
"""
import numpy as np

from oracle import oracle as O


def _interleave(gate, up, group=32):
    f, k = gate.shape
    return np.stack([gate.reshape(f // group, group, k), up.reshape(f // group, group, k)],
                    1).reshape(2 * f, k)


def block_forward(h, mod, freqs, w, heads, eps=1e-6, return_stages=False):
    """h: (B, S, D); mod: (B, 6, D) rows (shift1, scale1, gate1, shift2, scale2,
    gate2); freqs: (S, Dh/2, 2) float32; w: dict of bf16-bit weights qkv (3D, D),
    out (D, D), gate (F, D), up (F, D), down (D, F), norm_q, norm_k (Dh,)."""
    B, S, D = h.shape
    M = B * S
    hd = D // heads
    shift1, scale1, g1, shift2, scale2, g2 = (mod[:, i] for i in range(6))
    gate1 = O.f32_to_bf16(np.tanh(O.bf16_to_f32(g1).astype(np.float64)).astype(np.float32))
    gate2 = O.f32_to_bf16(np.tanh(O.bf16_to_f32(g2).astype(np.float64)).astype(np.float32))
    st = {}

    xq, xs = O.adaln_quantize(h, scale1, shift1, add_one=True, eps=eps)
    wq, ws = O.mx_quantize(w["qkv"])
    qkv = O.f32_to_bf16(O.mx_gemm(xq, xs, wq, ws)[:M])                    # (M, 3D)
    st["qkv"] = qkv
    q = qkv[:, :D].reshape(B, S, heads, hd)
    k = qkv[:, D:2 * D].reshape(B, S, heads, hd)
    oq, ok, _ = O.norm_rope_pack(q, k, q, w["norm_q"], w["norm_k"], freqs, epsq=eps, epsk=eps)
    st["q"], st["k"] = oq, ok
    v = np.ascontiguousarray(qkv[:, 2 * D:])
    aq, as_ = O.mx_quantize(v)
    oq_w, os_w = O.mx_quantize(w["out"])
    proj = O.f32_to_bf16(O.mx_gemm(aq, as_, oq_w, os_w)[:M]).reshape(B, S, D)
    h1 = O.residual(h, proj, gate1)
    st["h1"] = h1
    x2q, x2s = O.adaln_quantize(h1, scale2, shift2, add_one=True, eps=eps)
    gu_q, gu_s = O.mx_quantize(_interleave(w["gate"], w["up"]))
    acc = O.mx_gemm(x2q, x2s, gu_q, gu_s)[:M]
    F = acc.shape[1] // 2
    accg = acc.reshape(M, F // 32, 2, 32)[:, :, 0].reshape(M, F)
    accu = acc.reshape(M, F // 32, 2, 32)[:, :, 1].reshape(M, F)
    act_q, act_s = O.swiglu_quantize(O.f32_to_bf16(accg), O.f32_to_bf16(accu))
    dq, ds = O.mx_quantize(w["down"])
    down = O.f32_to_bf16(O.mx_gemm(act_q, act_s, dq, ds)[:M]).reshape(B, S, D)
    h2 = O.residual(h1, down, gate2)
    return (h2, st) if return_stages else h2
