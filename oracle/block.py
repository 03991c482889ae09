"""Oracle composition of one MMDiT block minus the attention core.

TEST INFRASTRUCTURE ONLY (imported by tests/, smoke() and bench.py's
cpu_baseline leg).  Composes the oracle's functions in the block order of the
reference's MXFP8 decode path (src/qwen_image_accel/optimizations/
quantized_decode.py:117-135; eager block WHL!transformer_qwenimage21.py:
615-649) with the MMDiT shift/scale/gate modulation and the attention stand-in
o = v.  All tensors are numpy bf16 bit patterns (uint16).

Every step of this block is local to a token row (LayerNorm, the per-row
MXFP8 blocks, each GEMM row, RMSNorm + RoPE at the token's position, the
residuals, SwiGLU), so ``rows=`` computes the block for a subset of the
B * S token rows only: the large configurations are checked on sampled rows.
"""
import numpy as np

from oracle import oracle as O


def interleave_gate_up(gate, up, group=32):
    """The SwiGLU weight with gate and up rows alternating in groups of 32."""
    f, k = gate.shape
    return np.stack([gate.reshape(f // group, group, k), up.reshape(f // group, group, k)],
                    1).reshape(2 * f, k)


def split_gate_up(acc, group=32):
    """(n, 2F) GEMM output of an interleaved weight -> gate (n, F), up (n, F)."""
    n, two_f = acc.shape
    pairs = acc.reshape(n, two_f // (2 * group), 2, group)
    return pairs[:, :, 0].reshape(n, -1), pairs[:, :, 1].reshape(n, -1)


def quantize_weights(w):
    """MXFP8 codes and scales of the block's weights (as MXFP8Linear holds
    them: rows = output features), gate/up interleaved."""
    return {"qkv": O.mx_quantize(w["qkv"]), "out": O.mx_quantize(w["out"]),
            "gate_up": O.mx_quantize(interleave_gate_up(w["gate"], w["up"])),
            "down": O.mx_quantize(w["down"])}


def tanh_bf16(g):
    return O.f32_to_bf16(np.tanh(O.bf16_to_f32(g).astype(np.float64)).astype(np.float32))


def _by_batch(bid, fn, *row_args):
    """Apply fn(b, *rows_of_batch_b) to each batch's rows and reassemble."""
    out = None
    for b in np.unique(bid):
        m = bid == b
        part = fn(int(b), *[a[m] for a in row_args])
        if out is None:
            out = np.empty((bid.size,) + part.shape[1:], dtype=part.dtype)
        out[m] = part
    return out


def modulate_quantize(x_rows, bid, scale, shift, eps):
    """MXFP8(LN(x) * (1 + scale[b]) + shift[b]) of the given rows (n, D)."""
    y = _by_batch(bid, lambda b, xr: O.adaln(xr[None], scale[b][None], shift[b][None], eps=eps,
                                            add_one=True)[0], x_rows)
    return O.mx_quantize(y)       # == adaln_quantize byte for byte (tests/test_oracle.py)


def gated_residual(h_rows, x_rows, bid, gate):
    return _by_batch(bid, lambda b, hr, xr: O.residual(hr[None], xr[None], gate[b][None])[0], h_rows, x_rows)


def gemm_bf16(aq, as_, wq_ws, n):
    return O.f32_to_bf16(O.mx_gemm(aq, as_, *wq_ws)[:n])


def block_forward(h, mod, freqs, w, heads, eps=1e-6, return_stages=False, rows=None, wq=None):
    """h: (B, S, D); mod: (B, 6, D) rows (shift1, scale1, gate1, shift2, scale2,
    gate2); freqs: (S, Dh/2, 2) float32; w: dict of bf16-bit weights qkv (3D, D),
    out (D, D), gate (F, D), up (F, D), down (D, F), norm_q, norm_k (Dh,).
    rows: token rows (indices into the B * S rows) to compute, default all;
    the result is (B, S, D) for all rows, else (len(rows), D).  wq: the
    quantize_weights(w) of these weights, if already computed."""
    B, S, D = h.shape
    sel = np.arange(B * S) if rows is None else np.asarray(rows, dtype=np.int64)
    n = sel.size
    bid, tok = sel // S, sel % S
    hd = D // heads
    wq = quantize_weights(w) if wq is None else wq
    shift1, scale1, g1, shift2, scale2, g2 = (mod[:, i] for i in range(6))
    gate1, gate2 = tanh_bf16(g1), tanh_bf16(g2)
    hs = h.reshape(B * S, D)[sel]
    st = {}

    x1 = modulate_quantize(hs, bid, scale1, shift1, eps)
    st["x1"] = x1
    qkv = gemm_bf16(*x1, wq["qkv"], n)                                      # (n, 3D)
    st["qkv_plain"] = qkv
    q = qkv[:, :D].reshape(1, n, heads, hd)
    k = qkv[:, D:2 * D].reshape(1, n, heads, hd)
    oq, ok, _ = O.norm_rope_pack(q, k, q, w["norm_q"], w["norm_k"], freqs[tok], epsq=eps, epsk=eps)
    st["q"], st["k"] = oq.reshape(n, D), ok.reshape(n, D)
    v = np.ascontiguousarray(qkv[:, 2 * D:])                               # attention stand-in o = v
    st["v"] = v
    proj = gemm_bf16(*O.mx_quantize(v), wq["out"], n)
    h1 = gated_residual(hs, proj, bid, gate1)
    st["h1"] = h1
    x2 = modulate_quantize(h1, bid, scale2, shift2, eps)
    st["x2"] = x2
    accg, accu = split_gate_up(O.mx_gemm(*x2, *wq["gate_up"])[:n])
    act = O.swiglu_quantize(O.f32_to_bf16(accg), O.f32_to_bf16(accu))
    st["a"] = act
    down = gemm_bf16(*act, wq["down"], n)
    h2 = gated_residual(h1, down, bid, gate2)
    st["h2"] = h2
    out = h2.reshape(B, S, D) if rows is None else h2
    return (out, st) if return_stages else out
