"""Pins of the CPU oracle (oracle/qim_oracle.c) -- no GPU.

Every oracle function is checked against something that does not share its
code: torch's own CPU library routines (float8 casts, layer_norm, silu,
complex multiply), brute-force searches, float64 arithmetic, the reference
test's permute form of the scale layout, closed forms and invariants.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from tests.helpers import (bf16_close, bf16_close_chain, bf16_randn, bf16_values, bits, from_bits, rel_fro,
                           swizzle_permute)

ALL_BF16 = np.arange(65536, dtype=np.uint16)


# ------------------------------------------------------------- E4M3 / E8M0 --

def test_e4m3_encode_exhaustive_bf16_vs_torch():
    """Every finite bf16 value below the NaN threshold: oracle == torch cast."""
    v = bf16_values(ALL_BF16)
    v = v[np.isfinite(v) & (np.abs(v) < 464)]
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.e4m3_encode(v), ref)


def test_e4m3_encode_random_fp32_vs_torch():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.uniform(-448, 448, 20000), rng.uniform(-0.02, 0.02, 20000),
        np.ldexp(rng.uniform(-1, 1, 5000), rng.integers(-20, 9, 5000)),
    ]).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.e4m3_encode(v), ref)


def test_e4m3_encode_is_nearest_even_brute_force():
    """Independent of torch: the code is the nearest E4M3 value, ties to the
    even code (mantissa LSB 0)."""
    table = O.e4m3_values().astype(np.float64)
    finite = np.where(np.isfinite(table))[0]
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.uniform(-448, 448, 3000),
                           (table[finite][:-1] + table[finite][1:]) / 2]).astype(np.float32)
    codes = O.e4m3_encode(vals)
    for v, c in zip(vals, codes):
        d = np.abs(table[finite] - float(v))
        best = finite[d == d.min()]
        if len(best) > 1:  # tie: +0/-0 or a true midpoint
            best = [b for b in best if (b & 1) == 0 and (np.signbit(table[b]) == np.signbit(v) or table[b] != 0)] or best
        assert c in best or table[c] == table[best[0]], (v, c, best)


def test_e4m3_decode_all_codes_vs_torch():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(O.e4m3_values(), ref, equal_nan=True)


@pytest.mark.parametrize("amax,e", [(448.0, 127), (450.0, 128), (1.0, 119), (0.0, 0),
                                    (1.75, 119), (1.7500001, 120), (2.0 ** -140, 0)])
def test_mx_exponent_kats(amax, e):
    assert O.mx_exponent(amax) == e


def test_mx_exponent_is_smallest_power_of_two_brute_force():
    """e = min{e in [0, 254] : amax / 2^(e-127) <= 448} (clamped), searched."""
    rng = np.random.default_rng(2)
    amaxes = np.concatenate([
        np.ldexp(rng.uniform(1, 2, 3000), rng.integers(-130, 120, 3000)),
        np.ldexp(1.75, np.arange(-120, 120)), np.ldexp(1.7500001, np.arange(-120, 120)),
    ]).astype(np.float32)
    for a in amaxes:
        a = float(a)
        want = next((e for e in range(255) if a / math.ldexp(1.0, e - 127) <= 448.0), 254)
        assert O.mx_exponent(a) == want, a


def test_swizzle_index_matches_reference_permute_form():
    m, k = 256, 512
    rng = np.random.default_rng(3)
    e = rng.integers(0, 255, (m, k // 32)).astype(np.uint8)
    flat = np.zeros(m * k // 32, dtype=np.uint8)
    for r in range(m):
        for kb in range(k // 32):
            flat[O.mx_scale_index(r, kb, k)] = e[r, kb]
    assert np.array_equal(flat, swizzle_permute(e))


def _brute_quantize(xv):
    """Per-block brute force: exponent by search, codes by nearest value."""
    table = O.e4m3_values()
    m, k = xv.shape
    codes = np.zeros((m, k), dtype=np.uint8)
    exps = np.zeros((m, k // 32), dtype=np.uint8)
    finite = np.where(np.isfinite(table) & ((np.arange(256) & 0x80) == 0))[0]
    pos = table[finite].astype(np.float64)
    for r in range(m):
        for kb in range(k // 32):
            blk = xv[r, kb * 32:(kb + 1) * 32].astype(np.float64)
            amax = np.abs(blk).max()
            e = 0 if amax == 0 else next((e for e in range(255) if amax / 2.0 ** (e - 127) <= 448), 254)
            exps[r, kb] = e
            for i, x in enumerate(blk * 2.0 ** (127 - e)):
                d = np.abs(pos - abs(x))
                cand = finite[d == d.min()]
                c = cand[0] if len(cand) == 1 else [c for c in cand if c % 2 == 0][0]
                codes[r, kb * 32 + i] = c | (0x80 if np.signbit(x) else 0)
    return codes, exps


def test_mx_quantize_brute_force_and_layout():
    g = torch.Generator().manual_seed(0)
    x = bf16_randn(g, (130, 256))
    x[:, ::64] *= 40
    x[7] *= 1e-3
    x[11, 32:64] = 0
    xb = bits(x)
    q, s = O.mx_quantize(xb)
    assert q.shape == (256, 256) and s.shape == (256 * 256 // 32,)
    xp = np.zeros((256, 256), dtype=np.float32)
    xp[:130] = bf16_values(xb)
    codes, exps = _brute_quantize(xp)
    assert np.array_equal(q, codes)
    assert np.array_equal(s, swizzle_permute(exps))
    assert not q[130:].any() and not exps[130:].any()


def test_mx_quantize_vs_reference_torch_ops():
    """The reference test's own torch formulation (check_mxfp8.py:20-30),
    evaluated with torch CPU ops (exp2, float8 cast) on outlier-heavy data."""
    g = torch.Generator().manual_seed(0)
    x = bf16_randn(g, (256, 4096))
    x[:, ::512] *= 40
    x[256 // 3] *= 1e-3
    xv = x.float().view(256, 128, 32)
    amax = xv.abs().amax(-1)
    b = amax.view(torch.int32)
    e = ((b >> 23) & 0xFF) - 8 + ((b & 0x7FFFFF) > 6291456).int()
    e = torch.where(amax == 0, torch.zeros_like(e), e.clamp(0, 254))
    rq = (xv * torch.exp2((127 - e).float())[..., None]).to(torch.float8_e4m3fn)
    q, s = O.mx_quantize(bits(x))
    assert np.array_equal(q, rq.view(torch.uint8).view(256, 4096).numpy())
    assert np.array_equal(s, swizzle_permute(e.to(torch.uint8).numpy()))


def test_mx_dequantize_error_bound():
    g = torch.Generator().manual_seed(5)
    x = bf16_randn(g, (128, 512))
    q, s = O.mx_quantize(bits(x))
    d = O.mx_dequantize(q, s)
    xv = x.float().numpy()
    # |x - deq| <= half an E4M3 ulp at 2^(e-127) scale: relative 2^-4 for normals
    assert np.all(np.abs(d - xv) <= np.maximum(np.abs(xv) * 2.0 ** -4, 2.0 ** -10 * np.abs(xv).max()))


# ------------------------------------------------------------- LayerNorm --

@pytest.mark.parametrize("d", [3072, 4096])
@pytest.mark.parametrize("scale_mag", [0.001, 1.0, 20.0])
def test_layer_norm_scale_vs_torch_cpu(d, scale_mag):
    g = torch.Generator().manual_seed(717)
    x = bf16_randn(g, (2, 33, d), scale_mag)
    s = bf16_randn(g, (2, 1, d))
    ref = F.layer_norm(x, (d,), eps=1e-6) * s
    out = O.adaln(bits(x), bits(s))
    ok, worst, _ = bf16_close(out, bits(ref))
    assert ok, worst


def test_layer_norm_against_float64():
    """t0 = bf16(LN(x)) is the correctly rounded float64 LayerNorm except within
    an fp32 ulp of a rounding midpoint: at most 1 bf16 ulp anywhere."""
    g = torch.Generator().manual_seed(1)
    x = bf16_randn(g, (1, 16, 3072), 3.0)
    one = torch.ones((1, 1, 3072), dtype=torch.bfloat16)
    out = O.adaln(bits(x), bits(one))
    xv = x.double().numpy()
    mu = xv.mean(-1, keepdims=True)
    ref = (xv - mu) / np.sqrt(xv.var(-1, keepdims=True) + 1e-6)
    ok, worst, _ = bf16_close(out, bits(torch.from_numpy(ref).to(torch.bfloat16)))
    assert ok, worst


def test_adaln_config1_chain_vs_torch_eager():
    """out = res + gate * ((1 + scale) * LN(x) + shift), each op a bf16 eager op."""
    g = torch.Generator().manual_seed(717)
    x = bf16_randn(g, (1, 64, 3072))
    res = bf16_randn(g, (1, 64, 3072))
    shift, scale, gate = (bf16_randn(g, (1, 1, 3072), 0.1) for _ in range(3))
    ref = res + gate * ((1 + scale) * F.layer_norm(x, (3072,), eps=1e-6) + shift)
    out = O.adaln(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True)
    ok, worst, _ = bf16_close(out, bits(ref))
    assert ok, worst


def test_adaln_quantize_equals_quantize_of_adaln():
    g = torch.Generator().manual_seed(0)
    x = bf16_randn(g, (2, 77, 512))
    x[..., ::128] *= 25
    s = bf16_randn(g, (2, 1, 512))
    q, sc = O.adaln_quantize(bits(x), bits(s))
    q2, sc2 = O.mx_quantize(O.adaln(bits(x), bits(s)).reshape(-1, 512))
    assert np.array_equal(q, q2) and np.array_equal(sc, sc2)


# ------------------------------------------------- residual, SwiGLU --

def test_residual_bit_exact_vs_torch():
    g = torch.Generator().manual_seed(91)
    h = bf16_randn(g, (2, 57, 256))
    x = bf16_randn(g, (2, 57, 256))
    gate = bf16_randn(g, (2, 1, 256)).tanh()
    assert np.array_equal(O.residual(bits(h), bits(x), bits(gate)), bits(h + gate * x))


def test_swiglu_vs_torch_cpu():
    g = torch.Generator().manual_seed(91)
    a = bf16_randn(g, (64, 1024), 3.0)
    b = bf16_randn(g, (64, 1024))
    ref = bits(F.silu(a) * b)
    out = O.swiglu(bits(a), bits(b))
    ok, worst, nmis = bf16_close(out, ref)
    assert ok, worst
    assert nmis <= out.size // 1000  # exp implementations differ only near midpoints


def test_swiglu_quantize_equals_quantize_of_swiglu():
    g = torch.Generator().manual_seed(4)
    a = bf16_randn(g, (130, 256), 2.0)
    b = bf16_randn(g, (130, 256))
    q, s = O.swiglu_quantize(bits(a), bits(b))
    q2, s2 = O.mx_quantize(O.swiglu(bits(a), bits(b)))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


# --------------------------------------------------- RMSNorm, RoPE --

def _torch_rmsnorm(x, w, eps):
    # Diffusers RMSNorm with a bf16 weight (normalization.py:553-565), in torch ops.
    var = x.to(torch.float32).pow(2).mean(-1, keepdim=True)
    return (x * torch.rsqrt(var + eps)).to(torch.bfloat16) * w


@pytest.mark.parametrize("mag", [0.001, 1.0, 20.0])
def test_rms_norm_vs_torch_cpu(mag):
    g = torch.Generator().manual_seed(721)
    x = bf16_randn(g, (3, 40, 24, 128), mag)
    w = (torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    ok, worst = bf16_close_chain(O.rms_norm(bits(x), bits(w)), bits(_torch_rmsnorm(x, w, 1e-6)))
    assert ok, worst


def _torch_rope(x, freqs):
    # apply_rotary_emb_qwen(use_real=False) (WHL!transformer_qwenimage21.py:128-133).
    xr = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
    return torch.view_as_real(xr * freqs.unsqueeze(1)).flatten(3).type_as(x)


def test_rope_vs_torch_complex_multiply():
    g = torch.Generator().manual_seed(91)
    q = bf16_randn(g, (2, 49, 4, 128))
    k = bf16_randn(g, (2, 49, 4, 128))
    phase = torch.randn(49, 64, generator=g)
    freqs = torch.polar(torch.ones_like(phase), phase)
    f = torch.view_as_real(freqs).numpy()
    oq, ok_ = O.rope(bits(q), bits(k), f)
    for out, x in ((oq, q), (ok_, k)):
        ok, worst, _ = bf16_close(out, bits(_torch_rope(x, freqs)))
        assert ok, worst


def test_rope_identity_at_zero_angle():
    g = torch.Generator().manual_seed(3)
    q = bf16_randn(g, (1, 5, 2, 64))
    f = np.zeros((5, 32, 2), dtype=np.float32)
    f[..., 0] = 1.0
    oq, okk = O.rope(bits(q), bits(q), f)
    assert np.array_equal(oq, bits(q)) and np.array_equal(okk, bits(q))


def test_norm_rope_pack_equals_separate_ops_with_prefix():
    g = torch.Generator().manual_seed(721)
    B, S, P, H, D = 2, 17, 5, 3, 128
    q, k, v = (bits(bf16_randn(g, (B, S, H, D))) for _ in range(3))
    ck, cv = (bits(bf16_randn(g, (B, P, H, D))) for _ in range(2))
    wq, wk = (bits((torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)) for _ in range(2))
    phase = torch.randn(S, D // 2, generator=g)
    f = torch.view_as_real(torch.polar(torch.ones_like(phase), phase)).numpy()
    oq, ok, ov = O.norm_rope_pack(q, k, v, wq, wk, f, ck, cv)
    rq, rk = O.rope(O.rms_norm(q, wq), O.rms_norm(k, wk), f)
    assert np.array_equal(oq, rq)
    assert np.array_equal(ok, np.concatenate([ck, rk], 1))
    assert np.array_equal(ov, np.concatenate([cv, v], 1))


def test_rope_freqs_closed_form_and_torch():
    pos = O.rope_positions(4, 1, 6, 6)
    assert pos.shape == (40, 3)
    assert tuple(pos[4]) == (4, -3, -3) and tuple(pos[-1]) == (4, 2, 2)
    f = O.rope_freqs(pos)
    assert f.shape == (40, 64, 2)
    assert np.allclose(np.hypot(f[..., 0], f[..., 1]), 1.0, atol=2e-7)
    assert np.array_equal(f[0], np.stack([np.ones(64), np.zeros(64)], -1).astype(np.float32))
    # the diffusers formula restated in torch CPU ops (transformer_qwenimage21.py:666-675)
    cols = []
    for a, dim in enumerate((16, 56, 56)):
        inv = 1.0 / torch.pow(10000, torch.arange(0, dim, 2).to(torch.float32).div(dim))
        ang = torch.outer(torch.from_numpy(pos[:, a]).float(), inv)
        cols.append(torch.polar(torch.ones_like(ang), ang))
    ref = torch.view_as_real(torch.cat(cols, -1)).numpy()
    assert np.max(np.abs(f - ref)) < 2e-6
    # negative positions give the conjugate of the positive ones
    fneg = O.rope_freqs(np.array([[3, -3, -5]], dtype=np.int64))
    fpos = O.rope_freqs(np.array([[3, 3, 5]], dtype=np.int64))
    assert np.allclose(fneg[0, 8:, 0], fpos[0, 8:, 0]) and np.allclose(fneg[0, 8:, 1], -fpos[0, 8:, 1])


# ----------------------------------------------------------------- GEMM --

def test_mx_gemm_vs_float64_matmul():
    g = torch.Generator().manual_seed(1)
    a = bf16_randn(g, (100, 384))
    w = bf16_randn(g, (256, 384), 0.02)
    aq, as_ = O.mx_quantize(bits(a))
    wq, ws = O.mx_quantize(bits(w))
    y = O.mx_gemm(aq, as_, wq, ws)
    ref = O.mx_dequantize(aq, as_).astype(np.float64) @ O.mx_dequantize(wq, ws).astype(np.float64).T
    assert y.shape == (128, 256)
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-9)
    assert not y[100:].any()
    rows = np.array([3, 99, 0], dtype=np.int64)
    assert np.array_equal(O.mx_gemm(aq, as_, wq, ws, rows=rows), y[rows])
    # and close to the unquantized product (MXFP8 error, not an indexing bug)
    assert rel_fro(y[:100], a.double().numpy() @ w.double().numpy().T) < 0.05


def test_mx_gemm_tiny_exact():
    """K = 32, powers of two: the product is exactly representable."""
    a = np.zeros((128, 128), dtype=np.uint16)
    a[0, :] = bits(torch.full((128,), 2.0, dtype=torch.bfloat16))
    w = np.zeros((256, 128), dtype=np.uint16)
    w[5, :] = bits(torch.full((128,), -0.5, dtype=torch.bfloat16))
    aq, as_ = O.mx_quantize(a)
    wq, ws = O.mx_quantize(w)
    y = O.mx_gemm(aq, as_, wq, ws)
    assert y[0, 5] == -128.0 and np.count_nonzero(y) == 1


def test_bf16_round_helper_vs_torch():
    rng = np.random.default_rng(9)
    v = np.concatenate([rng.standard_normal(10000).astype(np.float32),
                        rng.integers(0, 2 ** 32, 10000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    v = v[np.isfinite(v)]
    ref = bits(torch.from_numpy(v).to(torch.bfloat16))
    assert np.array_equal(O.f32_to_bf16(v), ref)


def test_golden_bits_roundtrip():
    x = torch.tensor([1.0, -2.5, 3e-39], dtype=torch.bfloat16)
    assert torch.equal(from_bits(bits(x)), x)


def test_block_rows_subset_equals_full_block():
    """oracle/block.py with rows= computes exactly those rows of the full
    block (every step is row-local: the per-batch modulation, the RoPE row of
    the token's position, the GEMM rows), across two batches."""
    from oracle import block as OB
    rng = np.random.default_rng(5)
    B, S, D, H, F = 2, 150, 256, 2, 512
    bf = lambda *shape, s=1.0: O.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * s)  # noqa: E731
    w = {"qkv": bf(3 * D, D, s=0.05), "out": bf(D, D, s=0.05), "gate": bf(F, D, s=0.05), "up": bf(F, D, s=0.05),
         "down": bf(D, F, s=0.05), "norm_q": O.f32_to_bf16(rng.uniform(0.8, 1.2, 128).astype(np.float32)),
         "norm_k": O.f32_to_bf16(rng.uniform(0.8, 1.2, 128).astype(np.float32))}
    h, mod = bf(B, S, D), bf(B, 6, D, s=0.3)
    f = O.rope_freqs(O.rope_positions(6, 1, 12, 12))
    full, st = OB.block_forward(h, mod, f, w, heads=H, return_stages=True)
    rows = np.array([0, 7, 149, 150, 151, 299])
    part = OB.block_forward(h, mod, f, w, heads=H, rows=rows)
    assert np.array_equal(part, full.reshape(B * S, D)[rows])
    assert np.isfinite(bf16_values(full)).all() and not np.array_equal(full, h)
