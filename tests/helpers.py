"""Conversions and comparison helpers shared by the tests (no GPU needed)."""
import numpy as np
import torch


def bits(t):
    """bf16 torch tensor -> numpy uint16 bit patterns."""
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def from_bits(b, device="cpu"):
    """numpy uint16 bit patterns -> bf16 torch tensor."""
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_values(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def ulp_bf16(v):
    """Spacing of bf16 values at |v| (the ulp of the reference value)."""
    a = np.abs(np.asarray(v, dtype=np.float32)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -133)))
    return np.maximum(2.0 ** (e - 7), 2.0 ** -133)


def bf16_close(got_bits, ref_bits, ulps=1, rel=4e-3):
    """Elementwise: |got - ref| <= ulps * ulp(ref) or <= rel * |ref|.
    Returns (ok, worst_ulps, n_mismatch)."""
    g = bf16_values(got_bits).astype(np.float64)
    r = bf16_values(ref_bits).astype(np.float64)
    d = np.abs(g - r)
    u = ulp_bf16(r)
    ok = (d <= ulps * u) | (d <= rel * np.abs(r))
    worst = float(np.max(d / u)) if d.size else 0.0
    return bool(ok.all()), worst, int((g != r).sum())


def bf16_close_chain(got_bits, ref_bits, frac=1e-3):
    """For chains with two bf16 rounding points (bf16(bf16(a) * w)): a last-bit
    difference in a reduction can flip the intermediate by 1 ulp, which the
    second rounding turns into up to 2 ulps.  Accept 1 ulp everywhere except a
    fraction `frac` of elements, which may be 2 ulps.  Returns (ok, worst)."""
    g = bf16_values(got_bits).astype(np.float64)
    r = bf16_values(ref_bits).astype(np.float64)
    u = ulp_bf16(r)
    d = np.abs(g - r) / u
    worst = float(d.max()) if d.size else 0.0
    return bool(worst <= 2 and (d > 1).sum() <= max(1, frac * d.size)), worst


def rel_fro(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def swizzle_permute(exponents):
    """The reference test's restatement of the 128x4 scale layout
    (tests/gpu/check_mxfp8.py:32-34) as a numpy reshape/transpose:
    (M, K/32) exponents -> flat swizzled array."""
    m, kb = exponents.shape
    return exponents.reshape(m // 128, 4, 32, kb // 4, 4).transpose(0, 3, 2, 1, 4).reshape(-1)


def bf16_randn(gen, shape, scale=1.0):
    """Seeded N(0, scale^2) bf16 tensor on the CPU."""
    return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)


def unswizzle_scales(flat, m, k):
    """Flat swizzled E8M0 bytes of an (m, k) quantization -> (m, k/32)
    exponents (the inverse of swizzle_permute; m % 128 == 0)."""
    return np.asarray(flat, dtype=np.uint8).reshape(m // 128, k // 128, 32, 4, 4).transpose(0, 3, 2, 1, 4).reshape(
        m, k // 32)


def quantized_rows(q, rows):
    """Codes (n, K) and exponents (n, K/32) of the given rows of a Quantized
    (row-major or tiled) on any device, as numpy uint8."""
    from qwen_image_accel.kernels import mxfp8
    codes = mxfp8.as_row_major(q).values.view(torch.uint8)
    mp, k = codes.shape
    idx = torch.as_tensor(np.asarray(rows), device=codes.device)
    exps = unswizzle_scales(q.scales.view(torch.uint8).cpu().numpy(), mp, k)
    return codes[idx].cpu().numpy(), exps[np.asarray(rows)]


def pack_quantized(codes, exps):
    """Rows of codes (n, K) and exponents (n, K/32) -> an oracle-style
    quantization of n rows: codes padded to a multiple of 128 rows with zeros
    and the exponents swizzled."""
    n, k = codes.shape
    mp = (n + 127) // 128 * 128
    q = np.zeros((mp, k), dtype=np.uint8)
    e = np.zeros((mp, k // 32), dtype=np.uint8)
    q[:n], e[:n] = codes, exps
    return q, swizzle_permute(e)
