"""Parity of the HIP kernels against the CPU oracle on identical seeded inputs.

Bars: MXFP8 codes and E8M0 scales bit-exact; bf16
ops within 1 bf16 ulp (or rel 4e-3) -- here tighter: LayerNorm, RMSNorm, RoPE,
the residual and SwiGLU are bit-exact (float64 row statistics rounded once,
as the oracle's; a SiLU equal to the oracle's on every bf16 input); GEMM
within rel-Frobenius 1e-2 of dequantize-then-matmul.
Every test prints its case before the GPU step so a failing run names it.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import block as OB
from oracle import oracle as O
from qwen_image_accel import _native
from qwen_image_accel.kernels import attention, bf16, elementwise, epilogue, gemm, layernorm, mxfp8
from tests.helpers import bf16_randn, bf16_values, bits, rel_fro

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def assert_bits_equal(got, ref):
    """Bit-exact comparison of bf16 bit patterns; on failure report how many
    elements differ and by how many ulps at most."""
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    bad = got != ref
    if bad.any():
        ulps = np.abs(got.astype(np.int32) - ref.astype(np.int32))[bad]
        raise AssertionError(f"{int(bad.sum())} of {bad.size} differ (max {int(ulps.max())} code steps)")


# ------------------------------------------------------------ conversions --

def test_e4m3_hardware_conversion_exhaustive(dev):
    """v_cvt_pk_fp8_f32 == oracle RNE on every finite bf16 value |v| < 448 and
    on random fp32 values inside the range (the only inputs the quantizers
    ever convert: block-scaled bf16 values)."""
    v = bf16_values(np.arange(65536, dtype=np.uint16))
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    rng = np.random.default_rng(0)
    v = np.concatenate([v, rng.uniform(-448, 448, 200000).astype(np.float32)])
    say("e4m3 exhaustive", v.size)
    x = torch.from_numpy(v).to(dev)
    out = torch.empty(v.size, dtype=torch.uint8, device=dev)
    _native.call("qim_debug_e4m3_encode", _native.ptr(x), _native.ptr(out), v.size, _native.stream())
    got = out.cpu().numpy()
    ref = O.e4m3_encode(v)
    bad = np.where(got != ref)[0]
    assert bad.size == 0, [(float(v[i]), int(got[i]), int(ref[i])) for i in bad[:10]]


@pytest.mark.parametrize("e", [0, 1, 100, 119, 127, 134, 200, 254])
def test_e4m3_scaled_conversion_exhaustive(dev, e):
    """The packed scaled conversion every quantizer uses
    (v_cvt_scalef32_pk_fp8_bf16 with the E8M0 exponent e in the scale
    operand) == oracle RNE of x * 2^(127 - e), on every bf16 x for which that
    is at most 448 in magnitude -- the only values the quantizers convert
    (their exponent rule guarantees it).  e = 0 is the scale operand 0.0."""
    raw = np.arange(65536, dtype=np.uint16)
    with np.errstate(invalid="ignore", over="ignore"):
        y = bf16_values(raw).astype(np.float64) * 2.0 ** (127 - e)
        ok = np.isfinite(y) & (np.abs(y) <= 448)
    say("e4m3 scaled exhaustive", e, int(ok.sum()))
    x = torch.from_numpy(raw.view(np.int16)).to(dev)
    out = torch.empty(65536, dtype=torch.uint8, device=dev)
    _native.call("qim_debug_e4m3_encode_scaled", _native.ptr(x), e, _native.ptr(out), 65536, _native.stream())
    got = out.cpu().numpy()
    ref = O.e4m3_encode(np.where(ok, y, 0.0).astype(np.float32))
    bad = np.where(ok & (got != ref))[0]
    assert bad.size == 0, [(hex(raw[i]), int(got[i]), int(ref[i])) for i in bad[:10]]


def test_bf16_hardware_rounding(dev):
    """v_cvt_pk_bf16_f32 == oracle RNE, subnormals included."""
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    sub = rng.integers(0, 1 << 23, 1 << 16, dtype=np.uint64).astype(np.uint32)
    v = np.concatenate([raw, sub, sub | 0x80000000]).view(np.float32)
    v = v[np.isfinite(v)]
    say("bf16 rounding", v.size)
    x = torch.from_numpy(v).to(dev)
    out = torch.empty(v.size, dtype=torch.int16, device=dev)
    _native.call("qim_debug_bf16_round", _native.ptr(x), _native.ptr(out), v.size, _native.stream())
    got = out.cpu().numpy().view(np.uint16)
    ref = O.f32_to_bf16(v)
    bad = np.where(got != ref)[0]
    assert bad.size == 0, [(float(v[i]), hex(got[i]), hex(ref[i])) for i in bad[:10]]


def test_scaled_mfma_lane_layout(dev):
    """One v_mfma_scale_f32_32x32x64_f8f6f4 against the oracle product."""
    rng = np.random.default_rng(2)
    table = O.e4m3_values()
    finite = np.where(np.isfinite(table))[0].astype(np.uint8)
    a = rng.choice(finite, (32, 64))
    b = rng.choice(finite, (32, 64))
    sa = rng.integers(120, 135, (32, 2)).astype(np.uint8)
    sb = rng.integers(120, 135, (32, 2)).astype(np.uint8)
    da = table[a] * np.exp2(np.repeat(sa.astype(np.float64), 32, 1) - 127)
    db = table[b] * np.exp2(np.repeat(sb.astype(np.float64), 32, 1) - 127)
    ref = da @ db.T
    # The scaled MFMA does not accumulate like sequential fp32: measured error is
    # about 2^-11 of sum|a_k b_k| (fixed-width alignment inside the dot-product
    # unit).  A layout mistake (wrong block scale) would be an O(1) error.
    bound = 2.0 ** -9 * (np.abs(da) @ np.abs(db).T)
    say("mfma tile")
    t = [torch.from_numpy(np.ascontiguousarray(z)).to(dev) for z in (a, b, sa, sb)]
    out = torch.zeros((32, 32), dtype=torch.float32, device=dev)
    _native.call("qim_debug_mfma_tile", *[_native.ptr(z) for z in t], _native.ptr(out), _native.stream())
    got = out.cpu().numpy()
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)
    assert rel_fro(got, ref) < 1e-3


def test_modulation_values_exhaustive(dev):
    """qim_modulation_values on every bf16 value: tanh rows equal the oracle's
    tanh (float64 tanh, rounded to fp32, then to bf16), 1 + x rows equal torch's
    bf16 addition on the CPU (fp32 sum rounded to nearest even), copied rows
    are unchanged."""
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(64, 1024)
    mod = torch.stack([allb, allb, allb], dim=1).contiguous()  # (64, 3, 1024)
    kinds = (elementwise.MOD_COPY, elementwise.MOD_ONE_PLUS, elementwise.MOD_TANH)
    out = elementwise.modulation_values(mod.to(dev), kinds).cpu()
    assert out.shape == (3, 64, 1024)
    got = {k: bits(out[i]).astype(np.int64) for i, k in enumerate(("copy", "one", "tanh"))}
    with np.errstate(invalid="ignore"):  # NaN inputs
        want = {"copy": bits(allb).astype(np.int64), "one": bits(1 + allb).astype(np.int64),
                "tanh": OB.tanh_bf16(bits(allb)).astype(np.int64)}
    for k in got:
        g, w = got[k], want[k]
        nan_g = (g & 0x7f80 == 0x7f80) & (g & 0x7f != 0)
        nan_w = (w & 0x7f80 == 0x7f80) & (w & 0x7f != 0)
        assert np.array_equal(nan_g, nan_w), k
        assert np.array_equal(g[~nan_g], w[~nan_w]), (k, int((g[~nan_g] != w[~nan_w]).sum()))
    # The cached-decode path (optimizations/decode.py) keeps torch's bf16
    # tanh, as the reference's precompute does (optimizations/fusion.py:48-53).
    # Count where torch's on-device tanh differs from the kernel's (printed
    # for the record; the CPU tanh equals the kernel's definition on every
    # input, tests/test_parity_bar.py).  At most a few last-bit differences.
    dev_tanh = bits(allb.to(dev).tanh().cpu().reshape(64, 1024)).astype(np.int64)
    live = ~((got["tanh"] & 0x7f80 == 0x7f80) & (got["tanh"] & 0x7f != 0))
    diff = got["tanh"][live] != dev_tanh[live]
    print(f"tanh: kernel vs torch on-device bf16 tanh differ on {int(diff.sum())} of {int(live.sum())} inputs, "
          f"max {int(np.abs(got['tanh'][live] - dev_tanh[live]).max())} ulp")
    assert np.abs(got["tanh"][live] - dev_tanh[live]).max() <= 1


def test_silu_exhaustive(dev):
    """The fast SiLU (estimate + rounding-band check + exact fallback) equals
    the oracle's bf16(g / (1 + expf(-g))) on every one of the 65536 bf16
    inputs, so every SwiGLU kernel's silu is pinned for all inputs."""
    raw = np.arange(65536, dtype=np.uint16)
    g = bf16_values(raw)
    say("silu exhaustive")
    x = torch.from_numpy(raw.view(np.int16)).to(dev)
    out = torch.empty(65536, dtype=torch.int16, device=dev)
    _native.call("qim_debug_silu", _native.ptr(x), _native.ptr(out), 65536, _native.stream())
    got = out.cpu().numpy().view(np.uint16)
    # swiglu(g, 1) = bf16(bf16(silu(g)) * 1) = bf16(silu(g)).
    ref = O.swiglu(raw.reshape(1, -1), O.f32_to_bf16(np.ones((1, 65536), np.float32))).reshape(-1)
    nan = np.isnan(g)
    assert np.array_equal(np.isnan(bf16_values(got))[~nan], np.isnan(bf16_values(ref))[~nan])
    bad = np.where((got != ref) & ~nan)[0]
    assert bad.size == 0, [(hex(raw[i]), hex(got[i]), hex(ref[i])) for i in bad[:10]]
    assert np.all(np.isnan(bf16_values(got)[nan]))


def test_rstd_exhaustive(dev):
    """The normalisations' reciprocal square root (v_rsq_f32 refined in
    float64, an interval check, the float64 expression as fallback) equals its
    definition fp32(1 / sqrt(double(var + eps))) for every one of the 2^32 fp32
    bit patterns of var (eps 0, so t = var + 0 runs over every fp32 value; and
    eps 1e-6, the configs' value), so RMSNorm's and AdaLN's rstd is pinned for
    all inputs.  The comparison runs on the device and counts disagreements."""
    for eps in (0.0, 1e-6):
        say("rstd exhaustive, eps", eps)
        bad = torch.tensor([0, -1], dtype=torch.int32, device=dev)
        for first in (0, 1 << 31):
            _native.call("qim_debug_rstd_sweep", first, 1 << 31, eps, _native.ptr(bad), _native.stream())
        n, low = (int(x) & 0xffffffff for x in bad.cpu().tolist())
        assert n == 0, (eps, n, hex(low))


def test_streaming_copy(dev):
    """The bandwidth/counter calibration copy and its ceiling variants move
    every byte, tails included, and nothing past the end."""
    n = (3 << 20) + 48
    say("copy", n)
    src = torch.randint(0, 256, (n,), dtype=torch.uint8).to(dev)
    dst = torch.zeros(n + 16, dtype=torch.uint8, device=dev)
    _native.call("qim_debug_copy", _native.ptr(src), _native.ptr(dst), n, _native.stream())
    got = dst.cpu()
    assert torch.equal(got[:n], src.cpu()) and int(got[n:].sum()) == 0
    for vpl in (1, 2, 4, 8):
        for bpc in (0, 1, 4):
            say("copy_ex", vpl, bpc)
            dst.zero_()
            _native.call("qim_debug_copy_ex", _native.ptr(src), _native.ptr(dst), n, vpl, bpc, _native.stream())
            got = dst.cpu()
            assert torch.equal(got[:n], src.cpu()) and int(got[n:].sum()) == 0, (vpl, bpc)


# ---------------------------------------------------------------- quantize --

@pytest.mark.parametrize("m,k", [(128, 4096), (1024, 4096), (1536, 4096), (2400, 4096), (4096, 12288),
                                 (16384, 4096), (77, 4096), (1, 4096), (4352, 3072)])
def test_quantize_bit_exact(dev, m, k):
    """Shapes and outliers of the reference check (tests/gpu/check_mxfp8.py:38-50)."""
    g = torch.Generator().manual_seed(0)
    x = bf16_randn(g, (m, k))
    x[:, ::512] *= 40
    if m > 200:
        x[m // 3] *= 1e-3
    say("quantize", m, k)
    a = mxfp8.quantize(x.to(dev))
    q, s = O.mx_quantize(bits(x))
    assert a.rows == m and a.values.shape == (mxfp8.padded_rows(m), k)
    assert a.scales.dtype == torch.float8_e8m0fnu
    assert np.array_equal(u8(a.values), q)
    assert np.array_equal(u8(a.scales), s)


def test_quantize_config4_outliers_and_strided_rows(dev):
    """Config 4a input (1% outliers x20) read through a row stride."""
    g = torch.Generator().manual_seed(0)
    big = bf16_randn(g, (4352, 3072 + 64))
    mask = torch.rand(big.shape, generator=g) < 0.01
    big[mask] *= 20
    x = big[:, 32:32 + 3072]
    say("quantize strided", x.shape, x.stride())
    a = mxfp8.quantize(x.to(dev))
    q, s = O.mx_quantize(bits(x.contiguous()))
    assert np.array_equal(u8(a.values), q) and np.array_equal(u8(a.scales), s)


# ----------------------------------------------------------- LayerNorm --

class _LN:
    def __init__(self, d, eps=1e-6):
        self.normalized_shape = (d,)
        self.eps = eps
        self.elementwise_affine = False

    def __call__(self, x):
        return F.layer_norm(x, self.normalized_shape, eps=self.eps)


@pytest.mark.parametrize("b,n,d", [(1, 49, 4096), (2, 257, 4096), (1, 1024, 4096), (1, 4096, 4096),
                                   (1, 16384, 4096), (1, 1280, 3072), (2, 33, 3072)])
@pytest.mark.parametrize("mag", [0.001, 1.0, 20.0])
def test_layer_norm_scale(dev, b, n, d, mag):
    """Shapes and magnitudes of the reference check (check_layernorm_ops.py:16-23)."""
    g = torch.Generator().manual_seed(717)
    x = bf16_randn(g, (b, n, d), mag)
    s = bf16_randn(g, (b, 1, d))
    say("layer_norm_scale", b, n, d, mag)
    before = _native.calls.get("qim_adaln", 0)
    out = layernorm.layer_norm_scale(x.to(dev), s.to(dev), _LN(d))
    assert _native.calls.get("qim_adaln", 0) == before + 1
    # float64 row statistics rounded once, as the oracle's: bit-exact.
    assert_bits_equal(bits(out), O.adaln(bits(x), bits(s)))


def test_adaln_config1_full_chain(dev):
    """Config 1: out = res + gate * ((1 + scale) * LN(x) + shift) at 512^2."""
    g = torch.Generator().manual_seed(717)
    x = bf16_randn(g, (1, 1280, 3072))
    shift, scale, gate = (bf16_randn(g, (1, 1, 3072), 0.1) for _ in range(3))
    res = bf16_randn(g, (1, 1280, 3072))
    say("adaln config1")
    out = layernorm.layer_norm_scale(x.to(dev), scale.to(dev), _LN(3072), shift=shift.to(dev),
                                     gate=gate.to(dev), residual=res.to(dev), add_one=True)
    ref = O.adaln(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True)
    assert_bits_equal(bits(out), ref)


@pytest.mark.parametrize("d", [136, 1000, 3072, 16384])
@pytest.mark.parametrize("parts", ["shift", "gate+res", "shift+res", "all-no-add-one"])
def test_adaln_optional_operands_and_widths(dev, d, parts):
    """Every subset of the optional operands (an absent one is a neutral value
    in the kernel, so signed zeros must survive) at widths that leave part of
    the last wave idle (136, 1000) and at the largest supported width."""
    g = torch.Generator().manual_seed(d)
    x = bf16_randn(g, (2, 37, d))
    x[0, 3] = 0.0                                      # a constant row: t0 = 0 (signed zeros)
    scale = bf16_randn(g, (2, 1, d), 0.1)
    scale[..., ::7] = -1.0                             # 1 + scale = 0 -> t2 = +-0
    scale[..., 1::7] = -3.0                            # 1 + scale < 0 -> t2 = -0 on the zero row
    shift = bf16_randn(g, (2, 1, d), 0.1) if "shift" in parts or "all" in parts else None
    gate = bf16_randn(g, (2, 1, d), 0.1) if "gate" in parts or "all" in parts else None
    res = bf16_randn(g, (2, 37, d)) if "res" in parts or "all" in parts else None
    add_one = "no-add-one" not in parts
    say("adaln parts", d, parts)
    dv = (lambda t: None if t is None else t.to(dev))
    out = layernorm.layer_norm_scale(x.to(dev), scale.to(dev), _LN(d), shift=dv(shift), gate=dv(gate),
                                     residual=dv(res), add_one=add_one)
    assert _native.calls.get("qim_adaln", 0) > 0
    nb = (lambda t: None if t is None else bits(t))
    ref = O.adaln(bits(x), bits(scale), nb(shift), nb(gate), nb(res), add_one=add_one)
    # Bit-exact, including the signed zeros of the row whose LayerNorm output is zero.
    assert_bits_equal(bits(out), ref)


@pytest.mark.parametrize("b,n,d", [(1, 1024, 4096), (1, 1536, 4096), (1, 2400, 4096), (1, 4096, 4096),
                                   (1, 16384, 4096), (2, 1024, 4096), (1, 77, 4096), (1, 4352, 3072),
                                   (1, 130, 3072)])
def test_layer_norm_scale_quantize(dev, b, n, d):
    """Fused == quantize(separate) byte-for-byte (check_mx_epilogue.py:28-38,
    the same shapes) and codes and scales bit-exact against the oracle."""
    g = torch.Generator().manual_seed(0)
    x = bf16_randn(g, (b, n, d))
    x[..., ::512] *= 25
    s = bf16_randn(g, (b, 1, d))
    say("layer_norm_scale_quantize", b, n, d)
    xd, sd = x.to(dev), s.to(dev)
    fused = epilogue.layer_norm_scale_quantize(xd, sd, _LN(d))
    sep = mxfp8.quantize(layernorm.layer_norm_scale(xd, sd, _LN(d)).reshape(-1, d))
    assert fused.rows == b * n and tuple(fused.shape) == (b, n, d)
    assert np.array_equal(u8(fused.values), u8(sep.values))
    assert np.array_equal(u8(fused.scales), u8(sep.scales))
    q, sc = O.adaln_quantize(bits(x), bits(s))
    assert np.array_equal(u8(fused.values), q)
    assert np.array_equal(u8(fused.scales), sc)


def _rows_with_offsets(g, rows, d):
    """Rows whose mean is large against their spread (mean/std up to ~1e3)
    and near-constant rows: the one-pass variance cannot settle the fp32
    rounding for most of them, so the kernels' second pass runs, beside rows
    where it settles it."""
    x = bf16_randn(g, (1, rows, d))
    offset = torch.tensor([0.0, 1.0, 8.0, 30.0, 100.0, 1e3])[torch.arange(rows) % 6]
    x = (x.float() + offset[None, :, None]).to(torch.bfloat16)
    x[0, 5::17] = 3.0
    x[0, 5::17, ::301] = 3.5
    return x


@pytest.mark.parametrize("d", [3072, 4096])
def test_adaln_second_pass_rows(dev, d):
    """The config-1 chain and the quantizing AdaLN on rows that take the
    second statistics pass: bit-exact against the oracle's two-pass float64
    statistics."""
    g = torch.Generator().manual_seed(d + 5)
    x = _rows_with_offsets(g, 300, d)
    shift, scale, gate = (bf16_randn(g, (1, 1, d), 0.1) for _ in range(3))
    res = bf16_randn(g, (1, 300, d))
    say("adaln second pass", d)
    out = layernorm.layer_norm_scale(x.to(dev), scale.to(dev), _LN(d), shift=shift.to(dev),
                                     gate=gate.to(dev), residual=res.to(dev), add_one=True)
    assert_bits_equal(bits(out), O.adaln(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True))
    fused = epilogue.layer_norm_scale_quantize(x.to(dev), scale.to(dev), _LN(d))
    q, sc = O.adaln_quantize(bits(x), bits(scale))
    assert np.array_equal(u8(fused.values), q)
    assert np.array_equal(u8(fused.scales), sc)


def test_adaln_wide_rows(dev):
    """Rows whose values span 2^-60 .. 2^60, so the float64 row sum S1 is no
    longer exact (the one-pass variance bound then includes S1's rounding),
    beside rows with a few 2^60 outliers among N(0, 1) values and rows of
    2^50 offsets over 2^-60 noise: bit-exact against the oracle (whose mean
    agrees with the kernel's after the fp32 rounding of the statistics)."""
    g = torch.Generator().manual_seed(60)
    d = 3072
    x = torch.randn(1, 96, d, generator=g)
    x[0, 0::3] *= torch.exp2(torch.randint(-60, 61, (32, d), generator=g).float())
    x[0, 1::3, ::700] = torch.randn(32, 5, generator=g) * 2.0 ** 60
    x[0, 2::3] = x[0, 2::3] * 2.0 ** -60 + 2.0 ** 50
    x = x.to(torch.bfloat16)
    scale, shift, gate = (bf16_randn(g, (1, 1, d), 0.1) for _ in range(3))
    res = bf16_randn(g, (1, 96, d))
    say("adaln wide rows")
    out = layernorm.layer_norm_scale(x.to(dev), scale.to(dev), _LN(d), shift=shift.to(dev),
                                     gate=gate.to(dev), residual=res.to(dev), add_one=True)
    assert_bits_equal(bits(out), O.adaln(bits(x), bits(scale), bits(shift), bits(gate), bits(res), add_one=True))
    fused = epilogue.layer_norm_scale_quantize(x.to(dev), scale.to(dev), _LN(d))
    q, sc = O.adaln_quantize(bits(x), bits(scale))
    assert np.array_equal(u8(fused.values), q)
    assert np.array_equal(u8(fused.scales), sc)


# --------------------------------------------------- residual, SwiGLU --

@pytest.mark.parametrize("b,s,d", [(1, 49, 4096), (2, 257, 4096), (1, 4352, 3072)])
def test_residual_bit_exact(dev, b, s, d):
    g = torch.Generator().manual_seed(91)
    h = bf16_randn(g, (b, s, d))
    x = bf16_randn(g, (b, s, d))
    gate = bf16_randn(g, (b, 1, d)).tanh()
    say("residual", b, s, d)
    out = elementwise.residual(h.to(dev), x.to(dev), gate.to(dev))
    assert np.array_equal(bits(out), O.residual(bits(h), bits(x), bits(gate)))


@pytest.mark.parametrize("m,f", [(1024, 12288), (128, 12288), (77, 256)])
def test_swiglu(dev, m, f):
    g = torch.Generator().manual_seed(91)
    a = bf16_randn(g, (m, f), 2.0)
    v = bf16_randn(g, (m, f))
    say("swiglu", m, f)
    out = bf16.swiglu(a.to(dev), v.to(dev))
    assert_bits_equal(bits(out), O.swiglu(bits(a), bits(v)))


def test_swiglu_strided_halves_config3(dev):
    """Config 3: gate/up are the two halves of one (M, 2F) tensor."""
    g = torch.Generator().manual_seed(91)
    X = bf16_randn(g, (4352, 2 * 12288))
    say("swiglu strided config3")
    Xd = X.to(dev)
    out = bf16.swiglu(Xd[:, :12288], Xd[:, 12288:])
    assert _native.calls.get("qim_swiglu", 0) > 0
    assert_bits_equal(bits(out), O.swiglu(bits(X[:, :12288]), bits(X[:, 12288:])))


@pytest.mark.parametrize("rows,width", [(1024, 12288), (2400, 12288), (16384, 12288), (128, 12288), (77, 256),
                                        (130, 384)])
def test_swiglu_quantize(dev, rows, width):
    """Fused == quantize(swiglu) byte for byte (check_mx_epilogue.py:40-46,
    the same shapes), and codes and scales bit-exact against the oracle.
    (130, 384): three 128-column chunks, so a workgroup's four waves span
    two row groups, and padding rows 130..255."""
    g = torch.Generator().manual_seed(0)
    a = bf16_randn(g, (rows, width))
    v = bf16_randn(g, (rows, width))
    say("swiglu_quantize", rows, width)
    ad, vd = a.to(dev), v.to(dev)
    fused = epilogue.swiglu_quantize(ad, vd)
    sep = mxfp8.quantize(bf16.swiglu(ad, vd))
    assert np.array_equal(u8(fused.values), u8(sep.values))
    assert np.array_equal(u8(fused.scales), u8(sep.scales))
    q, s = O.swiglu_quantize(bits(a), bits(v))
    assert np.array_equal(u8(fused.values), q)
    assert np.array_equal(u8(fused.scales), s)


def test_swiglu_quantize_over_grid_y_limit(dev):
    """262,344 rows: 65,600 row groups of four rows, above the 65,535 of one
    launch's grid y, so the launcher splits the rows over two launches; fused
    == quantize(swiglu) byte for byte, row-major and tiled."""
    g = torch.Generator(device=dev).manual_seed(3)
    rows = 262144 + 200
    a = torch.randn(rows, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(rows, 128, generator=g, device=dev).to(torch.bfloat16)
    say("swiglu_quantize grid fold", rows, 128)
    for tiled in (False, True):
        fused = epilogue.swiglu_quantize(a, v, tiled=tiled)
        sep = mxfp8.quantize(bf16.swiglu(a, v), tiled=tiled)
        assert torch.equal(fused.values.view(torch.uint8), sep.values.view(torch.uint8))
        assert torch.equal(fused.scales.view(torch.uint8), sep.scales.view(torch.uint8))


# ------------------------------------------------------ RMSNorm, RoPE --

@pytest.mark.parametrize("mag", [0.001, 1.0, 20.0])
def test_rms_norm(dev, mag):
    g = torch.Generator().manual_seed(721)
    x = bf16_randn(g, (1, 512, 24, 128), mag)
    w = (torch.rand(128, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    say("rms_norm", mag)
    out = bf16.rms_norm(x.to(dev), w.to(dev), 1e-6)
    # The float64 sums of squares agree with the oracle's to 2^-53 of the sum (exactly where a row's
    # squares lie within 2^30), so the fp32 statistics match: bit-exact vs the oracle.
    assert_bits_equal(bits(out), O.rms_norm(bits(x), bits(w)))


@pytest.mark.parametrize("b,s,h", [(1, 49, 32), (2, 257, 32), (1, 4096, 24)])
def test_rope_qk_bit_exact(dev, b, s, h):
    """Reference check shapes (check_fused.py:13-24), seed 91."""
    g = torch.Generator().manual_seed(91)
    q = bf16_randn(g, (b, s, h, 128))
    k = bf16_randn(g, (b, s, h, 128))
    phase = torch.randn(s, 64, generator=g)
    freqs = torch.polar(torch.ones_like(phase), phase)
    say("rope_qk", b, s, h)
    oq, ok = elementwise.rope_qk(q.to(dev), k.to(dev), freqs.to(dev))
    rq, rk = O.rope(bits(q), bits(k), torch.view_as_real(freqs).numpy())
    assert np.array_equal(bits(oq), rq) and np.array_equal(bits(ok), rk)


class _RMS:
    def __init__(self, w, eps=1e-6):
        self.weight, self.bias, self.eps = w, None, eps


@pytest.mark.parametrize("b,s,p,h", [(1, 49, 0, 32), (2, 257, 7, 32), (1, 1024, 99, 32), (1, 4096, 113, 32),
                                     (1, 16384, 113, 32), (2, 49, 1024, 32), (1, 300, 13, 24)])
@pytest.mark.parametrize("mag", [0.001, 1.0, 20.0])
def test_prepare_attention_inputs(dev, b, s, p, h, mag):
    """Reference check shapes (check_attention_ops.py:19-31), seed 721."""
    g = torch.Generator().manual_seed(721)
    q = bf16_randn(g, (b, s, h, 128), mag)
    k = bf16_randn(g, (b, s, h, 128), mag)
    v = bf16_randn(g, (b, s, h, 128))
    ck = bf16_randn(g, (b, p, h, 128))
    cv = bf16_randn(g, (b, p, h, 128))
    wq, wk = bf16_randn(g, (128,)), bf16_randn(g, (128,))
    phase = torch.randn(s, 64, generator=g)
    freqs = torch.polar(torch.ones_like(phase), phase)
    say("prepare_attention_inputs", b, s, p, h, mag)
    d = lambda t: t.to(dev)
    oq, ok, ov = attention.prepare_attention_inputs(d(q), d(k), d(v), _RMS(d(wq)), _RMS(d(wk)), d(freqs),
                                                    d(ck), d(cv))
    f = torch.view_as_real(freqs).numpy()
    rq, rk, rv = O.norm_rope_pack(bits(q), bits(k), bits(v), bits(wq), bits(wk), f, bits(ck), bits(cv))
    assert np.array_equal(bits(ov), rv)
    assert np.array_equal(bits(ok)[:, :p], rk[:, :p])
    assert_bits_equal(bits(oq), rq)
    assert_bits_equal(bits(ok), rk)
    _check_norm_rope(dev, q, k, wq, wk, f, bits(oq), bits(ok)[:, p:])


def _check_norm_rope(dev, q, k, wq, wk, f, got_q, got_k):
    """Fused RMSNorm + RoPE == RoPE of the separate rms_norm kernel's output
    (the invariant fused == separate) and == the oracle's RMSNorm then RoPE,
    bit for bit (the float64 sums of squares agree to 2^-53 of the sum --
    exactly where a row's squares lie within 2^30 -- so the fused and the
    separate kernel and the oracle share the fp32 statistic)."""
    nq = bf16.rms_norm(q.to(dev), wq.to(dev), 1e-6)
    nk = bf16.rms_norm(k.to(dev), wk.to(dev), 1e-6)
    oq_, ok_ = O.rms_norm(bits(q), bits(wq)), O.rms_norm(bits(k), bits(wk))
    assert_bits_equal(bits(nq), oq_)
    assert_bits_equal(bits(nk), ok_)
    rq, rk = O.rope(bits(nq), bits(nk), f)
    assert_bits_equal(got_q, rq)
    assert_bits_equal(got_k, rk)


# Every launch split of k_norm_rope: head dim 64 / 128 / 256, and head counts
# that take two vectors per lane (D >= 128, H % (1024 / D) == 0), two or three
# rows per lane with whole waves, or the masked kernel; with and without V and
# a cached prefix (which needs V).
@pytest.mark.parametrize("d,h,with_v,p", [(128, 24, False, 0), (128, 8, True, 4), (128, 12, False, 0),
                                          (128, 20, True, 3), (128, 4, False, 0), (64, 16, False, 0),
                                          (64, 24, True, 0), (64, 32, False, 0), (64, 10, True, 2),
                                          (256, 8, False, 0), (256, 4, True, 1), (256, 6, True, 0),
                                          (256, 5, False, 0)])
def test_norm_rope_pack_every_split(dev, d, h, with_v, p):
    g = torch.Generator().manual_seed(97)
    b, s = 2, 37
    q = bf16_randn(g, (b, s, h, d))
    k = bf16_randn(g, (b, s, h, d))
    v = bf16_randn(g, (b, s, h, d)) if with_v else None
    ck = bf16_randn(g, (b, p, h, d)) if p else None
    cv = bf16_randn(g, (b, p, h, d)) if p else None
    wq = (torch.rand(d, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    wk = (torch.rand(d, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    phase = torch.randn(s, d // 2, generator=g)
    freqs = torch.view_as_real(torch.polar(torch.ones_like(phase), phase)).reshape(s, d).contiguous()
    say("norm_rope split", d, h, with_v, p)
    dq, dk, dw_q, dw_k, df = (t.to(dev) for t in (q, k, wq, wk, freqs))
    dv = v.to(dev) if with_v else None
    dck = ck.to(dev) if p else None
    dcv = cv.to(dev) if p else None
    oq = torch.empty_like(dq)
    ok = torch.empty((b, p + s, h, d), dtype=torch.bfloat16, device=dev)
    ov = torch.empty_like(ok) if with_v else None
    _native.call("qim_qk_norm_rope_pack", _native.ptr(dq), _native.ptr(dk), _native.ptr(dv), _native.ptr(dck),
                 _native.ptr(dcv), _native.ptr(dw_q), _native.ptr(dw_k), _native.ptr(df), _native.ptr(oq),
                 _native.ptr(ok), _native.ptr(ov), b, s, p, h, d, h * d, 1e-6, 1e-6, _native.stream())
    rq, rk, rv = O.norm_rope_pack(bits(q), bits(k), bits(v) if with_v else bits(q), bits(wq), bits(wk),
                                  freqs.numpy(), bits(ck) if p else None, bits(cv) if p else None)
    assert_bits_equal(bits(oq), rq)
    if with_v:
        assert_bits_equal(bits(ok), rk)
        assert_bits_equal(bits(ov), rv)
    else:
        assert_bits_equal(bits(ok)[:, p:], rk[:, p:])


def test_prepare_attention_inputs_fallbacks(dev):
    """None for unsupported inputs (check_attention_ops.py:37-41)."""
    g = torch.Generator().manual_seed(721)
    q = bf16_randn(g, (1, 16, 4, 128)).to(dev)
    ck = bf16_randn(g, (1, 3, 4, 128)).to(dev)
    w = _RMS(bf16_randn(g, (128,)).to(dev))
    phase = torch.randn(16, 64, generator=g)
    f = torch.polar(torch.ones_like(phase), phase).to(dev)
    pai = attention.prepare_attention_inputs
    assert pai(q, q, q, w, w, None, ck, ck) is None
    assert pai(q.float(), q.float(), q.float(), w, w, f, ck, ck) is None
    assert pai(q.transpose(1, 2), q.transpose(1, 2), q.transpose(1, 2), w, w, f, ck, ck) is None
    assert pai(q, q, q, w, w, f, ck[:, :, :2], ck[:, :, :2]) is None


def test_prepare_attention_inputs_prefix_mutation(dev):
    """Outputs own their memory (check_attention_ops.py:33-37): changing the
    prefix afterwards changes neither the earlier outputs nor anything but
    the prefix part of a new call; a prefix of another batch size is
    unsupported (None)."""
    g = torch.Generator().manual_seed(721)
    b, s, p, h = 2, 49, 1024, 32
    q, k, v = (bf16_randn(g, (b, s, h, 128)).to(dev) for _ in range(3))
    ck, cv = (bf16_randn(g, (b, p, h, 128)).to(dev) for _ in range(2))
    w = _RMS(bf16_randn(g, (128,)).to(dev))
    phase = torch.randn(s, 64, generator=g)
    f = torch.polar(torch.ones_like(phase), phase).to(dev)
    say("prepare_attention_inputs prefix mutation")
    pai = attention.prepare_attention_inputs
    first = pai(q, k, v, w, w, f, ck, cv)
    saved = [x.clone() for x in first]
    ck.add_(1)
    cv.mul_(2)
    second = pai(q, k, v, w, w, f, ck, cv)
    torch.cuda.synchronize()
    for x, y in zip(first, saved):
        assert torch.equal(x, y)
    assert torch.equal(second[0], first[0])
    assert torch.equal(second[1][:, :p], ck) and torch.equal(second[1][:, p:], first[1][:, p:])
    assert torch.equal(second[2][:, :p], cv) and torch.equal(second[2][:, p:], first[2][:, p:])
    assert pai(q, k, v, w, w, f, ck[:1], cv[:1]) is None


def test_layer_norm_scale_fallbacks_equal_eager(dev):
    """Inputs the kernel does not take -- CPU fp32, an affine norm, a strided x
    -- return exactly the eager norm(x) * scale (check_layernorm_ops.py:28-33)."""
    g = torch.Generator().manual_seed(717)
    for device, dtype, affine, strided in [("cpu", torch.float32, False, False), (dev, torch.bfloat16, True, False),
                                           (dev, torch.bfloat16, False, True)]:
        say("layer_norm_scale fallback", device, dtype, affine, strided)
        x = torch.randn(2, 49, 8192 if strided else 4096, generator=g).to(device=device, dtype=dtype)
        if strided:
            x = x[..., ::2]
        scale = torch.randn(2, 1, 4096, generator=g).to(device=device, dtype=dtype)
        norm = torch.nn.LayerNorm(4096, eps=1e-6, elementwise_affine=affine).to(device, dtype)
        if affine:
            with torch.no_grad():
                norm.weight.copy_(torch.randn(4096, generator=g))
                norm.bias.copy_(torch.randn(4096, generator=g))
        before = _native.calls.get("qim_adaln", 0)
        with torch.no_grad():
            got = layernorm.layer_norm_scale(x, scale, norm)
            want = norm(x) * scale
        assert _native.calls.get("qim_adaln", 0) == before
        assert torch.equal(got, want)


def test_qk_norm_rope_config2_and_fused_qkv_view(dev):
    """Config 2 at 1024^2 with the real 3-axis table; q/k read as column
    blocks of a fused (S, 3*H*D) QKV output."""
    S, H, D = 4352, 24, 128
    g = torch.Generator().manual_seed(721)
    qkv = bf16_randn(g, (S, 3 * H * D))
    wq = (torch.rand(D, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    wk = (torch.rand(D, generator=g) * 0.4 + 0.8).to(torch.bfloat16)
    f = O.rope_freqs(O.rope_positions(256, 1, 64, 64))
    freqs = torch.view_as_complex(torch.from_numpy(f))
    say("qk_norm_rope config2")
    qd = qkv.to(dev)
    oq, ok = attention.qk_norm_rope(qd[:, :H * D], qd[:, H * D:2 * H * D], wq.to(dev), wk.to(dev),
                                    freqs.to(dev), heads=H)
    q = qkv[:, :H * D].contiguous().reshape(1, S, H, D)
    k = qkv[:, H * D:2 * H * D].contiguous().reshape(1, S, H, D)
    _check_norm_rope(dev, q, k, wq, wk, f, bits(oq), bits(ok))


# ----------------------------------------------------------------- GEMM --

def _quant_pair(g, m, n, k, wscale=0.02):
    a = bf16_randn(g, (m, k))
    w = bf16_randn(g, (n, k), wscale)
    return a, w


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (130, 512, 384), (1000, 768, 1024), (4352, 3072, 3072)])
def test_mxfp8_gemm_plain(dev, m, n, k):
    g = torch.Generator().manual_seed(1)
    a, w = _quant_pair(g, m, n, k)
    say("gemm", m, n, k)
    aq = mxfp8.quantize(a.to(dev))
    wq = mxfp8.quantize(w.to(dev))
    y = gemm.mx_matmul(aq, wq.values, wq.scales)
    assert y.shape == (m, n)
    rows = np.arange(m) if m * n * k <= 1 << 31 else np.random.default_rng(0).choice(m, 64, replace=False)
    ref = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales), rows=rows)
    got = y.float().cpu().numpy()[rows]
    assert rel_fro(got, ref) < 1e-2
    # bf16 output of an fp32 accumulation: every element within 1 bf16 ulp + accumulation slack
    assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-3 * np.abs(ref).max())


@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 12288), (12288, 4096)])
def test_mxfp8_gemm_reference_model_shapes(dev, k, n):
    """The reference model's linears at 4096 tokens (check_mxfp8.py:54-57:
    out 4096 -> 4096, qkv 4096 -> 12288, mlp_out 12288 -> 4096, every 256th
    input column x12), sampled rows against dequantize-then-matmul."""
    g = torch.Generator().manual_seed(1)
    a = bf16_randn(g, (4096, k))
    a[:, ::256] *= 12
    w = bf16_randn(g, (n, k), k ** -0.5)
    say("gemm model shape", 4096, n, k)
    aq = mxfp8.quantize(a.to(dev))
    wq = mxfp8.quantize(w.to(dev))
    y = gemm.mx_matmul(aq, wq.values, wq.scales)
    rows = np.random.default_rng(k + n).choice(4096, 48, replace=False)
    ref = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales), rows=rows)
    got = y.float().cpu().numpy()[rows]
    assert rel_fro(got, ref) < 1e-2
    assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-3 * np.abs(ref).max())


def test_mxfp8_gemm_bias_config4(dev):
    """Config 4b: [4352 x 3072] x [3072 x 12288] + bias, sampled rows."""
    g = torch.Generator().manual_seed(1)
    a = bf16_randn(g, (4352, 3072))
    mask = torch.rand(a.shape, generator=g) < 0.01
    a[mask] *= 20
    w = bf16_randn(g, (12288, 3072), 0.02)
    bias = bf16_randn(g, (12288,), 0.01)
    say("gemm bias config4")
    aq = mxfp8.quantize(a.to(dev))
    wq = mxfp8.quantize(w.to(dev))
    y = gemm.mx_matmul(aq, wq.values.t(), wq.scales, epilogue="bias", bias=bias.to(dev))
    rows = np.random.default_rng(0).choice(4352, 48, replace=False)
    ref = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales), rows=rows)
    ref = ref + bf16_values(bits(bias))[None, :]
    assert rel_fro(y.float().cpu().numpy()[rows], ref) < 1e-2
    # The path bench.py times: both operands quantized straight into the tiled
    # layout, the same bias epilogue.  Codes and scales equal the row-major
    # quantization's, and the product equals the row-major one bit for bit
    # (same MFMAs in the same order), so it is the oracle's within the bar.
    say("gemm bias config4 tiled")
    at = mxfp8.quantize(a.to(dev), tiled=True)
    wt = mxfp8.quantize(w.to(dev), tiled=True)
    assert torch.equal(mxfp8.as_row_major(at).values, aq.values) and torch.equal(at.scales, aq.scales)
    yt = gemm.mx_matmul(at, wt.values, wt.scales, epilogue="bias", bias=bias.to(dev), weight_tiled=True)
    assert_bits_equal(bits(yt), bits(y))
    assert rel_fro(yt.float().cpu().numpy()[rows], ref) < 1e-2


def _gemm_unsplit(aq, wq, epi, layouts, out, ldo, bias=None, gate=None, res=None, seq=0):
    """The same product through qim_mxfp8_gemm_ex: one workgroup per quarter
    tile over all of K, no workspace."""
    _native.call("qim_mxfp8_gemm_ex", _native.ptr(aq.values), _native.ptr(aq.scales), _native.ptr(wq.values),
                 _native.ptr(wq.scales), aq.rows, wq.values.shape[0], wq.values.shape[1], epi, layouts,
                 _native.ptr(bias), _native.ptr(gate), _native.ptr(res), seq or aq.rows, _native.ptr(out), ldo, None,
                 _native.stream(out.device))


@pytest.mark.parametrize("m,n,k", [(4352, 4096, 12288), (4352, 4096, 256), (4200, 4096, 384), (16640, 3072, 3072)])
def test_mxfp8_gemm_split_tail(dev, m, n, k):
    """Tile grids whose last partial round is a few quarter tiles (272 and 780
    tiles on 256 CUs): mx_matmul splits those quarter tiles over K through a
    workspace (qim_mxfp8_gemm_ws, then the summing epilogue launch).  Against
    the unsplit call the fp32 products differ only by the order of the
    partial sums, and the gated residual and bias outputs by at most that in
    bf16; the split rows are checked against the oracle too."""
    g = torch.Generator().manual_seed(11)
    a = bf16_randn(g, (m, k))
    w = bf16_randn(g, (n, k), 0.02)
    ws_bytes = _native.lib().qim_mxfp8_gemm_ws_bytes(m, n, k, _native.EPI_GATED_RESIDUAL)
    say("gemm split tail", m, n, k, ws_bytes)
    assert ws_bytes > 0
    aq, wq = mxfp8.quantize(a.to(dev)), mxfp8.quantize(w.to(dev))
    # fp32 output, plain epilogue
    before = _native.calls.get("qim_mxfp8_gemm_ws", 0)
    y32 = gemm.mx_matmul(aq, wq.values, wq.scales, dtype=torch.float32)
    assert _native.calls.get("qim_mxfp8_gemm_ws", 0) == before + 1
    u32 = torch.empty_like(y32)
    _gemm_unsplit(aq, wq, _native.EPI_NONE, _native.GEMM_OUT_F32, u32, n)
    torch.cuda.synchronize()
    d = (y32 - u32).abs().max().item()
    assert d <= 1e-5 * u32.abs().max().item(), d
    # sampled rows, the last ones among them, against the oracle
    rows = np.unique(np.concatenate([np.random.default_rng(m).choice(m, 48, replace=False), np.arange(m - 16, m)]))
    ref = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales), rows=rows)
    assert rel_fro(y32.cpu().numpy()[rows], ref) < 1e-2
    # gated residual (two batches) and bias, bf16
    res = bf16_randn(g, (m, n)).to(dev)
    gate = bf16_randn(g, (2, n)).tanh().to(dev)
    seq = (m + 1) // 2
    yg = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue="gated_residual", gate=gate, residual=res, seq=seq)
    ug = torch.empty_like(yg)
    _gemm_unsplit(aq, wq, _native.EPI_GATED_RESIDUAL, 0, ug, n, gate=gate, res=res, seq=seq)
    bias = bf16_randn(g, (n,), 0.01).to(dev)
    yb = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue="bias", bias=bias)
    ub = torch.empty_like(yb)
    _gemm_unsplit(aq, wq, _native.EPI_BIAS, 0, ub, n, bias=bias)
    torch.cuda.synchronize()
    for got, want in ((yg, ug), (yb, ub)):
        # bf16 roundings of fp32 values that differ in the last bits: at most one ulp apart
        diff = (got.float() - want.float()).abs()
        assert (diff <= want.float().abs() * 2.0 ** -7 + 1e-30).all(), diff.max().item()
        assert (diff > 0).float().mean().item() < 1e-2


def test_mxfp8_gemm_gated_residual(dev):
    g = torch.Generator().manual_seed(3)
    m, n, k = 300, 512, 768
    a, w = _quant_pair(g, m, n, k)
    res = bf16_randn(g, (m, n))
    gate = bf16_randn(g, (2, 1, n)).tanh()
    say("gemm gated residual")
    aq, wq = mxfp8.quantize(a.to(dev)), mxfp8.quantize(w.to(dev))
    y = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue="gated_residual", gate=gate.to(dev),
                       residual=res.to(dev), seq=150)
    acc = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales))[:m]
    proj = O.f32_to_bf16(acc).reshape(2, 150, n)
    ref = O.residual(bits(res).reshape(2, 150, n), proj, bits(gate))
    # the GEMM output is within a bf16 ulp of the oracle's; the residual then adds it
    got = bf16_values(bits(y)).reshape(2, 150, n)
    assert rel_fro(got - bf16_values(bits(res)).reshape(2, 150, n),
                   bf16_values(ref) - bf16_values(bits(res)).reshape(2, 150, n)) < 1e-2


def test_mxfp8_gemm_swiglu_epilogues(dev):
    g = torch.Generator().manual_seed(4)
    m, f, k = 260, 512, 384
    a = bf16_randn(g, (m, k))
    wg = bf16_randn(g, (f, k), 0.05)
    wu = bf16_randn(g, (f, k), 0.05)
    say("gemm swiglu")
    aq = mxfp8.quantize(a.to(dev))
    wgu = gemm.interleave_swiglu(wg.to(dev), wu.to(dev))
    wq = mxfp8.quantize(wgu)
    y = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue="swiglu")
    yq = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue="swiglu_quant")
    acc = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales))[:m]
    accg = acc.reshape(m, f // 32, 2, 32)[:, :, 0].reshape(m, f)
    accu = acc.reshape(m, f // 32, 2, 32)[:, :, 1].reshape(m, f)
    ref = O.swiglu(O.f32_to_bf16(accg), O.f32_to_bf16(accu))
    assert y.shape == (m, f)
    assert rel_fro(bf16_values(bits(y)), bf16_values(ref)) < 1e-2
    # the quantized epilogue == quantize of the bf16 epilogue, byte for byte
    sep = mxfp8.quantize(y)
    assert yq.rows == m and np.array_equal(u8(yq.values), u8(sep.values))
    assert np.array_equal(u8(yq.scales), u8(sep.scales))


@pytest.mark.parametrize("m,n,k", [(300, 128, 256), (1000, 640, 512), (4352, 3200, 384), (4352, 4224, 256)])
@pytest.mark.parametrize("epi", ["none", "bias", "gated_residual"])
def test_mxfp8_gemm_half_width_last_column(dev, m, n, k, epi):
    """N % 256 == 128 (the reference converts any N % 128 == 0): the last 128
    columns run as 128 x 128 quarter tiles beside the whole tiles (and, at
    4352 x 4224, beside the quarter tiles of a partial last round), with
    row-major and tiled operands.  Sampled rows and all columns against the
    oracle."""
    g = torch.Generator().manual_seed(m + n + k)
    a = bf16_randn(g, (m, k))
    w = bf16_randn(g, (n, k), 0.05)
    rows = np.unique(np.concatenate([np.random.default_rng(n).choice(m, 24, replace=False), [0, m - 1]]))
    kw = {}
    if epi == "bias":
        kw["bias"] = bf16_randn(g, (n,), 0.01).to(dev)
    elif epi == "gated_residual":
        kw.update(residual=bf16_randn(g, (m, n)).to(dev), gate=bf16_randn(g, (1, 1, n)).tanh().to(dev), seq=m)
    for tiled in (False, True):
        say("gemm half column", m, n, k, epi, tiled)
        aq = mxfp8.quantize(a.to(dev), tiled=tiled)
        wq = mxfp8.quantize(w.to(dev), tiled=tiled)
        y = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue=epi, weight_tiled=tiled, **kw)
        rm_a, rm_w = mxfp8.as_row_major(aq), mxfp8.as_row_major(wq)
        acc = O.mx_gemm(u8(rm_a.values), u8(rm_a.scales), u8(rm_w.values), u8(rm_w.scales), rows=rows)
        if epi == "bias":
            ref = acc + bf16_values(bits(kw["bias"].cpu()))[None, :]
        elif epi == "gated_residual":
            res = bf16_values(bits(kw["residual"].cpu()))[rows]
            ref = res + bf16_values(bits(kw["gate"].cpu())).reshape(1, n) * bf16_values(O.f32_to_bf16(acc))
            got = bf16_values(bits(y))[rows]
            assert rel_fro(got - res, ref - res) < 1e-2
            continue
        else:
            ref = acc
        got = bf16_values(bits(y))[rows]
        assert rel_fro(got, ref) < 1e-2
        assert rel_fro(got[:, -128:], ref[:, -128:]) < 1e-2      # the half-width column block


@pytest.mark.parametrize("m,n,k", [(300, 512, 256), (4352, 384, 512)])
def test_mxfp8_gemm_fp32_and_fp16_outputs(dev, m, n, k):
    """out_dtype of torch._scaled_mm (optimizations/mxfp8.py:34-35): the fp32
    output against the oracle, and the bf16 and fp16 outputs equal to it
    rounded (all three come from the same accumulators)."""
    g = torch.Generator().manual_seed(m + n)
    a = bf16_randn(g, (m, k))
    w = bf16_randn(g, (n, k), 0.05)
    say("gemm out dtypes", m, n, k)
    aq = mxfp8.quantize(a.to(dev))
    wq = mxfp8.quantize(w.to(dev))
    y32 = gemm.mx_matmul(aq, wq.values, wq.scales, dtype=torch.float32)
    y16 = gemm.mx_matmul(aq, wq.values, wq.scales, dtype=torch.float16)
    yb = gemm.mx_matmul(aq, wq.values, wq.scales)
    assert y32.dtype == torch.float32 and y16.dtype == torch.float16 and y32.shape == (m, n)
    rows = np.random.default_rng(1).choice(m, 32, replace=False)
    ref = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales), rows=rows)
    assert rel_fro(y32.cpu().numpy()[rows], ref) < 1e-2
    assert torch.equal(y32.to(torch.bfloat16).view(torch.int16), yb.view(torch.int16))
    assert torch.equal(y32.to(torch.float16).view(torch.int16), y16.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(4352, 4096, 512), (4200, 4096, 384)])
@pytest.mark.parametrize("epi", ["none", "bias", "gated_residual", "swiglu", "swiglu_quant"])
def test_mxfp8_gemm_tail_quarter_tiles(dev, m, n, k, epi):
    """272 tiles on 256 CUs: the last 16 (tile row 16, rows >= 4096) run as
    128 x 128 quarter tiles (with M = 4200 the bottom quarters are padding).
    Every epilogue against the oracle on rows of both kinds of tile."""
    g = torch.Generator().manual_seed(6)
    a = bf16_randn(g, (m, k))
    w = bf16_randn(g, (n, k), 0.05)
    say("gemm tail", m, n, k, epi)
    aq = mxfp8.quantize(a.to(dev))
    wq = mxfp8.quantize(w.to(dev))
    rows = np.concatenate([np.random.default_rng(2).choice(4096, 12, replace=False),
                           np.arange(4096, m, 17), [m - 1]])
    acc = O.mx_gemm(u8(aq.values), u8(aq.scales), u8(wq.values), u8(wq.scales), rows=rows)
    kw, ref = {}, None
    if epi == "bias":
        kw["bias"] = bf16_randn(g, (n,), 0.01).to(dev)
        ref = acc + bf16_values(bits(kw["bias"].cpu()))[None, :]
    elif epi == "gated_residual":
        res, gate = bf16_randn(g, (m, n)), bf16_randn(g, (2, 1, n)).tanh()
        kw.update(residual=res.to(dev), gate=gate.to(dev), seq=m // 2)
        proj = bf16_values(O.f32_to_bf16(acc))
        ref = bf16_values(bits(res))[rows] + bf16_values(bits(gate)).reshape(2, n)[rows // (m // 2)] * proj
    elif epi in ("swiglu", "swiglu_quant"):
        f = n // 2
        accg = acc.reshape(len(rows), f // 32, 2, 32)[:, :, 0].reshape(len(rows), f)
        accu = acc.reshape(len(rows), f // 32, 2, 32)[:, :, 1].reshape(len(rows), f)
        ref = bf16_values(O.swiglu(O.f32_to_bf16(accg), O.f32_to_bf16(accu)))
    else:
        ref = acc
    y = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue=epi, **kw)
    if epi == "swiglu_quant":
        yb = gemm.mx_matmul(aq, wq.values, wq.scales, epilogue="swiglu")
        sep = mxfp8.quantize(yb)
        assert y.rows == m and np.array_equal(u8(y.values), u8(sep.values))
        assert np.array_equal(u8(y.scales), u8(sep.scales))
        y = yb
    got = bf16_values(bits(y))[rows]
    assert rel_fro(got, ref) < 1e-2
    for part in (rows < 4096, rows >= 4096):
        assert rel_fro(got[part], ref[part]) < 1e-2
