// Device helpers shared by every libqim kernel (gfx950 / CDNA4 only).
//
// bf16 values travel as uint16 bit patterns, packed two per dword; E4M3 codes
// four per dword.  Conversions use the gfx950 hardware instructions
// (v_cvt_pk_bf16_f32: round to nearest even; v_cvt_pk_fp8_f32: OCP E4M3, round
// to nearest even); both are checked exhaustively against the CPU oracle
// through qim_debug_bf16_round / qim_debug_e4m3_encode.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qim {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- bf16 ----

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Two fp32 -> packed bf16x2 (a in the low half), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Eager ".to(bfloat16)" boundary: the fp32 value of the bf16 rounding of x.
// Converting the pair (0, x) puts bf16(x) in the high half above a zero low
// half, which is that fp32 value: one v_cvt_pk_bf16_f32 and no unpacking.
__device__ __forceinline__ float rbf(float x) { return __uint_as_float(pack_bf16x2(0.0f, x)); }

// Round two values to bf16: two such conversions (one conversion of the pair
// and two unpacking operations would take three instructions).
__device__ __forceinline__ void rbf2(float &a, float &b) {
    a = rbf(a);
    b = rbf(b);
}

// Unpack 8 bf16 (one 16-byte vector) to fp32.
__device__ __forceinline__ void unpack8(const uint4 &u, float *f) {
    f[0] = bf_lo(u.x); f[1] = bf_hi(u.x); f[2] = bf_lo(u.y); f[3] = bf_hi(u.y);
    f[4] = bf_lo(u.z); f[5] = bf_hi(u.z); f[6] = bf_lo(u.w); f[7] = bf_hi(u.w);
}

// Pack 8 fp32 to 8 bf16 (round to nearest even).
__device__ __forceinline__ uint4 pack8(const float *f) {
    uint4 u;
    u.x = pack_bf16x2(f[0], f[1]); u.y = pack_bf16x2(f[2], f[3]);
    u.z = pack_bf16x2(f[4], f[5]); u.w = pack_bf16x2(f[6], f[7]);
    return u;
}

// Streaming (non-temporal) 16- and 8-byte accesses for operands read or written
// exactly once: they bypass the cache-allocation policy of L2/MALL, which
// raises achieved HBM bandwidth (measured 6.4 vs 6.0 TB/s on a copy).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld_nt(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(void *p, const uint4 &u) {
    const u32x4_t v = {u.x, u.y, u.z, u.w};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(p));
}
__device__ __forceinline__ void st_nt(void *p, const uint2 &u) {
    const u32x2_t v = {u.x, u.y};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x2_t *>(p));
}

// ------------------------------------------------------------ MXFP8 ----

// E8M0 exponent of a 32-element block with maximum |x| = amax: the smallest
// power of two 2^(e-127) with amax / 2^(e-127) <= 448, read from the fp32 bits
// (reference: src/qwen_image_accel/kernels/mxfp8.py:42-48).
__device__ __forceinline__ int mx_exponent(float amax) {
    uint32_t b = __float_as_uint(amax);
    int e = (int)((b >> 23) & 0xffu) - 8 + ((b & 0x7fffffu) > 0x600000u ? 1 : 0);
    e = e < 0 ? 0 : (e > 254 ? 254 : e);
    return amax == 0.0f ? 0 : e;
}

// 2^(127 - e) as an exact fp32 bit pattern (kernels/mxfp8.py:49-51).
__device__ __forceinline__ float mx_inverse(int e) { return __uint_as_float((uint32_t)(254 - e) << 23); }

// Four fp32 -> four E4M3 codes packed little-endian in a dword.
__device__ __forceinline__ uint32_t cvt_e4m3x4(float a, float b, float c, float d) {
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
    return (uint32_t)r;
}

// Scaled conversions (v_cvt_scalef32_pk_fp8_f32 / _bf16): E4M3 RNE of
// x / 2^(E - 127), E the exponent field of the fp32 scale operand (its
// mantissa is ignored; a field of 0 means 2^-127).  With the scale operand
// e << 23 they give the codes of x * 2^(127 - e), i.e. of x * mx_inverse(e),
// without the multiply; the bf16 form also takes its two inputs packed.
// Measured on MI355X over every bf16 input: equal to the oracle's E4M3 RNE of
// x * 2^(127 - e) wherever that is at most 448 in magnitude, for e = 0 (scale
// operand 0.0f), 1, 127 and 254; non-finite and out-of-range inputs convert as
// v_cvt_pk_fp8_f32 converts them.
typedef short i16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float mx_scale_operand(int e) { return __uint_as_float((uint32_t)e << 23); }

// Four fp32 values a..d -> four codes (bytes 0..3) of v / 2^(e - 127).
__device__ __forceinline__ uint32_t cvt_e4m3x4_scaled(float a, float b, float c, float d, float scale) {
    i16x2_t r = {0, 0};
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, a, b, scale, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, c, d, scale, true);
    return __builtin_bit_cast(uint32_t, r);
}

// Two packed bf16 pairs (low half first) -> four codes (bytes 0..3).
__device__ __forceinline__ uint32_t cvt_e4m3x4_bf16(uint32_t ab, uint32_t cd, float scale) {
    i16x2_t r = {0, 0};
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2_t, ab), scale, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2_t, cd), scale, true);
    return __builtin_bit_cast(uint32_t, r);
}

// Byte offset of the E8M0 exponent of (row r, block kb) of a (rows, K) tensor
// in the 128x4 swizzled layout (kernels/mxfp8.py:53-56).
__device__ __forceinline__ int64_t mx_scale_offset(int64_t r, int64_t kb, int64_t K) {
    return ((r >> 7) * (K >> 7) + (kb >> 2)) * 512 + (r & 31) * 16 + ((r & 127) >> 5) * 4 + (kb & 3);
}

// Position of 16-byte chunk c (0..3) of row r's 64-byte K-slab in LDS and in
// the tiled code layout: chunk c ^ swizzle(r), which spreads the rows read by
// one ds_read_b128 group over distinct banks.
__device__ __forceinline__ int mx_chunk_swizzle(int64_t r) { return (int)(((r >> 1) ^ (r >> 2)) & 3); }

// Byte offset of code (r, k) of an (R, K) E4M3 matrix (R % 128 == 0) in the
// tiled layout: rows in super-blocks of 256 (the last holds R % 256 rows if
// that is 128); inside a super-block of n rows from row r0, 64-byte K-slab s
// is n * 64 contiguous bytes at r0 * K + s * n * 64, row r's 64 bytes at
// (r - r0) * 64 inside it, and its 16-byte chunk c at chunk c ^ swizzle(r).
// One 16-row group of one slab is then exactly the 1 KiB LDS image the GEMM
// loads with one contiguous DMA instruction.
__device__ __forceinline__ int64_t mxt_offset(int64_t r, int64_t k, int64_t R, int64_t K) {
    const int64_t r0 = r & ~int64_t(255);
    const int64_t n = R - r0 < 256 ? R - r0 : 256;
    return r0 * K + (k >> 6) * n * 64 + (r - r0) * 64 + ((((k >> 4) & 3) ^ mx_chunk_swizzle(r)) << 4) + (k & 15);
}

// |x| maximum of 8 values, as an fp32 bit pattern compared as unsigned
// (monotonic for non-NaN values; no canonicalisation needed).
__device__ __forceinline__ uint32_t absmax_bits8(const float *f) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t a = __float_as_uint(f[i]) & 0x7fffffffu;
        m = a > m ? a : m;
    }
    return m;
}

// --------------------------------------------------------- shuffles ----

// Lane exchange with lane ^ MASK inside the wave.  MASK 1, 2 use DPP quad
// permutes; masks below 32 use ds_swizzle (bit mode); 32 uses ds_bpermute.
template <int MASK>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (MASK == 1) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
    } else if constexpr (MASK == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
    } else if constexpr (MASK < 32) {
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (MASK << 10) | 0x1F);
    } else {
        return (uint32_t)__shfl_xor((int)v, MASK, 64);
    }
}

template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
    return __uint_as_float(xor_lane<MASK>(__float_as_uint(v)));
}

// Row-local DPP moves: lane i reads lane (i ^ 1), (i ^ 2) inside its quad, the
// mirrored lane of its 8-lane half-row (i ^ 7) and of its 16-lane row (i ^ 15).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __uint_as_float(dpp_mov<CTRL>(__float_as_uint(v)));
}
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_ROW_MIRROR = 0x140;
// row_shl:n -- lane l of a 16-lane row receives lane l + n of the same row
// (lanes past the row's end are not meaningful).
constexpr int DPP_ROW_SHL4 = 0x104, DPP_ROW_SHL8 = 0x108, DPP_ROW_SHL12 = 0x10C;

// Reduction over groups of WIDTH consecutive lanes (WIDTH a power of two <= 64);
// every lane of the group receives the total.  Widths up to 16 stay in DPP
// (quad permutes, then the half-row and row mirrors: after the quad steps every
// lane holds its quad's total, and a mirror pairs each lane with a lane of the
// other half); 32 and 64 add a swizzle and a cross-half exchange.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (WIDTH >= 2) v += dpp_mov<DPP_QUAD_XOR1>(v);
    if constexpr (WIDTH >= 4) v += dpp_mov<DPP_QUAD_XOR2>(v);
    if constexpr (WIDTH >= 8) v += dpp_mov<DPP_HALF_MIRROR>(v);
    if constexpr (WIDTH >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
    if constexpr (WIDTH >= 32) v += xor_lane<16>(v);
    if constexpr (WIDTH >= 64) v += xor_lane<32>(v);
    return v;
}

// fp64 versions of the lane moves (each half moved separately) and of
// group_sum, for the row statistics of the normalisations.
template <int CTRL>
__device__ __forceinline__ double dpp_mov(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = dpp_mov<CTRL>((uint32_t)u), hi = dpp_mov<CTRL>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, lo | (hi << 32));
}
template <int MASK>
__device__ __forceinline__ double xor_lane(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = xor_lane<MASK>((uint32_t)u), hi = xor_lane<MASK>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, lo | (hi << 32));
}
template <int WIDTH>
__device__ __forceinline__ double group_sum(double v) {
    if constexpr (WIDTH >= 2) v += dpp_mov<DPP_QUAD_XOR1>(v);
    if constexpr (WIDTH >= 4) v += dpp_mov<DPP_QUAD_XOR2>(v);
    if constexpr (WIDTH >= 8) v += dpp_mov<DPP_HALF_MIRROR>(v);
    if constexpr (WIDTH >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
    if constexpr (WIDTH >= 32) v += xor_lane<16>(v);
    if constexpr (WIDTH >= 64) v += xor_lane<32>(v);
    return v;
}

// Total over the 64 lanes of a wave, returned wave-uniform, without LDS: the
// 16-lane rows reduce by DPP (every lane then holds its row's total), DPP
// row_bcast:15 adds the last lane of rows 0 and 2 into rows 1 and 3, and
// row_bcast:31 adds lane 31 into rows 2 and 3, so lane 63 holds the total.
// Lanes of rows a broadcast does not write add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_bcast(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xF, false);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xF, false);
    return __builtin_bit_cast(double, lo | (hi << 32));
}
constexpr int DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143;

__device__ __forceinline__ double wave_total(double v) {
    v = group_sum<16>(v);
    v += dpp_bcast<DPP_ROW_BCAST15, 0xA>(v);
    v += dpp_bcast<DPP_ROW_BCAST31, 0xC>(v);
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
    return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}

// Reciprocal square root of (var + eps) as the normalisations' reference
// statistics define it: t = var + eps in fp32, then R = fp32(1 / sqrt(t))
// evaluated in float64 (IEEE sqrt and divide) and rounded once.
//
// Fast path with the same result: y = v_rsq_f32(t) (relative error d < 2^-22)
// refined by one float64 Newton step, after which the relative error is
// 1.5 d^2 + O(2^-52) < 2^-42, so the exact 1/sqrt(t) and the float64 value of
// R both lie within y (1 +- 2^-38) (the margin allows d up to 2^-19).  When
// both ends of that interval round to the same fp32 value, so does everything
// inside it, R included; otherwise (a value within 2^-38 of an fp32 rounding
// midpoint, about one in 8000, a non-finite t, or a t that is not positive:
// v_rsq_f32 takes a negative denormal for -0 and the step then gives -inf,
// not NaN) the float64 expression is evaluated.  Checked against that
// expression for all 2^32 fp32 values of var (qim_debug_rstd_sweep).
__device__ __forceinline__ float rstd_of(float var, float eps) {
    const float t = var + eps;
    const double td = (double)t;
    double y = (double)__builtin_amdgcn_rsqf(t);
    y = __builtin_fma(y, __builtin_fma(-td * y, y, 1.0) * 0.5, y);
    const float lo = (float)(y * (1.0 - 0x1p-38)), hi = (float)(y * (1.0 + 0x1p-38));
    if (__builtin_expect(lo == hi && t > 0.0f, 1)) return lo;
    return (float)(1.0 / sqrt(td));
}

// Per-head RMSNorm + RoPE of one 8-value chunk of a head row (Diffusers
// RMSNorm: n = bf16(x * rsqrt(mean(x^2) + eps)), out = bf16(n * w); then the
// complex rotation of the pairs (x[2j], x[2j+1]), reference
// kernels/bf16.py:52-55 and kernels/elementwise.py:53-56).
//
// The sum of squares is taken in float64.  The square of a bf16 value has at
// most 16 significant bits, so the sum of a 128-value row is exact while its
// nonzero squares lie within 2^30 of each other, and it then does not depend on
// how the lanes of a row are reduced; it is rounded once to the fp32 mean.
// With a wider spread the smallest squares are rounded at 2^-53 of the sum, and
// another reduction order can change the fp32 mean only when the exact value
// lies within that distance of an fp32 rounding boundary.
// (The square of a bf16 value is exact in float64, so the fused multiply-add
// rounds exactly as a multiply then an add would.)
__device__ __forceinline__ double head_sumsq8(const float *x) {
    double ss = 0.0;
#pragma unroll
    for (int t = 0; t < 8; ++t) ss = __builtin_fma((double)x[t], (double)x[t], ss);
    return ss;
}
// x: the chunk; ss: the row's total sum of squares over `width` values; w: the
// chunk's 8 weights.  Roundings are paired (one v_cvt_pk_bf16_f32 per two).
// head_rmsnorm8 with the row's reciprocal square root r already computed.
__device__ __forceinline__ void head_rmsnorm8_r(float *x, float r, const float *w) {
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        float a = x[t] * r, b = x[t + 1] * r;
        rbf2(a, b);
        a *= w[t];
        b *= w[t + 1];
        rbf2(a, b);
        x[t] = a;
        x[t + 1] = b;
    }
}
__device__ __forceinline__ void head_rmsnorm8(float *x, double ss, int width, float eps, const float *w) {
    const float r = rstd_of((float)(ss / (double)width), eps);
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        float a = x[t] * r, b = x[t + 1] * r;
        rbf2(a, b);
        a *= w[t];
        b *= w[t + 1];
        rbf2(a, b);
        x[t] = a;
        x[t + 1] = b;
    }
}
// f0, f1: the (cos, sin) pairs of the chunk's 4 complex positions.  Same FMA
// order as the CUDA complex multiply the reference keeps.
__device__ __forceinline__ void head_rope8(float *x, const float4 &f0, const float4 &f1) {
    const float c[4] = {f0.x, f0.z, f1.x, f1.z};
    const float s[4] = {f0.y, f0.w, f1.y, f1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float xr = x[2 * j], xi = x[2 * j + 1];
        const float re = __builtin_fmaf(xr, c[j], -(xi * s[j]));
        const float im = __builtin_fmaf(xi, c[j], xr * s[j]);
        x[2 * j] = re;
        x[2 * j + 1] = im;
    }
}

template <int WIDTH>
__device__ __forceinline__ uint32_t group_umax(uint32_t v) {
    uint32_t o;
    if constexpr (WIDTH >= 2) { o = dpp_mov<DPP_QUAD_XOR1>(v); v = o > v ? o : v; }
    if constexpr (WIDTH >= 4) { o = dpp_mov<DPP_QUAD_XOR2>(v); v = o > v ? o : v; }
    if constexpr (WIDTH >= 8) { o = dpp_mov<DPP_HALF_MIRROR>(v); v = o > v ? o : v; }
    if constexpr (WIDTH >= 16) { o = dpp_mov<DPP_ROW_MIRROR>(v); v = o > v ? o : v; }
    if constexpr (WIDTH >= 32) { o = xor_lane<16>(v); v = o > v ? o : v; }
    if constexpr (WIDTH >= 64) { o = xor_lane<32>(v); v = o > v ? o : v; }
    return v;
}

// Quantize one lane's 8 values, which are one quarter of a 32-element block
// spread over lanes (4j .. 4j+3).  Returns the packed codes; e = exponent.
__device__ __forceinline__ uint2 quantize8(const float *f, int &e) {
    uint32_t m = absmax_bits8(f);
    m = group_umax<4>(m);
    e = mx_exponent(__uint_as_float(m));
    const float s = mx_scale_operand(e);
    uint2 c;
    c.x = cvt_e4m3x4_scaled(f[0], f[1], f[2], f[3], s);
    c.y = cvt_e4m3x4_scaled(f[4], f[5], f[6], f[7], s);
    return c;
}

// fp32 bits of the largest magnitude among 8 packed bf16 values: the
// magnitudes as unsigned 16-bit halves (their order is the values' order,
// NaN above everything) through packed 16-bit maxima, widened to fp32 bits --
// the same as absmax_bits8 of the unpacked values.
__device__ __forceinline__ uint32_t absmax_bits_bf16x8(const uint4 &u) {
    typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
    const u16x2_t a = __builtin_bit_cast(u16x2_t, u.x & 0x7fff7fffu), b = __builtin_bit_cast(u16x2_t, u.y & 0x7fff7fffu);
    const u16x2_t c = __builtin_bit_cast(u16x2_t, u.z & 0x7fff7fffu), d = __builtin_bit_cast(u16x2_t, u.w & 0x7fff7fffu);
    const u16x2_t m = __builtin_elementwise_max(__builtin_elementwise_max(a, b), __builtin_elementwise_max(c, d));
    const uint32_t hi = m.y, lo = m.x;
    return (hi > lo ? hi : lo) << 16;
}

// quantize8 of 8 packed bf16 values (one 16-byte vector): the same codes and
// exponent as quantize8 of the unpacked values, without unpacking them.
__device__ __forceinline__ uint2 quantize8_bf16(const uint4 &u, int &e) {
    uint32_t m = group_umax<4>(absmax_bits_bf16x8(u));
    e = mx_exponent(__uint_as_float(m));
    const float s = mx_scale_operand(e);
    return make_uint2(cvt_e4m3x4_bf16(u.x, u.y, s), cvt_e4m3x4_bf16(u.z, u.w, s));
}

// ------------------------------------------------------------- math ----

// SiLU with the reference's rounding: bf16(g / (1 + exp(-g))) with an IEEE
// (correctly rounded) fp32 divide -- the default for '/' in HIP without
// fast-math -- and the device library's expf (kernels/bf16.py:17-22).
__device__ __forceinline__ float silu_exact(float g) { return g / (1.0f + expf(-g)); }

// Width, in fp32 ulps, of the band around each bf16 rounding midpoint in which
// the fast SiLU estimate is not trusted.  The estimate is within 3 ulps of
// silu_exact for every bf16 input with |g| < 64 (measured exhaustively).
constexpr uint32_t SILU_BAND = 8;

// bf16(silu(g)) for bf16 values g, bit-identical to rbf(silu_exact(g)).
// Fast path: e^-g = 2^t (v_exp_f32) with the rounding error of t = -g log2(e)
// folded back in to first order, and a hardware reciprocal (v_rcp_f32); its
// result is used when it lies more than SILU_BAND ulps from a bf16 rounding
// midpoint, where an error below the band cannot change the rounding.  The
// rare rest (about 2^-12 of the inputs) and |g| >= 64 (where v_rcp_f32 flushes
// the tiny reciprocal of 1 + e^-g) take the exact path.  An exhaustive GPU test
// over all 65536 bf16 inputs checks the identity.
__device__ __forceinline__ float silu_fast(float g) {
    constexpr float NL1 = -1.44269502f;                    // -log2(e), rounded
    constexpr float NL2 = -1.92596299e-08f;                // -(log2(e) - 1.44269502f)
    const float t = g * NL1;
    float r = __builtin_fmaf(g, NL1, -t);                  // exact error of the product
    r = __builtin_fmaf(g, NL2, r);
    float e = __builtin_amdgcn_exp2f(t);
    e = __builtin_fmaf(e * r, 0.693147181f, e);            // e * 2^r to first order
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// Distance (mod 2^16, in fp32 ulps, offset by SILU_BAND) of y from the next
// bf16 rounding midpoint: below 2 * SILU_BAND means "within the band".
__device__ __forceinline__ uint32_t silu_band_key(float y) {
    return (__float_as_uint(y) + (SILU_BAND - 0x8000u)) & 0xffffu;
}

// N values at once: the N fast estimates (independent chains the scheduler
// can interleave), rounded in pairs; the band test and the |g| < 64 test are
// folded into a running minimum and maximum, and one rarely taken branch
// redoes, exactly, the values that need it.  y[i] is rounded to bf16.
template <int N>
__device__ __forceinline__ void silu_bf16_n(const float *g, float *y) {
    uint32_t key = 0xffffu;
    float gmax = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        y[i] = silu_fast(g[i]);
        const uint32_t k = silu_band_key(y[i]);
        key = k < key ? k : key;
        gmax = __builtin_fmaxf(gmax, __builtin_fabsf(g[i]));  // NaN inputs: y is NaN either way
    }
#pragma unroll
    for (int i = 0; i + 1 < N; i += 2) rbf2(y[i], y[i + 1]);
    if constexpr (N % 2) y[N - 1] = rbf(y[N - 1]);
    if (__builtin_expect(key < 2u * SILU_BAND || !(gmax < 64.0f), 0)) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float f = silu_fast(g[i]);
            if (silu_band_key(f) < 2u * SILU_BAND || !(__builtin_fabsf(g[i]) < 64.0f)) y[i] = rbf(silu_exact(g[i]));
        }
    }
}

__device__ __forceinline__ float silu_bf16(float g) {
    float y;
    silu_bf16_n<1>(&g, &y);
    return y;
}


}  // namespace qim
