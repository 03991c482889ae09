// Row-normalisation kernels: modulated LayerNorm (AdaLN) with optional shift,
// gate and residual, its MXFP8-producing variant, per-head RMSNorm, complex
// RoPE, and the fused QK-RMSNorm + RoPE + prefix K/V pack.
//
// LayerNorm: one workgroup per row; lane l of the W waves holds the 16-byte
// vectors l, l + 64 W, ... of the row in registers, so the row is read from
// HBM exactly once; mean and variance are two-pass float64 sums reduced across
// the workgroup and rounded once to fp32.  RMSNorm/RoPE: one head row of
// D = 128 is 16 lanes x 8 bf16; the float64 sum of squares is reduced inside
// the 16-lane group and the RoPE pairs (x[2j], x[2j+1]) sit in the same lane,
// so no data leaves the lane.
#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

// ---------------------------------------------------------------- AdaLN ----

struct AdaLNArgs {
    const uint16_t *x, *scale, *shift, *gate, *res;
    uint16_t *out;
    uint8_t *q, *qs;
    int64_t rows;      // live rows
    int64_t rows_pad;  // rows launched (Mp for the quantizing variant)
    int D;
    int64_t seq;
    float eps;
    int flags;
    int tiled;         // quantized codes in the GEMM's tiled layout (mxt_offset over rows_pad rows)
    double inv_d;      // fl(1 / D), set by launch_adaln
};

// Byte offset of codes [8j, 8j + 8) of a quantized row.
__device__ __forceinline__ int64_t adaln_code_offset(const AdaLNArgs &p, int64_t row, int j) {
    return p.tiled ? mxt_offset(row, (int64_t)j * 8, p.rows_pad, p.D) : row * p.D + (int64_t)j * 8;
}

constexpr int ADALN_MAX_WAVES = 16;    // 1024 threads per row (masked kernel)
constexpr int ADALN_FULL_WAVES = 4;    // full-coverage kernels: 256 threads, no register cap below 512

// bf16x2 words of the neutral operand of each optional step: adding -0 and
// multiplying by 1 return a bf16 value unchanged (signed zeros included).
constexpr uint32_t BF16X2_NEG_ZERO = 0x80008000u, BF16X2_ONE = 0x3f803f80u;

// The biased variance of a row, rounded to fp32, from one pass: S2 = sum(x^2)
// and mean_d = fl(S1 / D), S1 the float64 sum of the row in any order.  The
// reference value is fl32(fl(V / D)), V the float64 two-pass sum of
// (x - mean_d)^2 in any order.  Both that value and v1 = S2 / D - mean_d^2
// (evaluated below) lie within
//   E = (4D + 32) 2^-53 (|v1| + mean_d^2) (1 + 2^-20)
// of sum((x - mean_d)^2) / D = S2/D - mean_d^2 + 2 mean_d (mean_d - sum(x)/D):
//  - the two-pass sum of D positive terms, each rounded three times, is within
//    (D + 3) 2^-53 of it relatively;
//  - S2 (D - 1 additions of exact squares), the product by fl(1/D), mean_d^2
//    and the subtraction give (D + 2) 2^-53 of the variance plus (D + 4) 2^-53
//    of mean^2;
//  - the last term: mean_d is within 2^-53 |mean_d| of S1 / D, and S1 within
//    (D - 1) 2^-53 sum|x| <= (D - 1) 2^-53 sqrt(D S2) of the exact sum (S1 is
//    exact only while the row's values lie within about 2^(45 - log2 D) of
//    each other), so the term is at most 2^-52 mean_d^2 +
//    (D - 1) 2^-52 |mean_d| sqrt(S2 / D) <= (2D - 1) 2^-53 (mean_d^2 + |v|).
// When v1 - E and v1 + E round to the same fp32 value, so does the reference
// value (rounding is monotonic), and it is returned; otherwise (false) the
// caller runs the second pass.  NaN or infinite sums give a NaN interval end,
// which compares unequal.
__device__ __forceinline__ bool ln_variance(double s2, double mean_d, int D, double inv_d, float &var) {
    const double sq = mean_d * mean_d;
    const double v1 = s2 * inv_d - sq;
    const double e = (4.0 * D + 32.0) * 0x1p-53 * (__builtin_fabs(v1) + sq) * (1.0 + 0x1p-20);
    const float lo = (float)(v1 - e), hi = (float)(v1 + e);
    var = lo;
    return lo == hi;
}

// One modulated LayerNorm row per workgroup of W waves (reference chain, eager
// rounding points: t0 = bf16(LN x), t1 = scale or bf16(1 + scale),
// t2 = bf16(t1 t0), t3 = bf16(t2 + shift), t4 = bf16(gate t3),
// out = bf16(res + t4); kernels/layernorm.py:49-55, kernels/epilogue.py:56-63).
// Thread t holds the 16-byte vectors t, t + 64 W, ... (NV of them) of the row;
// the two-pass float64 statistics are reduced inside each wave, then across
// the W waves through LDS.  Every load is issued before the first reduction.
// FULL: the W * 64 * NV vectors cover the row exactly (D = 3072: NV 3, W 2),
// so no lane tests its index and the optional operands are wave-uniform
// branches; otherwise lanes past the row end hold zeros (any D % 8 == 0).
// Two waves of three vectors per lane was the fastest split of config 1
// measured on MI355X.
// RG: the call has a residual or a gate.  Without them (the block's
// LN * (1 + scale) + shift) the kernel skips their loads, registers and
// arithmetic: with gate 1 and residual -0 those steps return t3 unchanged.
// ALL: shift, residual and gate are all present (config 1's chain): their
// loads are unconditional and issued in the order x, gate, scale, shift,
// residual.  The loads' counter drains in issue order, and loads under a
// branch make every later wait assume the fewest outstanding loads, so with
// the optional-operand branches the statistics waited for the residual too;
// here they wait for x alone, the chain for the column vectors, and only the
// final add for the residual (the last loads).
// PLAIN: the scale is used as given (no QIM_ADALN_ADD_ONE); the general form
// adds -0 and rounds, which leaves a bf16 value unchanged, at 2.5 vector
// instructions per element.
template <bool QUANT, int NV, bool FULL, bool RG, bool ALL = false, bool PLAIN = false>
__global__ __launch_bounds__(FULL ? 64 * ADALN_FULL_WAVES : 64 * ADALN_MAX_WAVES) void k_adaln(AdaLNArgs p) {
    __shared__ double red[3][FULL ? ADALN_FULL_WAVES : ADALN_MAX_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = blockDim.x, nw = nthr >> 6;
    const int64_t row = blockIdx.x;
    const int nvec = p.D >> 3;
    if (row >= p.rows) {
        // Padding row of the quantized output: codes 0, exponents 0.
        if constexpr (QUANT) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int j = tid + nthr * i;
                if (!FULL && j >= nvec) break;
                st_nt(p.q + adaln_code_offset(p, row, j), make_uint2(0, 0));
                if ((lane & 15) == 0)
                    *reinterpret_cast<uint32_t *>(p.qs + mx_scale_offset(row, j >> 2, p.D)) = 0u;
            }
        }
        return;
    }
    const uint32_t b = (uint32_t)row / (uint32_t)p.seq;
    const uint4 *xr = reinterpret_cast<const uint4 *>(p.x + row * p.D);
    const uint4 *sc = reinterpret_cast<const uint4 *>(p.scale + (int64_t)b * p.D);
    const uint4 zero = make_uint4(0, 0, 0, 0);
    const uint4 neg0 = make_uint4(BF16X2_NEG_ZERO, BF16X2_NEG_ZERO, BF16X2_NEG_ZERO, BF16X2_NEG_ZERO);
    const uint4 one = make_uint4(BF16X2_ONE, BF16X2_ONE, BF16X2_ONE, BF16X2_ONE);

    uint4 xv[NV], rv[NV], sv[NV], hv[NV], gv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = tid + nthr * i;
        const bool ok = FULL || j < nvec;
        xv[i] = ok ? ld_nt(xr + j) : zero;
    }
    static_assert(!ALL || (RG && !QUANT), "the all-operand form is the bf16 chain with residual and gate");
    if constexpr (ALL) {
        const uint4 *ga = reinterpret_cast<const uint4 *>(p.gate + (int64_t)b * p.D);
        const uint4 *sh = reinterpret_cast<const uint4 *>(p.shift + (int64_t)b * p.D);
        const uint4 *rr = reinterpret_cast<const uint4 *>(p.res + row * p.D);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = tid + nthr * i;
            gv[i] = (FULL || j < nvec) ? ga[j] : one;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = tid + nthr * i;
            sv[i] = (FULL || j < nvec) ? sc[j] : zero;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = tid + nthr * i;
            hv[i] = (FULL || j < nvec) ? sh[j] : neg0;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = tid + nthr * i;
            rv[i] = (FULL || j < nvec) ? ld_nt(rr + j) : neg0;
        }
    }
    // The per-batch scale and shift vectors (L2-resident, shared by every row)
    // are loaded with x in the bf16-output kernel and after the statistics in
    // the quantizing one, where the shorter live range lowers the register
    // count from 120 to 96 (5 waves per SIMD instead of 4; 4352 rows:
    // 15.4 -> 14.9 us; the bf16 kernel measured no gain).
    constexpr bool LATE = QUANT;
    auto load_scale_shift = [&]() {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = tid + nthr * i;
            sv[i] = (FULL || j < nvec) ? sc[j] : zero;
        }
        if (p.shift) {
            const uint4 *sh = reinterpret_cast<const uint4 *>(p.shift + (int64_t)b * p.D);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int j = tid + nthr * i;
                hv[i] = (FULL || j < nvec) ? sh[j] : neg0;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) hv[i] = neg0;
        }
    };
    if constexpr (!LATE && !ALL) load_scale_shift();
    if constexpr (!ALL) {
        if (RG && p.res) {
            const uint4 *rr = reinterpret_cast<const uint4 *>(p.res + row * p.D);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int j = tid + nthr * i;
                rv[i] = (FULL || j < nvec) ? ld_nt(rr + j) : neg0;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) rv[i] = neg0;
        }
        if (RG && p.gate) {
            const uint4 *ga = reinterpret_cast<const uint4 *>(p.gate + (int64_t)b * p.D);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int j = tid + nthr * i;
                gv[i] = (FULL || j < nvec) ? ga[j] : one;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) gv[i] = one;
        }
    }
    float x[NV][8];
#pragma unroll
    for (int i = 0; i < NV; ++i) unpack8(xv[i], x[i]);

    // Row statistics in float64 (the reference statistics: mean = fp32(S1/D)
    // with S1 the exact float64 sum of the row's bf16 values, and the biased
    // variance fp32(sum((x - mean_d)^2) / D) of a second pass).  One pass
    // gathers S1 and S2 = sum(x^2) (each square exact, so the FMA rounds as
    // the sum would); ln_variance decides the variance's fp32 rounding from
    // them when it can, else (a rare row: var near an fp32 rounding midpoint,
    // or cancellation) the second pass runs.  Absent vectors hold zeros.
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const double v = (double)x[i][t];
            s1 += v;
            s2 = __builtin_fma(v, v, s2);
        }
    s1 = wave_total(s1);
    s2 = wave_total(s2);
    if (lane == 0) {
        red[0][wave] = s1;
        red[1][wave] = s2;
    }
    if constexpr (FULL) {
        // The slots of absent waves hold +0, which leaves the sums unchanged,
        // so every wave adds the four slots in one fixed order.
        static_assert(ADALN_FULL_WAVES == 4, "the cross-wave sums add four slots");
        if (wave == 0 && lane >= nw && lane < ADALN_FULL_WAVES) {
            red[0][lane] = 0.0;
            red[1][lane] = 0.0;
        }
        __syncthreads();
        s1 = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        s2 = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    } else {
        __syncthreads();
        s1 = 0.0;
        s2 = 0.0;
        for (int w = 0; w < nw; ++w) {
            s1 += red[0][w];
            s2 += red[1][w];
        }
    }
    const double mean_d = s1 / (double)p.D;
    float var;
    if (!ln_variance(s2, mean_d, p.D, p.inv_d, var)) {  // uniform over the workgroup
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const bool ok = FULL || tid + nthr * i < nvec;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const double d = ok ? (double)x[i][t] - mean_d : 0.0;
                ss += d * d;
            }
        }
        ss = wave_total(ss);
        if (lane == 0) red[2][wave] = ss;
        __syncthreads();
        ss = 0.0;
        for (int w = 0; w < nw; ++w) ss += red[2][w];
        var = (float)(ss / (double)p.D);
    }
    const float mean = (float)mean_d;
    const float rstd = rstd_of(var, p.eps);
    // Quantized output addressing.  The row is uniform, so vector i's code
    // and scale offsets (mxt_offset or row-major, and mx_scale_offset, at
    // k = 8 j, j = tid + nthr i) are a per-row base, a per-lane 32-bit term
    // and i times a uniform step: nthr is a multiple of 64, so i moves the
    // 64-byte K-slab by nthr / 8, keeps the chunk and byte inside it, and
    // moves the scale dword (4 blocks of 32) by nthr / 16.
    [[maybe_unused]] uint8_t *qrow = nullptr, *srow = nullptr;
    [[maybe_unused]] uint32_t qlane = 0, qstep = 0, slane = 0, sstep = 0;
    if constexpr (QUANT) {
        if (p.tiled) {
            const int64_t r0 = row & ~int64_t(255);
            const uint32_t slab = (uint32_t)(p.rows_pad - r0 < 256 ? p.rows_pad - r0 : 256) * 64;
            qrow = p.q + r0 * p.D + (row - r0) * 64;
            qlane = (uint32_t)(tid >> 3) * slab + ((uint32_t)(((tid >> 1) & 3) ^ mx_chunk_swizzle(row)) << 4) +
                    (uint32_t)(tid & 1) * 8;
            qstep = (uint32_t)(nthr >> 3) * slab;
        } else {
            qrow = p.q + row * p.D;
            qlane = (uint32_t)tid * 8;
            qstep = (uint32_t)nthr * 8;
        }
        srow = p.qs + (row >> 7) * (p.D >> 7) * 512 + (row & 31) * 16 + ((row & 127) >> 5) * 4;
        slane = (uint32_t)(tid >> 4) * 512;
        sstep = (uint32_t)(nthr >> 4) * 512;
    }
    // t1 = bf16(scale + 1) with add_one, else scale (+ -0 leaves it unchanged).
    const float scale_add = (p.flags & QIM_ADALN_ADD_ONE) ? 1.0f : -0.0f;
    if constexpr (LATE) load_scale_shift();

#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = tid + nthr * i;
        if (!FULL && j >= nvec) break;  // uniform inside each 16-lane group when D % 128 == 0
        float sf[8], hf[8], gf[8], rf[8];
        unpack8(sv[i], sf);
        unpack8(hv[i], hf);
        if constexpr (RG) {
            unpack8(gv[i], gf);
            unpack8(rv[i], rf);
        }
        // The output's last rounding (t3 without residual and gate, out with
        // them) packs two values per dword and stays packed: it is what the
        // bf16 store writes and what the quantizer reads.
        uint32_t ow[4];
#pragma unroll
        for (int t = 0; t < 8; t += 2) {
            float a0 = (x[i][t] - mean) * rstd, a1 = (x[i][t + 1] - mean) * rstd;
            rbf2(a0, a1);                                             // t0
            float m0 = sf[t], m1 = sf[t + 1];
            if constexpr (!PLAIN) {
                m0 += scale_add;
                m1 += scale_add;
                rbf2(m0, m1);                                         // t1
            }
            a0 *= m0;
            a1 *= m1;
            rbf2(a0, a1);                                             // t2
            a0 += hf[t];
            a1 += hf[t + 1];
            if constexpr (RG) {
                rbf2(a0, a1);                                         // t3
                a0 *= gf[t];
                a1 *= gf[t + 1];
                rbf2(a0, a1);                                         // t4
                ow[t / 2] = pack_bf16x2(rf[t] + a0, rf[t + 1] + a1);  // out
            } else {
                ow[t / 2] = pack_bf16x2(a0, a1);                      // t3
            }
        }
        const uint4 packed = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        if constexpr (!QUANT) {
            st_nt(reinterpret_cast<uint4 *>(p.out + row * p.D) + j, packed);
        } else {
            // A 32-element block is 4 adjacent lanes; 4 adjacent blocks (16
            // lanes) own one dword of the swizzled scale array.
            // The exponents of lanes + 4, + 8, + 12 arrive by DPP row shifts
            // (inside the lane's 16-lane row).
            int e;
            const uint2 c = quantize8_bf16(packed, e);
            st_nt(qrow + (qlane + (uint32_t)i * qstep), c);
            const uint32_t e1 = dpp_mov<DPP_ROW_SHL4>((uint32_t)e);
            const uint32_t e2 = dpp_mov<DPP_ROW_SHL8>((uint32_t)e);
            const uint32_t e3 = dpp_mov<DPP_ROW_SHL12>((uint32_t)e);
            if ((lane & 15) == 0) {
                const uint32_t word = (uint32_t)e | (e1 << 8) | (e2 << 16) | (e3 << 24);
                *reinterpret_cast<uint32_t *>(srow + (slane + (uint32_t)i * sstep)) = word;
            }
        }
    }
}

// Picks the split of a row: full coverage with NV in {3, 4, 2, 1} vectors per
// lane (the first that divides D/8 into at most 4 whole waves; D = 3072: 3 x 2,
// D = 4096: 4 x 2), else the masked kernel with 2 vectors per lane.
template <bool QUANT, bool RG>
static int launch_adaln_rg(const AdaLNArgs &a, hipStream_t st) {
    const int nvec = a.D / 8;
    if (a.rows_pad >= (1ll << 31) || a.seq >= (1ll << 31)) return fail(QIM_ERR_SHAPE, "adaln: too many rows");
    const dim3 grid((unsigned)a.rows_pad);
    if (nvec % 64 == 0) {
        const int k = nvec / 64;
        // Vectors per lane: 3 (two waves per row at D = 3072) for the quantizing
        // kernel, 2 (three waves) for the bf16 one -- measured at D = 3072:
        // quantizing 15.3 vs 17.0 us (4352 rows), bf16 with residual and gate
        // 7.92 vs 7.76 us (1280 rows).
        if constexpr (!QUANT && RG) {
            // The full chain (shift, residual, gate): branch-free loads; two
            // waves of 3 vectors per lane at D = 3072 (config 1: 6.67 us
            // against 6.75 with three waves of 2, same box).
            if (a.shift && a.res && a.gate) {
                if (k % 3 == 0 && k / 3 <= ADALN_FULL_WAVES) {
                    launch((k_adaln<false, 3, true, true, true>), grid, dim3(64 * (k / 3)), 0, st, a);
                    return QIM_OK;
                }
                if (k % 2 == 0 && k / 2 <= ADALN_FULL_WAVES) {
                    launch((k_adaln<false, 2, true, true, true>), grid, dim3(64 * (k / 2)), 0, st, a);
                    return QIM_OK;
                }
            }
        }
        if (!QUANT && k % 2 == 0 && k / 2 <= ADALN_FULL_WAVES) {
            launch((k_adaln<QUANT, 2, true, RG>), grid, dim3(64 * (k / 2)), 0, st, a);
            return QIM_OK;
        }
        // The block's quantizing AdaLN (no residual or gate, the scale used as
        // given) takes the PLAIN form at D = 3072 (NV 3) and D = 4096 (NV 4).
        constexpr bool PLAIN_OK = QUANT && !RG;
        const bool plain = PLAIN_OK && !(a.flags & QIM_ADALN_ADD_ONE);
        if (k % 3 == 0 && k / 3 <= ADALN_FULL_WAVES) {
            if constexpr (PLAIN_OK) {
                if (plain) {
                    launch((k_adaln<QUANT, 3, true, RG, false, true>), grid, dim3(64 * (k / 3)), 0, st, a);
                    return QIM_OK;
                }
            }
            launch((k_adaln<QUANT, 3, true, RG>), grid, dim3(64 * (k / 3)), 0, st, a);
            return QIM_OK;
        }
        if (k % 4 == 0 && k / 4 <= ADALN_FULL_WAVES) {
            if constexpr (PLAIN_OK) {
                if (plain) {
                    launch((k_adaln<QUANT, 4, true, RG, false, true>), grid, dim3(64 * (k / 4)), 0, st, a);
                    return QIM_OK;
                }
            }
            launch((k_adaln<QUANT, 4, true, RG>), grid, dim3(64 * (k / 4)), 0, st, a);
            return QIM_OK;
        }
        if (k % 2 == 0 && k / 2 <= ADALN_FULL_WAVES) {
            launch((k_adaln<QUANT, 2, true, RG>), grid, dim3(64 * (k / 2)), 0, st, a);
            return QIM_OK;
        }
        if (k <= ADALN_FULL_WAVES) {
            launch((k_adaln<QUANT, 1, true, RG>), grid, dim3(64 * k), 0, st, a);
            return QIM_OK;
        }
    }
    const int waves = (nvec + 127) / 128;
    if (waves > ADALN_MAX_WAVES) return fail(QIM_ERR_SHAPE, "adaln: D=%d exceeds %d", a.D, 8 * 128 * ADALN_MAX_WAVES);
    launch((k_adaln<QUANT, 2, false, RG>), grid, dim3(64 * waves), 0, st, a);
    return QIM_OK;
}

template <bool QUANT>
static int launch_adaln(AdaLNArgs a, hipStream_t st) {
    a.inv_d = 1.0 / (double)a.D;
    return (a.res || a.gate) ? launch_adaln_rg<QUANT, true>(a, st) : launch_adaln_rg<QUANT, false>(a, st);
}

// ---------------------------------------------------- RMSNorm + RoPE ----

struct NormRopeArgs {
    const uint16_t *q, *k, *v, *ck, *cv, *wq, *wk;
    const float *freqs;  // (S, D/2) complex64 = (S, D) fp32 (cos, sin interleaved)
    uint16_t *oq, *ok, *ov;
    int64_t T;           // tokens B * S
    int64_t S, P, H;
    int64_t ldt;         // elements between consecutive tokens of q, k, v (>= H * D)
    float epsq, epsk;
    uint32_t groups;     // head groups of one tensor of one token
    uint32_t main_waves; // waves of the norm/rope part: T * tensors * groups
    int64_t main_blocks; // workgroups of the norm/rope part; the rest copy the prefix
};

// Head rows per lane of one wave: with V 16-byte vectors of a row per lane, a
// row is D / (8 V) lanes and a wave owns U * (64 / (D / (8 V))) heads of one
// tensor of one token.  Measured on MI355X at config 2 (steady-state clocks,
// rotating buffers), V = 1: U = 2 19.4 us, U = 3 19.6 us, U = 1 24-26 us,
// U = 6 (a whole tensor of a token per wave) 21.0 us; a copy-only kernel of
// the same shape 19.3-19.7 us.  The kernel is bound by its vector ALU as much
// as by HBM (~250 vector instructions per wave, ~70 % of its time at
// 4 cycles each), and the per-row work (the float64 row-sum reduction and the
// reciprocal square root) is repeated by every lane of a row, so the launch
// prefers V = 2 (half as many lanes per row, each row's work done once per
// 16 values instead of 8) when the heads divide into whole waves; the other
// splits keep V = 1 and pick U in {2, 3, 4} so that no lane tests its head
// index; other head counts take the masked kernel with U = 3.
constexpr int NR_ROWS = 3;

// Normalise (optionally) and rotate (optionally) the V 8-value chunks a lane
// holds of one head row (chunks c and c + LPR, ... of the row: each 16-byte
// load instruction of the wave covers whole 8 * LPR-value row segments); LPR
// lanes share the row (the helpers are in qim_device.h).
template <int LPR, int V, bool NORM, bool ROPE>
__device__ __forceinline__ void norm_rope_chunks(const uint4 (&xv)[V], uint4 (&out)[V], const float (&w)[V][8],
                                                 float eps, const float4 (&f0)[V], const float4 (&f1)[V]) {
    float x[V][8];
#pragma unroll
    for (int v = 0; v < V; ++v) unpack8(xv[v], x[v]);
    if constexpr (NORM) {
        // The float64 sum of the squares of bf16 values is exact (short of a
        // 2^30 spread of the squares), so adding the chunks' sums first leaves
        // it unchanged.
        double ss = head_sumsq8(x[0]);
#pragma unroll
        for (int v = 1; v < V; ++v) ss += head_sumsq8(x[v]);
        ss = group_sum<LPR>(ss);
        const float r = rstd_of((float)(ss / (double)(LPR * 8 * V)), eps);
#pragma unroll
        for (int v = 0; v < V; ++v) head_rmsnorm8_r(x[v], r, w[v]);
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
        if constexpr (ROPE) head_rope8(x[v], f0[v], f1[v]);
        out[v] = pack8(x[v]);
    }
}

// q/k: (B, S, H, D) -> oq (B, S, H, D), ok (B, P+S, H, D); v -> ov at the
// packed index; the last (gridDim.x - main_blocks) workgroups copy the cached
// prefix ck/cv (B, P, H, D) in front of each batch's rows.
//
// Wave w of the main part owns head group w % groups of tensor
// (w / groups) % NTENS (0 = q, 1 = k, 2 = v) of token w / (NTENS * groups):
// U head rows per lane, LPR lanes per row, V vectors per lane per row, all
// loads issued before any arithmetic.  Neighbouring waves share a token, so
// its RoPE row is read from HBM once and from L2 by the others.  Head slots
// past H are skipped (uniform over the LPR lanes of a row).  v is copied
// unchanged.
template <int D, bool NORM, bool ROPE, int NTENS, int U, bool FULL, int V>
__global__ __launch_bounds__(256) void k_norm_rope(NormRopeArgs p) {
    constexpr int LPR = D / (8 * V);  // lanes per head row
    constexpr int RPI = 64 / LPR;     // head rows per wave instruction
    const int lane = threadIdx.x & 63;
    const int g = lane / LPR, c = lane % LPR;
    if ((int64_t)blockIdx.x < p.main_blocks) {
        // The work item is wave-uniform: computed in scalar registers (the
        // divisions run on the scalar unit); a lane adds only its own offset
        // g * D + c * 8 inside the item's run of head rows.
        const uint32_t w = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (w >= p.main_waves) return;  // whole wave
        const uint32_t per_token = NTENS * p.groups;
        const uint32_t t = w / per_token;
        const uint32_t r = w - t * per_token;
        const uint32_t tensor = r / p.groups;
        const int hb = (int)(r - tensor * p.groups) * (RPI * U);  // first head of the item
        const int h0 = hb + g;
        const int H = (int)p.H;
        const uint32_t bb = t / (uint32_t)p.S, tok = t - bb * (uint32_t)p.S;
        const uint16_t *src = (tensor == 0 ? p.q : tensor == 1 ? p.k : p.v) + (int64_t)t * p.ldt + (int64_t)hb * D;
        uint16_t *dst;
        if (tensor == 0) {
            dst = p.oq + ((int64_t)t * H + hb) * D;
        } else {
            const int64_t kv_row = ((int64_t)bb * (p.P + p.S) + p.P + tok) * H + hb;
            dst = (tensor == 1 ? p.ok : p.ov) + kv_row * D;
        }
        const int off = g * D + c * 8;  // this lane's first vector within the item; vector v at + 8 LPR v
        uint4 x[U][V];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int h = h0 + u * RPI;
            if (FULL || h < H) {
#pragma unroll
                for (int v = 0; v < V; ++v) x[u][v] = ld_nt(src + off + u * RPI * D + v * 8 * LPR);
            }
        }
        if (NTENS == 3 && tensor == 2) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int h = h0 + u * RPI;
                if (FULL || h < H) {
#pragma unroll
                    for (int v = 0; v < V; ++v) st_nt(dst + off + u * RPI * D + v * 8 * LPR, x[u][v]);
                }
            }
            return;
        }
        float4 f0[V], f1[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            f0[v] = make_float4(0.f, 0.f, 0.f, 0.f);
            f1[v] = f0[v];
            if constexpr (ROPE) {
                const float4 *fr = reinterpret_cast<const float4 *>(p.freqs + (int64_t)tok * D + (c + v * LPR) * 8);
                f0[v] = fr[0];
                f1[v] = fr[1];
            }
        }
        float wt[V][8];
        if constexpr (NORM) {
#pragma unroll
            for (int v = 0; v < V; ++v)
                unpack8(*reinterpret_cast<const uint4 *>((tensor == 0 ? p.wq : p.wk) + (c + v * LPR) * 8), wt[v]);
        }
        const float eps = tensor == 0 ? p.epsq : p.epsk;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int h = h0 + u * RPI;
            if (FULL || h < H) {
                uint4 o[V];
                norm_rope_chunks<LPR, V, NORM, ROPE>(x[u], o, wt, eps, f0, f1);
#pragma unroll
                for (int v = 0; v < V; ++v) st_nt(dst + off + u * RPI * D + v * 8 * LPR, o[v]);
            }
        }
    } else if constexpr (NTENS == 3) {
        // Prefix copy: B * P * H rows of D, D / 8 lanes per row.
        constexpr int LPC = D / 8;
        const int cc = lane % LPC;
        const int64_t gi = ((int64_t)blockIdx.x - p.main_blocks) * 256 + threadIdx.x;
        const int64_t row = gi / LPC;
        const int64_t PH = p.P * p.H;
        const int64_t B = p.T / p.S;
        if (row >= B * PH) return;
        const int64_t bb = row / PH, within = row - bb * PH;
        const int64_t dst = (bb * (p.P + p.S) * p.H + within) * D + cc * 8;
        *reinterpret_cast<uint4 *>(p.ok + dst) = *reinterpret_cast<const uint4 *>(p.ck + row * D + cc * 8);
        *reinterpret_cast<uint4 *>(p.ov + dst) = *reinterpret_cast<const uint4 *>(p.cv + row * D + cc * 8);
    }
}

template <int D, bool NORM, bool ROPE, int NTENS, int U, bool FULL, int V = 1>
static void launch_norm_rope_shape(NormRopeArgs a, int64_t prefix_blocks, hipStream_t st) {
    const int64_t rows_per_wave = U * (512 * V / D);
    const int64_t groups = (a.H + rows_per_wave - 1) / rows_per_wave;
    const int64_t waves = a.T * NTENS * groups;
    a.groups = (uint32_t)groups;
    a.main_waves = (uint32_t)waves;
    a.main_blocks = (waves + 3) / 4;
    launch((k_norm_rope<D, NORM, ROPE, NTENS, U, FULL, V>), dim3((unsigned)(a.main_blocks + prefix_blocks)),
                       dim3(256), 0, st, a);
}

template <int D, bool NORM, bool ROPE, int NTENS>
static void launch_norm_rope_d(const NormRopeArgs &a, int64_t prefix_blocks, hipStream_t st) {
    constexpr int64_t RPI = 512 / D;
    if (D >= 128 && a.H % (2 * RPI) == 0)
        launch_norm_rope_shape<D, NORM, ROPE, NTENS, 1, true, 2>(a, prefix_blocks, st);
    else if (a.H % (2 * RPI) == 0) launch_norm_rope_shape<D, NORM, ROPE, NTENS, 2, true>(a, prefix_blocks, st);
    else if (a.H % (3 * RPI) == 0) launch_norm_rope_shape<D, NORM, ROPE, NTENS, 3, true>(a, prefix_blocks, st);
    else if (a.H % (4 * RPI) == 0) launch_norm_rope_shape<D, NORM, ROPE, NTENS, 4, true>(a, prefix_blocks, st);
    else launch_norm_rope_shape<D, NORM, ROPE, NTENS, NR_ROWS, false>(a, prefix_blocks, st);
}

template <bool NORM, bool ROPE, int NTENS>
static int launch_norm_rope(const NormRopeArgs &a, int64_t D, int64_t B, hipStream_t st) {
    if (D != 64 && D != 128 && D != 256)
        return fail(QIM_ERR_SHAPE, "norm/rope: head dim %lld not in {64, 128, 256}", (long long)D);
    // The most waves any split launches (2 head rows per lane per wave).
    const int64_t max_waves = a.T * NTENS * ((a.H + 2 * (512 / D) - 1) / (2 * (512 / D)));
    const int64_t prefix_blocks = (NTENS == 3 && a.P > 0) ? (B * a.P * a.H * (D / 8) + 255) / 256 : 0;
    if (max_waves >= (1ll << 31) || a.H >= (1ll << 30) || a.T >= (1ll << 31) ||
        (max_waves + 3) / 4 + prefix_blocks >= (1ll << 31))
        return fail(QIM_ERR_SHAPE, "norm/rope: too large (%lld tokens x %lld heads)", (long long)a.T, (long long)a.H);
    switch (D) {
        case 64: launch_norm_rope_d<64, NORM, ROPE, NTENS>(a, prefix_blocks, st); break;
        case 128: launch_norm_rope_d<128, NORM, ROPE, NTENS>(a, prefix_blocks, st); break;
        default: launch_norm_rope_d<256, NORM, ROPE, NTENS>(a, prefix_blocks, st); break;
    }
    return QIM_OK;
}

}  // namespace qim

using namespace qim;

static int adaln_common(const char *what, const void *x, const void *scale, const void *res, int64_t rows,
                        int64_t D, int64_t seq, const void *shift, const void *gate) {
    QIM_REQUIRE(x && scale, QIM_ERR_ARG, "%s: null pointer", what);
    QIM_REQUIRE(rows > 0 && D > 0 && seq > 0, QIM_ERR_SHAPE, "%s: empty input", what);
    QIM_REQUIRE(D % 8 == 0 && D <= 16384, QIM_ERR_SHAPE, "%s: D=%lld unsupported (D %% 8 == 0, D <= 16384)", what,
                (long long)D);
    QIM_REQUIRE(aligned16(x) && aligned16(scale) && (!res || aligned16(res)) && (!shift || aligned16(shift)) &&
                    (!gate || aligned16(gate)),
                QIM_ERR_LAYOUT, "%s: operands must be 16-byte aligned", what);
    return QIM_OK;
}

extern "C" int qim_adaln(const void *x, const void *scale, const void *shift, const void *gate, const void *res,
                         void *out, int64_t rows, int64_t D, int64_t seq, float eps, int flags, void *stream) {
    int rc = adaln_common("qim_adaln", x, scale, res, rows, D, seq, shift, gate);
    if (rc) return rc;
    QIM_REQUIRE(out && aligned16(out), QIM_ERR_LAYOUT, "qim_adaln: out must be a 16-byte aligned pointer");
    AdaLNArgs a{(const uint16_t *)x, (const uint16_t *)scale, (const uint16_t *)shift, (const uint16_t *)gate,
                (const uint16_t *)res, (uint16_t *)out, nullptr, nullptr, rows, rows, (int)D, seq, eps, flags, 0};
    rc = launch_adaln<false>(a, as_stream(stream));
    return rc ? rc : check_launch("qim_adaln");
}

extern "C" int qim_adaln_quantize(const void *x, const void *scale, const void *shift, const void *gate,
                                  const void *res, void *q, void *scales, int64_t rows, int64_t D, int64_t seq,
                                  float eps, int flags, void *stream) {
    int rc = adaln_common("qim_adaln_quantize", x, scale, res, rows, D, seq, shift, gate);
    if (rc) return rc;
    QIM_REQUIRE(D % 128 == 0, QIM_ERR_SHAPE, "qim_adaln_quantize: D=%lld is not a multiple of 128", (long long)D);
    QIM_REQUIRE(q && scales && aligned16(q) && aligned16(scales), QIM_ERR_LAYOUT,
                "qim_adaln_quantize: q and scales must be 16-byte aligned pointers");
    AdaLNArgs a{(const uint16_t *)x, (const uint16_t *)scale, (const uint16_t *)shift, (const uint16_t *)gate,
                (const uint16_t *)res, nullptr, (uint8_t *)q, (uint8_t *)scales, rows, (rows + 127) / 128 * 128,
                (int)D, seq, eps, flags, (flags & QIM_ADALN_TILED) != 0};
    rc = launch_adaln<true>(a, as_stream(stream));
    return rc ? rc : check_launch("qim_adaln_quantize");
}

extern "C" int qim_rms_norm(const void *x, const void *w, void *out, int64_t rows, int64_t D, float eps,
                            void *stream) {
    QIM_REQUIRE(x && w && out, QIM_ERR_ARG, "qim_rms_norm: null pointer");
    QIM_REQUIRE(rows > 0, QIM_ERR_SHAPE, "qim_rms_norm: empty input");
    QIM_REQUIRE(aligned16(x) && aligned16(w) && aligned16(out), QIM_ERR_LAYOUT,
                "qim_rms_norm: operands must be 16-byte aligned");
    // No table and no per-token state: the rows are the heads of one token.
    NormRopeArgs a{(const uint16_t *)x, nullptr, nullptr, nullptr, nullptr, (const uint16_t *)w, nullptr,
                   nullptr, (uint16_t *)out, nullptr, nullptr, 1, 1, 0, rows, rows * D, eps, eps, 0, 0, 0};
    int rc = launch_norm_rope<true, false, 1>(a, D, 1, as_stream(stream));
    return rc ? rc : check_launch("qim_rms_norm");
}

extern "C" int qim_rope_qk(const void *q, const void *k, const void *freqs, void *oq, void *ok, int64_t B,
                           int64_t S, int64_t H, int64_t D, void *stream) {
    QIM_REQUIRE(q && k && freqs && oq && ok, QIM_ERR_ARG, "qim_rope_qk: null pointer");
    QIM_REQUIRE(B > 0 && S > 0 && H > 0, QIM_ERR_SHAPE, "qim_rope_qk: empty input");
    QIM_REQUIRE(aligned16(q) && aligned16(k) && aligned16(freqs) && aligned16(oq) && aligned16(ok),
                QIM_ERR_LAYOUT, "qim_rope_qk: operands must be 16-byte aligned");
    NormRopeArgs a{(const uint16_t *)q, (const uint16_t *)k, nullptr, nullptr, nullptr, nullptr, nullptr,
                   (const float *)freqs, (uint16_t *)oq, (uint16_t *)ok, nullptr, B * S, S, 0, H, H * D, 0.f, 0.f,
                   0, 0, 0};
    int rc = launch_norm_rope<false, true, 2>(a, D, B, as_stream(stream));
    return rc ? rc : check_launch("qim_rope_qk");
}

extern "C" int qim_qk_norm_rope_pack(const void *q, const void *k, const void *v, const void *ck, const void *cv,
                                     const void *wq, const void *wk, const void *freqs, void *oq, void *ok,
                                     void *ov, int64_t B, int64_t S, int64_t P, int64_t H, int64_t D, int64_t ldt,
                                     float epsq, float epsk, void *stream) {
    QIM_REQUIRE(q && k && wq && wk && freqs && oq && ok, QIM_ERR_ARG, "qim_qk_norm_rope_pack: null pointer");
    QIM_REQUIRE(B > 0 && S > 0 && H > 0 && P >= 0, QIM_ERR_SHAPE, "qim_qk_norm_rope_pack: empty input");
    QIM_REQUIRE((v == nullptr) == (ov == nullptr), QIM_ERR_ARG, "qim_qk_norm_rope_pack: v and ov go together");
    QIM_REQUIRE(P == 0 || (ck && cv && v), QIM_ERR_ARG,
                "qim_qk_norm_rope_pack: a prefix (P > 0) needs ck, cv, v and ov");
    QIM_REQUIRE(ldt >= H * D && ldt % 8 == 0, QIM_ERR_LAYOUT, "qim_qk_norm_rope_pack: token stride %lld < H*D or not a multiple of 8",
                (long long)ldt);
    const void *ptrs[] = {q, k, v, ck, cv, wq, wk, freqs, oq, ok, ov};
    for (const void *pp : ptrs)
        QIM_REQUIRE(!pp || aligned16(pp), QIM_ERR_LAYOUT, "qim_qk_norm_rope_pack: operands must be 16-byte aligned");
    NormRopeArgs a{(const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v, (const uint16_t *)ck,
                   (const uint16_t *)cv, (const uint16_t *)wq, (const uint16_t *)wk, (const float *)freqs,
                   (uint16_t *)oq, (uint16_t *)ok, (uint16_t *)ov, B * S, S, P, H, ldt, epsq, epsk, 0, 0, 0};
    int rc = v ? launch_norm_rope<true, true, 3>(a, D, B, as_stream(stream))
               : launch_norm_rope<true, true, 2>(a, D, B, as_stream(stream));
    return rc ? rc : check_launch("qim_qk_norm_rope_pack");
}
