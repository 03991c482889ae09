// Row-normalisation kernels: modulated LayerNorm (AdaLN) with optional shift,
// gate and residual, its MXFP8-producing variant, per-head RMSNorm, complex
// RoPE, and the fused QK-RMSNorm + RoPE + prefix K/V pack.
//
// LayerNorm: one wave per row; lane l holds the 16-byte vectors l, l+64, ...
// of the row in registers (D = 3072 -> 6 vectors), so the row is read from HBM
// exactly once; mean and variance are exact two-pass fp32 sums reduced across
// the wave.  RMSNorm/RoPE: one head row of D = 128 is 16 lanes x 8 bf16; the
// sum of squares is reduced inside the 16-lane group and the RoPE pairs
// (x[2j], x[2j+1]) sit in the same lane, so no data leaves the lane.
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
};

constexpr int ADALN_NV = 2;            // 16-byte vectors per lane
constexpr int ADALN_MAX_WAVES = 16;    // 1024 threads: D <= 16384

// bf16x2 words of the neutral operand of each optional step: adding -0 and
// multiplying by 1 return a bf16 value unchanged (signed zeros included), so
// an absent shift, gate or residual costs arithmetic but no branch.
constexpr uint32_t BF16X2_NEG_ZERO = 0x80008000u, BF16X2_ONE = 0x3f803f80u;

// One modulated LayerNorm row per workgroup of W waves (reference chain, eager
// rounding points: t0 = bf16(LN x), t1 = scale or bf16(1 + scale),
// t2 = bf16(t1 t0), t3 = bf16(t2 + shift), t4 = bf16(gate t3),
// out = bf16(res + t4); kernels/layernorm.py:49-55, kernels/epilogue.py:127-133).
// Thread t holds vectors t and t + 64 W of the row; the two-pass statistics
// are reduced inside each wave, then across the W waves through LDS.  Every
// load is issued before the first reduction.
template <bool QUANT>
__global__ __launch_bounds__(1024) void k_adaln(AdaLNArgs p) {
    constexpr int NV = ADALN_NV;
    __shared__ float red[2][ADALN_MAX_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = blockDim.x, nw = nthr >> 6;
    const int64_t row = blockIdx.x;
    const int nvec = p.D >> 3;
    const bool live = row < p.rows;
    const int64_t b = live ? row / p.seq : 0;
    const uint4 *xr = reinterpret_cast<const uint4 *>(p.x + row * p.D);
    const uint4 *rr = p.res ? reinterpret_cast<const uint4 *>(p.res + row * p.D) : nullptr;
    const uint4 *sc = reinterpret_cast<const uint4 *>(p.scale + b * p.D);
    const uint4 *sh = p.shift ? reinterpret_cast<const uint4 *>(p.shift + b * p.D) : nullptr;
    const uint4 *ga = p.gate ? reinterpret_cast<const uint4 *>(p.gate + b * p.D) : nullptr;
    const uint4 neg0 = make_uint4(BF16X2_NEG_ZERO, BF16X2_NEG_ZERO, BF16X2_NEG_ZERO, BF16X2_NEG_ZERO);
    const uint4 one = make_uint4(BF16X2_ONE, BF16X2_ONE, BF16X2_ONE, BF16X2_ONE);

    uint4 xv[NV], rv[NV], sv[NV], hv[NV], gv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = tid + nthr * i;
        const bool ok = live && j < nvec;
        xv[i] = ok ? ld_nt(xr + j) : make_uint4(0, 0, 0, 0);
        rv[i] = (ok && rr) ? ld_nt(rr + j) : neg0;
        sv[i] = ok ? sc[j] : make_uint4(0, 0, 0, 0);
        hv[i] = (ok && sh) ? sh[j] : neg0;
        gv[i] = (ok && ga) ? ga[j] : one;
    }
    float x[NV][8];
#pragma unroll
    for (int i = 0; i < NV; ++i) unpack8(xv[i], x[i]);

    // Two-pass statistics in fp32 (absent vectors hold zeros and add nothing).
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) s += x[i][t];
    s = group_sum<64>(s);
    if (lane == 0) red[0][wave] = s;
    __syncthreads();
    s = 0.0f;
    for (int w = 0; w < nw; ++w) s += red[0][w];
    const float mean = s / (float)p.D;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const bool ok = tid + nthr * i < nvec;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float d = ok ? x[i][t] - mean : 0.0f;
            ss = __builtin_fmaf(d, d, ss);
        }
    }
    ss = group_sum<64>(ss);
    if (lane == 0) red[1][wave] = ss;
    __syncthreads();
    ss = 0.0f;
    for (int w = 0; w < nw; ++w) ss += red[1][w];
    const float rstd = 1.0f / sqrtf(ss / (float)p.D + p.eps);
    // t1 = bf16(scale + 1) with add_one, else scale (+ -0 leaves it unchanged).
    const float scale_add = (p.flags & QIM_ADALN_ADD_ONE) ? 1.0f : -0.0f;

#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = tid + nthr * i;
        if (j >= nvec) break;  // uniform inside each 16-lane group when D % 128 == 0
        float sf[8], hf[8], gf[8], rf[8], o[8];
        unpack8(sv[i], sf);
        unpack8(hv[i], hf);
        unpack8(gv[i], gf);
        unpack8(rv[i], rf);
#pragma unroll
        for (int t = 0; t < 8; t += 2) {
            float a0 = (x[i][t] - mean) * rstd, a1 = (x[i][t + 1] - mean) * rstd;
            rbf2(a0, a1);                                             // t0
            float m0 = sf[t] + scale_add, m1 = sf[t + 1] + scale_add;
            rbf2(m0, m1);                                             // t1
            a0 *= m0;
            a1 *= m1;
            rbf2(a0, a1);                                             // t2
            a0 += hf[t];
            a1 += hf[t + 1];
            rbf2(a0, a1);                                             // t3
            a0 *= gf[t];
            a1 *= gf[t + 1];
            rbf2(a0, a1);                                             // t4
            o[t] = rf[t] + a0;
            o[t + 1] = rf[t + 1] + a1;
        }
        if (!live) {
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t] = 0.0f;  // padding rows of the quantized output
        }
        if constexpr (!QUANT) {
            st_nt(reinterpret_cast<uint4 *>(p.out + row * p.D) + j, pack8(o));
        } else {
            rbf2(o[0], o[1]);
            rbf2(o[2], o[3]);
            rbf2(o[4], o[5]);
            rbf2(o[6], o[7]);
            // A 32-element block is 4 adjacent lanes; 4 adjacent blocks (16
            // lanes) own one dword of the swizzled scale array.
            const uint32_t m = group_umax<4>(absmax_bits8(o));
            const int e = mx_exponent(__uint_as_float(m));
            const float inv = mx_inverse(e);
            uint2 c;
            c.x = cvt_e4m3x4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
            c.y = cvt_e4m3x4(o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv);
            st_nt(reinterpret_cast<uint2 *>(p.q + row * p.D) + j, c);
            const uint32_t e1 = (uint32_t)__shfl((int)e, lane + 4, 64);
            const uint32_t e2 = (uint32_t)__shfl((int)e, lane + 8, 64);
            const uint32_t e3 = (uint32_t)__shfl((int)e, lane + 12, 64);
            if ((lane & 15) == 0) {
                const int64_t kb = (int64_t)j >> 2;  // block index of this lane, multiple of 4
                const uint32_t word = (uint32_t)e | (e1 << 8) | (e2 << 16) | (e3 << 24);
                *reinterpret_cast<uint32_t *>(p.qs + mx_scale_offset(row, kb, p.D)) = word;
            }
        }
    }
}

template <bool QUANT>
static int launch_adaln(const AdaLNArgs &a, hipStream_t st) {
    const int nvec = a.D / 8;
    const int waves = (nvec + 64 * ADALN_NV - 1) / (64 * ADALN_NV);
    if (waves > ADALN_MAX_WAVES) return fail(QIM_ERR_SHAPE, "adaln: D=%d exceeds %d", a.D, 8 * 64 * ADALN_NV * ADALN_MAX_WAVES);
    if (a.rows_pad >= (1ll << 31)) return fail(QIM_ERR_SHAPE, "adaln: too many rows");
    hipLaunchKernelGGL((k_adaln<QUANT>), dim3((unsigned)a.rows_pad), dim3(64 * waves), 0, st, a);
    return QIM_OK;
}

// ---------------------------------------------------- RMSNorm + RoPE ----

struct NormRopeArgs {
    const uint16_t *q, *k, *v, *ck, *cv, *wq, *wk;
    const float *freqs;  // (S, D/2) complex64 = (S, D) fp32 (cos, sin interleaved)
    uint16_t *oq, *ok, *ov;
    int64_t rows;        // B * S * H
    int64_t S, P, H;
    int64_t ldt;         // elements between consecutive tokens of q, k, v (>= H * D)
    float epsq, epsk;
    int64_t main_blocks; // workgroups of the norm/rope part; the rest copy the prefix
};

// Normalise (optionally) and rotate (optionally) one 8-value chunk of a head
// row; LPR lanes share the row.  Roundings are paired (one v_cvt_pk_bf16_f32
// per two values).
template <int LPR, bool NORM, bool ROPE>
__device__ __forceinline__ uint4 norm_rope_chunk(const uint4 &xv, const float *w, float eps, const float4 &f0,
                                                 const float4 &f1) {
    float x[8];
    unpack8(xv, x);
    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) ss = __builtin_fmaf(x[t], x[t], ss);
        ss = group_sum<LPR>(ss);
        const float r = 1.0f / sqrtf(ss / (float)(LPR * 8) + eps);
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
    if constexpr (ROPE) {
        const float c[4] = {f0.x, f0.z, f1.x, f1.z};
        const float s[4] = {f0.y, f0.w, f1.y, f1.w};
        float o[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float xr = x[2 * j], xi = x[2 * j + 1];
            // Same FMA order as the CUDA complex multiply the reference keeps
            // (kernels/elementwise.py:53-56).
            o[2 * j] = __builtin_fmaf(xr, c[j], -(xi * s[j]));
            o[2 * j + 1] = __builtin_fmaf(xi, c[j], xr * s[j]);
        }
        return pack8(o);
    } else {
        return pack8(x);
    }
}

// q/k: (B, S, H, D) -> oq (B, S, H, D), ok (B, P+S, H, D); v -> ov at the
// packed index; the last (gridDim.x - main_blocks) workgroups copy the
// cached prefix ck/cv (B, P, H, D) in front of each batch's rows.
//
// One wave per token: its LPR-lane groups walk the token's heads (RPI heads per
// instruction), so each lane loads its 8-value slice of the RoPE table and of
// the two norm weights once and reuses them for every head; all loads of the
// token are issued before any arithmetic.  Head slots past H are skipped (for
// H % RPI == 0 a whole wave skips them together).
template <int D, bool NORM, bool ROPE, bool HAS_K, bool HAS_V>
__global__ __launch_bounds__(256) void k_norm_rope(NormRopeArgs p) {
    constexpr int LPR = D / 8;       // lanes per head row
    constexpr int RPI = 64 / LPR;    // head rows per wave instruction
    constexpr int UNROLL = 8;        // head rows in flight per lane
    const int lane = threadIdx.x & 63;
    const int g = lane / LPR, c = lane % LPR;
    if ((int64_t)blockIdx.x < p.main_blocks) {
        const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // token, 0 .. B*S-1
        if (t * p.H >= p.rows) return;                                   // whole wave
        const int64_t bb = t / p.S, tok = t - bb * p.S;
        const int H = (int)p.H;
        float4 f0 = make_float4(0.f, 0.f, 0.f, 0.f), f1 = f0;
        if constexpr (ROPE) {
            const float4 *fr = reinterpret_cast<const float4 *>(p.freqs + tok * D + c * 8);
            f0 = fr[0];
            f1 = fr[1];
        }
        float wq[8], wk[8];
        if constexpr (NORM) {
            unpack8(*reinterpret_cast<const uint4 *>(p.wq + c * 8), wq);
            if constexpr (HAS_K) unpack8(*reinterpret_cast<const uint4 *>(p.wk + c * 8), wk);
        }
        const uint16_t *qsrc = p.q + t * p.ldt + c * 8;
        const uint16_t *ksrc = HAS_K ? p.k + t * p.ldt + c * 8 : nullptr;
        const uint16_t *vsrc = HAS_V ? p.v + t * p.ldt + c * 8 : nullptr;
        uint16_t *qdst = p.oq + t * H * D + c * 8;
        const int64_t kv_row = (bb * (p.P + p.S) + p.P + tok) * H;
        for (int h0 = 0; h0 < H; h0 += RPI * UNROLL) {
            uint4 qv[UNROLL], kv[UNROLL], vv[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const int h = h0 + u * RPI + g;
                if (h < H) {  // uniform over the LPR lanes of a row
                    qv[u] = ld_nt(qsrc + h * D);
                    if constexpr (HAS_K) kv[u] = ld_nt(ksrc + h * D);
                    if constexpr (HAS_V) vv[u] = ld_nt(vsrc + h * D);
                }
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const int h = h0 + u * RPI + g;
                if (h < H) {
                    st_nt(qdst + h * D, norm_rope_chunk<LPR, NORM, ROPE>(qv[u], wq, p.epsq, f0, f1));
                    if constexpr (HAS_K)
                        st_nt(p.ok + (kv_row + h) * D + c * 8,
                              norm_rope_chunk<LPR, NORM, ROPE>(kv[u], wk, p.epsk, f0, f1));
                    if constexpr (HAS_V) st_nt(p.ov + (kv_row + h) * D + c * 8, vv[u]);
                }
            }
        }
    } else if constexpr (HAS_V) {
        // Prefix copy: B * P * H rows of D, RPI rows per wave instruction.
        const int64_t gi = ((int64_t)blockIdx.x - p.main_blocks) * 256 + threadIdx.x;
        const int64_t row = gi / LPR;
        const int64_t PH = p.P * p.H;
        const int64_t B = p.rows / (p.S * p.H);
        if (row >= B * PH) return;
        const int64_t bb = row / PH, within = row - bb * PH;
        const int64_t dst = (bb * (p.P + p.S) * p.H + within) * D + c * 8;
        *reinterpret_cast<uint4 *>(p.ok + dst) = *reinterpret_cast<const uint4 *>(p.ck + row * D + c * 8);
        *reinterpret_cast<uint4 *>(p.ov + dst) = *reinterpret_cast<const uint4 *>(p.cv + row * D + c * 8);
    }
}

template <bool NORM, bool ROPE, bool HAS_K, bool HAS_V>
static int launch_norm_rope(NormRopeArgs a, int64_t D, int64_t B, hipStream_t st) {
    const int64_t tokens = a.rows / a.H;   // one wave per token, 4 waves per workgroup
    a.main_blocks = (tokens + 3) / 4;
    const int64_t prefix_blocks = (HAS_V && a.P > 0) ? (B * a.P * a.H * (D / 8) + 255) / 256 : 0;
    const int64_t blocks = a.main_blocks + prefix_blocks;
    if (blocks >= (1ll << 31)) return fail(QIM_ERR_SHAPE, "norm/rope: too large");
    dim3 grid((unsigned)blocks), block(256);
    switch (D) {
        case 64: hipLaunchKernelGGL((k_norm_rope<64, NORM, ROPE, HAS_K, HAS_V>), grid, block, 0, st, a); break;
        case 128: hipLaunchKernelGGL((k_norm_rope<128, NORM, ROPE, HAS_K, HAS_V>), grid, block, 0, st, a); break;
        case 256: hipLaunchKernelGGL((k_norm_rope<256, NORM, ROPE, HAS_K, HAS_V>), grid, block, 0, st, a); break;
        default: return fail(QIM_ERR_SHAPE, "norm/rope: head dim %lld not in {64, 128, 256}", (long long)D);
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
                (const uint16_t *)res, (uint16_t *)out, nullptr, nullptr, rows, rows, (int)D, seq, eps, flags};
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
                (int)D, seq, eps, flags};
    rc = launch_adaln<true>(a, as_stream(stream));
    return rc ? rc : check_launch("qim_adaln_quantize");
}

extern "C" int qim_rms_norm(const void *x, const void *w, void *out, int64_t rows, int64_t D, float eps,
                            void *stream) {
    QIM_REQUIRE(x && w && out, QIM_ERR_ARG, "qim_rms_norm: null pointer");
    QIM_REQUIRE(rows > 0, QIM_ERR_SHAPE, "qim_rms_norm: empty input");
    QIM_REQUIRE(aligned16(x) && aligned16(w) && aligned16(out), QIM_ERR_LAYOUT,
                "qim_rms_norm: operands must be 16-byte aligned");
    // No table and no per-token state: view the rows as tokens of `heads` rows so
    // that every lane group of the one-wave-per-token kernel has work.
    const int64_t rpi = D > 0 ? 512 / (D > 512 ? 512 : D) : 1;  // 64 lanes x 8 values / D
    const int64_t heads = (rpi > 0 && rows % rpi == 0) ? rpi : 1;
    NormRopeArgs a{(const uint16_t *)x, nullptr, nullptr, nullptr, nullptr, (const uint16_t *)w, nullptr,
                   nullptr, (uint16_t *)out, nullptr, nullptr, rows, rows / heads, 0, heads, heads * D, eps, eps, 0};
    int rc = launch_norm_rope<true, false, false, false>(a, D, 1, as_stream(stream));
    return rc ? rc : check_launch("qim_rms_norm");
}

extern "C" int qim_rope_qk(const void *q, const void *k, const void *freqs, void *oq, void *ok, int64_t B,
                           int64_t S, int64_t H, int64_t D, void *stream) {
    QIM_REQUIRE(q && k && freqs && oq && ok, QIM_ERR_ARG, "qim_rope_qk: null pointer");
    QIM_REQUIRE(B > 0 && S > 0 && H > 0, QIM_ERR_SHAPE, "qim_rope_qk: empty input");
    QIM_REQUIRE(aligned16(q) && aligned16(k) && aligned16(freqs) && aligned16(oq) && aligned16(ok),
                QIM_ERR_LAYOUT, "qim_rope_qk: operands must be 16-byte aligned");
    NormRopeArgs a{(const uint16_t *)q, (const uint16_t *)k, nullptr, nullptr, nullptr, nullptr, nullptr,
                   (const float *)freqs, (uint16_t *)oq, (uint16_t *)ok, nullptr, B * S * H, S, 0, H, H * D, 0.f, 0.f, 0};
    int rc = launch_norm_rope<false, true, true, false>(a, D, B, as_stream(stream));
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
                   (uint16_t *)oq, (uint16_t *)ok, (uint16_t *)ov, B * S * H, S, P, H, ldt, epsq, epsk, 0};
    int rc = v ? launch_norm_rope<true, true, true, true>(a, D, B, as_stream(stream))
               : launch_norm_rope<true, true, true, false>(a, D, B, as_stream(stream));
    return rc ? rc : check_launch("qim_qk_norm_rope_pack");
}
