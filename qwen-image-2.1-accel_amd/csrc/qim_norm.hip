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

// One modulated LayerNorm row per wave (reference chain, eager rounding
// points: t0 = bf16(LN x), t1 = scale or bf16(1 + scale), t2 = bf16(t1 t0),
// t3 = bf16(t2 + shift), t4 = bf16(gate t3), out = bf16(res + t4);
// kernels/layernorm.py:49-55, kernels/epilogue.py:127-133).
template <int NV, bool QUANT>
__global__ __launch_bounds__(256) void k_adaln(AdaLNArgs p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows_pad) return;
    const int nvec = p.D >> 3;
    const bool live = row < p.rows;
    const int64_t b = live ? row / p.seq : 0;
    const uint4 *xr = reinterpret_cast<const uint4 *>(p.x + row * p.D);
    const uint4 *rr = p.res ? reinterpret_cast<const uint4 *>(p.res + row * p.D) : nullptr;

    uint4 xv[NV], rv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = lane + 64 * i;
        const bool ok = live && j < nvec;
        xv[i] = ok ? xr[j] : make_uint4(0, 0, 0, 0);
        rv[i] = (ok && rr) ? rr[j] : make_uint4(0, 0, 0, 0);
    }
    // Two-pass statistics in fp32.
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float f[8];
        unpack8(xv[i], f);
#pragma unroll
        for (int t = 0; t < 8; ++t) s += f[t];
    }
    const float mean = group_sum<64>(s) / (float)p.D;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (lane + 64 * i < nvec) {
            float f[8];
            unpack8(xv[i], f);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float d = f[t] - mean;
                ss += d * d;
            }
        }
    }
    const float var = group_sum<64>(ss) / (float)p.D;
    const float rstd = 1.0f / sqrtf(var + p.eps);

    const uint4 *sc = reinterpret_cast<const uint4 *>(p.scale + b * p.D);
    const uint4 *sh = p.shift ? reinterpret_cast<const uint4 *>(p.shift + b * p.D) : nullptr;
    const uint4 *ga = p.gate ? reinterpret_cast<const uint4 *>(p.gate + b * p.D) : nullptr;
    const bool add_one = (p.flags & QIM_ADALN_ADD_ONE) != 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = lane + 64 * i;
        if (j >= nvec) continue;  // uniform for all lanes of a 16-lane group when D % 128 == 0
        float o[8];
        if (live) {
            float f[8], sf[8], hf[8], gf[8], rf[8];
            unpack8(xv[i], f);
            unpack8(sc[j], sf);
            if (sh) unpack8(sh[j], hf);
            if (ga) unpack8(ga[j], gf);
            if (rr) unpack8(rv[i], rf);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float t0 = rbf((f[t] - mean) * rstd);
                const float t1 = add_one ? rbf(1.0f + sf[t]) : sf[t];
                float v = rbf(t1 * t0);
                if (sh) v = rbf(v + hf[t]);
                if (ga) v = rbf(gf[t] * v);
                if (rr) v = rbf(rf[t] + v);
                o[t] = v;
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t] = 0.0f;
        }
        if constexpr (!QUANT) {
            reinterpret_cast<uint4 *>(p.out + row * p.D)[j] = pack8(o);
        } else {
            // A 32-element block is 4 adjacent lanes; 4 adjacent blocks (16
            // lanes) own one dword of the swizzled scale array.
            int e;
            uint32_t m = group_umax<4>(absmax_bits8(o));
            e = mx_exponent(__uint_as_float(m));
            const float inv = mx_inverse(e);
            uint2 c;
            c.x = cvt_e4m3x4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
            c.y = cvt_e4m3x4(o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv);
            reinterpret_cast<uint2 *>(p.q + row * p.D)[j] = c;
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
    const int nv = (a.D / 8 + 63) / 64;
    dim3 grid((unsigned)((a.rows_pad + 3) / 4)), block(256);
#define QIM_ADALN_CASE(N)                                                         \
    if (nv <= N) {                                                                \
        hipLaunchKernelGGL((k_adaln<N, QUANT>), grid, block, 0, st, a);           \
        return QIM_OK;                                                            \
    }
    QIM_ADALN_CASE(2)
    QIM_ADALN_CASE(4)
    QIM_ADALN_CASE(6)
    QIM_ADALN_CASE(8)
    QIM_ADALN_CASE(12)
    QIM_ADALN_CASE(16)
#undef QIM_ADALN_CASE
    return fail(QIM_ERR_SHAPE, "adaln: D=%d exceeds 8192", a.D);
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
// row; LPR lanes share the row.
template <int LPR, bool NORM, bool ROPE>
__device__ __forceinline__ uint4 norm_rope_chunk(const uint4 &xv, const uint4 &wv, float eps, const float4 &f0,
                                                 const float4 &f1) {
    float x[8];
    unpack8(xv, x);
    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) ss += x[t] * x[t];
        ss = group_sum<LPR>(ss);
        const float r = 1.0f / sqrtf(ss / (float)(LPR * 8) + eps);
        float w[8];
        unpack8(wv, w);
#pragma unroll
        for (int t = 0; t < 8; ++t) x[t] = rbf(rbf(x[t] * r) * w[t]);
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
template <int D, bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void k_norm_rope(NormRopeArgs p) {
    constexpr int LPR = D / 8;
    if ((int64_t)blockIdx.x < p.main_blocks) {
        const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
        const int64_t row = g / LPR;
        const int c = (int)(g % LPR);
        if (row >= p.rows) return;  // whole LPR-lane groups leave together
        const int64_t SH = p.S * p.H;
        const int64_t bb = row / SH, within = row % SH;
        const int64_t tok = within / p.H;
        const int64_t dst = (bb * (p.P + p.S) * p.H + p.P * p.H + within) * D + c * 8;
        const int64_t src = (row / p.H) * p.ldt + (row % p.H) * D + c * 8;
        const int64_t dq = row * D + c * 8;
        float4 f0 = make_float4(0.f, 0.f, 0.f, 0.f), f1 = f0;
        if constexpr (ROPE) {
            const float4 *fr = reinterpret_cast<const float4 *>(p.freqs + tok * D + c * 8);
            f0 = fr[0];
            f1 = fr[1];
        }
        uint4 wqv = make_uint4(0, 0, 0, 0), wkv = wqv;
        if constexpr (NORM) {
            wqv = *reinterpret_cast<const uint4 *>(p.wq + c * 8);
            if (p.k) wkv = *reinterpret_cast<const uint4 *>(p.wk + c * 8);
        }
        const uint4 qv = *reinterpret_cast<const uint4 *>(p.q + src);
        uint4 kv = make_uint4(0, 0, 0, 0), vv = kv;
        if (p.k) kv = *reinterpret_cast<const uint4 *>(p.k + src);
        if (p.v) vv = *reinterpret_cast<const uint4 *>(p.v + src);
        *reinterpret_cast<uint4 *>(p.oq + dq) = norm_rope_chunk<LPR, NORM, ROPE>(qv, wqv, p.epsq, f0, f1);
        if (p.k) *reinterpret_cast<uint4 *>(p.ok + dst) = norm_rope_chunk<LPR, NORM, ROPE>(kv, wkv, p.epsk, f0, f1);
        if (p.v) *reinterpret_cast<uint4 *>(p.ov + dst) = vv;
    } else {
        // Prefix copy: B * P * H rows of D.
        const int64_t g = ((int64_t)blockIdx.x - p.main_blocks) * 256 + threadIdx.x;
        const int64_t row = g / LPR;
        const int c = (int)(g % LPR);
        const int64_t PH = p.P * p.H;
        const int64_t B = p.rows / (p.S * p.H);
        if (row >= B * PH) return;
        const int64_t bb = row / PH, within = row % PH;
        const int64_t dst = (bb * (p.P + p.S) * p.H + within) * D + c * 8;
        *reinterpret_cast<uint4 *>(p.ok + dst) = *reinterpret_cast<const uint4 *>(p.ck + row * D + c * 8);
        *reinterpret_cast<uint4 *>(p.ov + dst) = *reinterpret_cast<const uint4 *>(p.cv + row * D + c * 8);
    }
}

template <bool NORM, bool ROPE>
static int launch_norm_rope(NormRopeArgs a, int64_t D, int64_t B, hipStream_t st) {
    const int64_t lanes = a.rows * (D / 8);
    a.main_blocks = (lanes + 255) / 256;
    const int64_t prefix_blocks = (a.P > 0 && a.ov) ? (B * a.P * a.H * (D / 8) + 255) / 256 : 0;
    const int64_t blocks = a.main_blocks + prefix_blocks;
    if (blocks >= (1ll << 31)) return fail(QIM_ERR_SHAPE, "norm/rope: too large");
    dim3 grid((unsigned)blocks), block(256);
    switch (D) {
        case 64: hipLaunchKernelGGL((k_norm_rope<64, NORM, ROPE>), grid, block, 0, st, a); break;
        case 128: hipLaunchKernelGGL((k_norm_rope<128, NORM, ROPE>), grid, block, 0, st, a); break;
        case 256: hipLaunchKernelGGL((k_norm_rope<256, NORM, ROPE>), grid, block, 0, st, a); break;
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
    QIM_REQUIRE(D % 8 == 0 && D <= 8192, QIM_ERR_SHAPE, "%s: D=%lld unsupported (D %% 8 == 0, D <= 8192)", what,
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
    NormRopeArgs a{(const uint16_t *)x, nullptr, nullptr, nullptr, nullptr, (const uint16_t *)w, nullptr,
                   nullptr, (uint16_t *)out, nullptr, nullptr, rows, rows, 0, 1, D, eps, eps, 0};
    int rc = launch_norm_rope<true, false>(a, D, 1, as_stream(stream));
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
    int rc = launch_norm_rope<false, true>(a, D, B, as_stream(stream));
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
    int rc = launch_norm_rope<true, true>(a, D, B, as_stream(stream));
    return rc ? rc : check_launch("qim_qk_norm_rope_pack");
}
