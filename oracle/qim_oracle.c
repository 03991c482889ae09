/*
 * qim_oracle.c -- CPU restatement of the reference's per-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels in
 * libqim.so: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  No product code path calls it.
 *
 * Every function restates the eager PyTorch semantics that the reference's
 * Triton kernels reproduce bit-for-bit on its own GPU, with the same rounding
 * points (bf16 round after each eager op boundary).  Citations are to files
 * under the reference tree (src/qwen_image_accel/...), and "WHL!" names a file
 * inside the vendored diffusers wheel (read as text).
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).  Floating point
 * contraction is off so that every a*b+c below is two roundings unless it is
 * written as fmaf(), exactly like the reference's enable_fp_fusion=False.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 -- */

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quiet). */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* Value of the bf16 rounding of f, as fp32 (the eager ".to(bf16)" boundary). */
static inline float rbf(float f) { return bf16_to_f32(f32_to_bf16(f)); }

void oracle_f32_to_bf16(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int oracle_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* --------------------------------------------------------- E4M3 / E8M0 -- */

/* OCP E4M3 ("fn": no infinities, one NaN code per sign, max 448), round to
 * nearest even, restated from the OCP 8-bit floating point specification.
 * Finite inputs with |v| >= 464 (half way to the next binade step) and
 * non-finite inputs give the NaN code 0x7f, as torch's float8_e4m3fn cast does.
 * The quantizer never reaches that branch: it scales every block to |v| <= 448
 * (kernels/mxfp8.py:42-52). */
uint8_t oracle_e4m3_encode(float v) {
    uint32_t u = f2u(v);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    u &= 0x7fffffffu;
    if (u >= 0x7f800000u) return (uint8_t)(sign | 0x7fu);
    float a = u2f(u);
    if (a < 0.015625f) {                  /* below 2^-6: subnormal grid 2^-9 */
        float t = a * 512.0f;             /* exact: power-of-two scaling      */
        int m = (int)rintf(t);            /* current mode = nearest even      */
        return (uint8_t)(sign | m);       /* m == 8 is the smallest normal    */
    }
    u += 0x7ffffu + ((u >> 20) & 1u);     /* round 23-bit mantissa to 3 bits  */
    int e = (int)(u >> 23) - 127 + 7;
    int m = (int)((u >> 20) & 7u);
    int code = (e << 3) | m;
    if (e > 15 || code > 0x7e) return (uint8_t)(sign | 0x7fu);
    return (uint8_t)(sign | code);
}

float oracle_e4m3_decode(uint8_t c) {
    int e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return (c & 0x80) ? -v : v;
}

/* E8M0 exponent of one 32-element block: the smallest power of two 2^(e-127)
 * with amax / 2^(e-127) <= 448, read from the fp32 bits of amax
 * (kernels/mxfp8.py:42-48; tests/gpu/check_mxfp8.py:24-27). */
int oracle_mx_exponent(float amax) {
    uint32_t b = f2u(amax);
    int e = (int)((b >> 23) & 0xffu) - 8 + ((b & 0x7fffffu) > 0x600000u ? 1 : 0);
    if (amax == 0.0f) return 0;
    if (e < 0) e = 0;
    if (e > 254) e = 254;
    return e;
}

/* Byte offset of the scale of (row r, 32-element block kb) in the 128x4
 * swizzled layout: within a (128 rows x 4 blocks) tile the 512 bytes are
 * ordered (r % 32, (r % 128) / 32, kb % 4) (kernels/mxfp8.py:53-56). */
int64_t oracle_mx_scale_index(int64_t r, int64_t kb, int64_t K) {
    return ((r / 128) * (K / 128) + kb / 4) * 512 + (r % 32) * 16 + ((r % 128) / 32) * 4 + kb % 4;
}

/* Quantize one block of 32 fp32 values (each already a bf16 value). */
static inline uint8_t quant_block(const float *v, uint8_t *q) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) { float a = fabsf(v[i]); if (a > amax) amax = a; }
    int e = oracle_mx_exponent(amax);
    float inv = u2f((uint32_t)(254 - e) << 23);   /* 2^(127-e), exact */
    for (int i = 0; i < 32; ++i) q[i] = oracle_e4m3_encode(v[i] * inv);
    return (uint8_t)e;
}

/* quantize(x): bf16 (M,K) with row stride ldx -> E4M3 codes (Mp,K) and the
 * flat swizzled E8M0 bytes, Mp = ceil(M/128)*128; padding rows are code 0 and
 * exponent 0 (kernels/mxfp8.py:20-22, 30-67). */
void oracle_mx_quantize(const uint16_t *x, int64_t ldx, int64_t M, int64_t K,
                        uint8_t *q, uint8_t *s) {
    int64_t Mp = (M + 127) / 128 * 128;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < Mp; ++r) {
        float v[32];
        for (int64_t kb = 0; kb < K / 32; ++kb) {
            for (int i = 0; i < 32; ++i)
                v[i] = r < M ? bf16_to_f32(x[r * ldx + kb * 32 + i]) : 0.0f;
            s[oracle_mx_scale_index(r, kb, K)] = quant_block(v, q + r * K + kb * 32);
        }
    }
}

/* Quantize fp32 rows whose values are already bf16-rounded (used by the fused
 * producers: the unfused path stores bf16 and then quantizes). */
static void quant_row_f32(const float *row, int64_t r, int64_t K, uint8_t *q, uint8_t *s) {
    for (int64_t kb = 0; kb < K / 32; ++kb)
        s[oracle_mx_scale_index(r, kb, K)] = quant_block(row + kb * 32, q + r * K + kb * 32);
}

void oracle_mx_dequantize(const uint8_t *q, const uint8_t *s, int64_t M, int64_t K, float *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < M; ++r)
        for (int64_t k = 0; k < K; ++k) {
            int e = s[oracle_mx_scale_index(r, k / 32, K)];
            out[r * K + k] = oracle_e4m3_decode(q[r * K + k]) * ldexpf(1.0f, e - 127);
        }
}

/* ------------------------------------------------------------ LayerNorm -- */

enum { ORACLE_ADD_ONE = 1 };

/* Row statistics of LayerNorm (biased variance, no affine).  Computed in
 * float64 and rounded once to fp32, i.e. the exact value that any fp32
 * reduction order (the reference's Welford merge tree, kernels/layernorm.py:
 * 26-47) approximates. */
static void ln_stats(const uint16_t *x, int64_t D, float eps, float *mean_f, float *rstd_f) {
    double s = 0.0;
    for (int64_t i = 0; i < D; ++i) s += bf16_to_f32(x[i]);
    double mean = s / (double)D, v = 0.0;
    for (int64_t i = 0; i < D; ++i) { double d = bf16_to_f32(x[i]) - mean; v += d * d; }
    float var_f = (float)(v / (double)D);
    float t = var_f + eps;
    *mean_f = (float)mean;
    *rstd_f = (float)(1.0 / sqrt((double)t));
}

/* One modulated LayerNorm row, the eager chain of the reference's block
 * (WHL!transformer_qwenimage21.py:613-644 with the shift of the MMDiT form):
 *   t0 = bf16(LN(x)); t1 = add_one ? bf16(1 + scale) : scale;
 *   t2 = bf16(t1 * t0); t3 = shift ? bf16(t2 + shift) : t2;
 *   t4 = gate ? bf16(gate * t3) : t3; out = res ? bf16(res + t4) : t4.
 * layer_norm_scale (kernels/layernorm.py:49-55) is the case without shift,
 * gate and residual. */
static void adaln_row(const uint16_t *x, const uint16_t *scale, const uint16_t *shift,
                      const uint16_t *gate, const uint16_t *res, int64_t D, float eps,
                      int flags, float *out) {
    float mean, rstd;
    ln_stats(x, D, eps, &mean, &rstd);
    for (int64_t i = 0; i < D; ++i) {
        float t0 = rbf((bf16_to_f32(x[i]) - mean) * rstd);
        float t1 = bf16_to_f32(scale[i]);
        if (flags & ORACLE_ADD_ONE) t1 = rbf(1.0f + t1);
        float t = rbf(t1 * t0);
        if (shift) t = rbf(t + bf16_to_f32(shift[i]));
        if (gate) t = rbf(bf16_to_f32(gate[i]) * t);
        if (res) t = rbf(bf16_to_f32(res[i]) + t);
        out[i] = t;
    }
}

/* x (rows, D) with rows = B*seq; scale/shift/gate are per batch (B, D);
 * res and out are (rows, D).  Optional operands may be NULL. */
void oracle_adaln(const uint16_t *x, const uint16_t *scale, const uint16_t *shift,
                  const uint16_t *gate, const uint16_t *res, uint16_t *out,
                  int64_t rows, int64_t D, int64_t seq, float eps, int flags) {
    #pragma omp parallel
    {
        float *tmp = (float *)malloc((size_t)D * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            int64_t b = r / seq;
            adaln_row(x + r * D, scale + b * D, shift ? shift + b * D : NULL,
                      gate ? gate + b * D : NULL, res ? res + r * D : NULL, D, eps, flags, tmp);
            for (int64_t i = 0; i < D; ++i) out[r * D + i] = f32_to_bf16(tmp[i]);
        }
        free(tmp);
    }
}

/* layer_norm_scale_quantize == quantize(layer_norm_scale(x).reshape(-1, D))
 * byte-for-byte (kernels/epilogue.py:23-73; tests/gpu/check_mx_epilogue.py:
 * 34-36).  Rows past `rows` up to the 128-row padding quantize to zero. */
void oracle_adaln_quantize(const uint16_t *x, const uint16_t *scale, const uint16_t *shift,
                           const uint16_t *gate, const uint16_t *res, uint8_t *q, uint8_t *s,
                           int64_t rows, int64_t D, int64_t seq, float eps, int flags) {
    int64_t Mp = (rows + 127) / 128 * 128;
    #pragma omp parallel
    {
        float *tmp = (float *)malloc((size_t)D * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < Mp; ++r) {
            if (r < rows) {
                int64_t b = r / seq;
                adaln_row(x + r * D, scale + b * D, shift ? shift + b * D : NULL,
                          gate ? gate + b * D : NULL, res ? res + r * D : NULL, D, eps, flags, tmp);
            } else {
                for (int64_t i = 0; i < D; ++i) tmp[i] = 0.0f;
            }
            quant_row_f32(tmp, r, D, q, s);
        }
        free(tmp);
    }
}

/* ------------------------------------------------------- gated residual -- */

/* residual(h, x, gate): out = bf16(h + bf16(gate * x)), gate (B, D) broadcast
 * over each batch's seq rows (kernels/elementwise.py:10-34). */
void oracle_residual(const uint16_t *h, const uint16_t *x, const uint16_t *gate, uint16_t *out,
                     int64_t rows, int64_t D, int64_t seq) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *g = gate + (r / seq) * D;
        for (int64_t i = 0; i < D; ++i) {
            float p = rbf(bf16_to_f32(x[r * D + i]) * bf16_to_f32(g[i]));
            out[r * D + i] = f32_to_bf16(bf16_to_f32(h[r * D + i]) + p);
        }
    }
}

/* --------------------------------------------------------------- SwiGLU -- */

/* silu(g) * v with the reference's rounding: s = bf16(g / (1 + exp(-g))) with
 * an IEEE divide, then an fp32 multiply (no subnormal flush), rounded to bf16
 * (kernels/bf16.py:17-24; eager F.silu(g) * v, WHL!transformer_qwenimage21.py:
 * 212).  expf is the C library's. */
static inline float swiglu_f(float g, float v) {
    float s = rbf(g / (1.0f + expf(-g)));
    return rbf(s * v);
}

/* g, v: (M, F) with row strides ldg, ldv (the two halves of one (M, 2F)
 * tensor are strided views); out (M, F) with row stride ldo. */
void oracle_swiglu(const uint16_t *g, int64_t ldg, const uint16_t *v, int64_t ldv,
                   uint16_t *out, int64_t ldo, int64_t M, int64_t F) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < M; ++r)
        for (int64_t i = 0; i < F; ++i)
            out[r * ldo + i] = f32_to_bf16(swiglu_f(bf16_to_f32(g[r * ldg + i]),
                                                    bf16_to_f32(v[r * ldv + i])));
}

/* swiglu_quantize == quantize(swiglu(g, v)) byte-for-byte
 * (kernels/epilogue.py:95-136; tests/gpu/check_mx_epilogue.py:43-45). */
void oracle_swiglu_quantize(const uint16_t *g, int64_t ldg, const uint16_t *v, int64_t ldv,
                            uint8_t *q, uint8_t *s, int64_t M, int64_t F) {
    int64_t Mp = (M + 127) / 128 * 128;
    #pragma omp parallel
    {
        float *tmp = (float *)malloc((size_t)F * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < Mp; ++r) {
            for (int64_t i = 0; i < F; ++i)
                tmp[i] = r < M ? swiglu_f(bf16_to_f32(g[r * ldg + i]), bf16_to_f32(v[r * ldv + i]))
                               : 0.0f;
            quant_row_f32(tmp, r, F, q, s);
        }
        free(tmp);
    }
}

/* ----------------------------------------------------- RMSNorm and RoPE -- */

/* Diffusers RMSNorm on one row of D values (WHL!diffusers/models/
 * normalization.py:553-565; kernels/bf16.py:52-55):
 *   var = mean(x^2) (fp32); n = bf16(x * rsqrt(var + eps)); out = bf16(n * w). */
static void rms_row(const uint16_t *x, const uint16_t *w, int64_t D, float eps, float *out) {
    double ss = 0.0;
    for (int64_t i = 0; i < D; ++i) { double t = bf16_to_f32(x[i]); ss += t * t; }
    float var = (float)(ss / (double)D);
    float t = var + eps;
    float r = (float)(1.0 / sqrt((double)t));
    for (int64_t i = 0; i < D; ++i) {
        float n = rbf(bf16_to_f32(x[i]) * r);
        out[i] = rbf(n * bf16_to_f32(w[i]));
    }
}

void oracle_rms_norm(const uint16_t *x, const uint16_t *w, uint16_t *out,
                     int64_t rows, int64_t D, float eps) {
    #pragma omp parallel
    {
        float *tmp = (float *)malloc((size_t)D * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            rms_row(x + r * D, w, D, eps, tmp);
            for (int64_t i = 0; i < D; ++i) out[r * D + i] = f32_to_bf16(tmp[i]);
        }
        free(tmp);
    }
}

/* Complex RoPE on one (re, im) pair with the FMA order of the CUDA complex
 * multiply: re = fma(xr, c, -(xi*s)), im = fma(xi, c, xr*s)
 * (kernels/elementwise.py:53-56; eager apply_rotary_emb_qwen(use_real=False),
 * WHL!transformer_qwenimage21.py:128-133). */
static inline void rope_pair(float xr, float xi, float c, float s, float *orr, float *oi) {
    *orr = fmaf(xr, c, -(xi * s));
    *oi = fmaf(xi, c, xr * s);
}

/* rope_qk(q, k, freqs): q, k (B, S, H, D) bf16; freqs (S, D/2) complex64 as
 * interleaved fp32 (cos, sin); outputs bf16 (kernels/elementwise.py:37-69). */
void oracle_rope(const uint16_t *q, const uint16_t *k, const float *freqs,
                 uint16_t *oq, uint16_t *ok, int64_t B, int64_t S, int64_t H, int64_t D) {
    int64_t rows = B * S * H;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        int64_t tok = (r / H) % S;
        const float *f = freqs + tok * D;   /* D/2 complex = D floats */
        for (int64_t j = 0; j < D / 2; ++j) {
            float a, b;
            rope_pair(bf16_to_f32(q[r * D + 2 * j]), bf16_to_f32(q[r * D + 2 * j + 1]),
                      f[2 * j], f[2 * j + 1], &a, &b);
            oq[r * D + 2 * j] = f32_to_bf16(a); oq[r * D + 2 * j + 1] = f32_to_bf16(b);
            rope_pair(bf16_to_f32(k[r * D + 2 * j]), bf16_to_f32(k[r * D + 2 * j + 1]),
                      f[2 * j], f[2 * j + 1], &a, &b);
            ok[r * D + 2 * j] = f32_to_bf16(a); ok[r * D + 2 * j + 1] = f32_to_bf16(b);
        }
    }
}

/* prepare_attention_inputs: rope(RMSNorm_q(q)), cat[ck, rope(RMSNorm_k(k))],
 * cat[cv, v] along the sequence axis, with bf16 rounding after the norm, after
 * the weight and after RoPE (kernels/attention.py:48-89; tests/gpu/
 * check_attention_ops.py:25-31).  q, k, v: (B, S, H, D); ck, cv: (B, P, H, D)
 * (may be NULL when P == 0); oq: (B, S, H, D); ok, ov: (B, P+S, H, D). */
void oracle_norm_rope_pack(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                           const uint16_t *ck, const uint16_t *cv,
                           const uint16_t *wq, const uint16_t *wk, const float *freqs,
                           uint16_t *oq, uint16_t *ok, uint16_t *ov,
                           int64_t B, int64_t S, int64_t P, int64_t H, int64_t D,
                           float epsq, float epsk) {
    #pragma omp parallel
    {
        float *nq = (float *)malloc((size_t)D * sizeof(float));
        float *nk = (float *)malloc((size_t)D * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < B * S * H; ++r) {
            int64_t b = r / (S * H), tok = (r / H) % S, hh = r % H;
            const float *f = freqs + tok * D;
            rms_row(q + r * D, wq, D, epsq, nq);
            rms_row(k + r * D, wk, D, epsk, nk);
            int64_t dst = ((b * (P + S) + P + tok) * H + hh) * D;
            for (int64_t j = 0; j < D / 2; ++j) {
                float a, c;
                rope_pair(nq[2 * j], nq[2 * j + 1], f[2 * j], f[2 * j + 1], &a, &c);
                oq[r * D + 2 * j] = f32_to_bf16(a); oq[r * D + 2 * j + 1] = f32_to_bf16(c);
                rope_pair(nk[2 * j], nk[2 * j + 1], f[2 * j], f[2 * j + 1], &a, &c);
                ok[dst + 2 * j] = f32_to_bf16(a); ok[dst + 2 * j + 1] = f32_to_bf16(c);
            }
            memcpy(ov + dst, v + r * D, (size_t)D * sizeof(uint16_t));
        }
        free(nq); free(nk);
    }
    for (int64_t b = 0; b < B; ++b)
        for (int64_t p = 0; p < P; ++p) {
            size_t n = (size_t)(H * D);
            memcpy(ok + (b * (P + S) + p) * H * D, ck + (b * P + p) * H * D, n * sizeof(uint16_t));
            memcpy(ov + (b * (P + S) + p) * H * D, cv + (b * P + p) * H * D, n * sizeof(uint16_t));
        }
}

/* 3-axis RoPE table (WHL!transformer_qwenimage21.py:652-710): for each token
 * the positions (frame, h, w), each axis a of width dims[a] contributes
 * dims[a]/2 complex entries polar(1, pos * theta^(-2i/dims[a])), all in fp32.
 * out: (S, sum(dims)/2) complex64 as interleaved (cos, sin). */
void oracle_rope_freqs(const int64_t *pos, int64_t S, const int64_t *dims, float theta, float *out) {
    int64_t half = (dims[0] + dims[1] + dims[2]) / 2;
    for (int64_t t = 0; t < S; ++t) {
        int64_t col = 0;
        for (int a = 0; a < 3; ++a) {
            for (int64_t i = 0; i < dims[a] / 2; ++i, ++col) {
                float expo = (float)(2 * i) / (float)dims[a];
                float inv = 1.0f / powf(theta, expo);
                float ang = (float)pos[t * 3 + a] * inv;
                out[(t * half + col) * 2] = cosf(ang);
                out[(t * half + col) * 2 + 1] = sinf(ang);
            }
        }
    }
}

/* ----------------------------------------------------------------- GEMM -- */

/* MXFP8 GEMM core: Y[m, n] = sum_k deq(A)[m, k] * deq(B)[n, k] where A codes
 * are (Mp, K) row-major, B codes are (N, K) row-major (the reference keeps the
 * quantized weight as values.t(), a column-major (K, N) view of the same bytes,
 * optimizations/mxfp8.py:27-30), and both scale arrays are in the swizzled
 * layout over their own rows.  Each product of two dequantized values is exact
 * in float64; the sum is accumulated in float64 and rounded once to fp32.
 * `rows` (length nrows) selects which rows of A to compute (NULL: 0..nrows-1);
 * out is (nrows, N).  This is the dequantize-then-matmul the reference's
 * torch._scaled_mm call (optimizations/mxfp8.py:32-36) is checked against. */
void oracle_mx_gemm(const uint8_t *aq, const uint8_t *as, const uint8_t *bq, const uint8_t *bs,
                    const int64_t *rows, int64_t nrows, int64_t N, int64_t K, float *out) {
    float *bd = (float *)malloc((size_t)(N * K) * sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            bd[n * K + k] = oracle_e4m3_decode(bq[n * K + k]) *
                            ldexpf(1.0f, (int)bs[oracle_mx_scale_index(n, k / 32, K)] - 127);
    #pragma omp parallel
    {
        float *ad = (float *)malloc((size_t)K * sizeof(float));
        #pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < nrows; ++i) {
            int64_t m = rows ? rows[i] : i;
            for (int64_t k = 0; k < K; ++k)
                ad[k] = oracle_e4m3_decode(aq[m * K + k]) *
                        ldexpf(1.0f, (int)as[oracle_mx_scale_index(m, k / 32, K)] - 127);
            for (int64_t n = 0; n < N; ++n) {
                const float *b = bd + n * K;
                double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int64_t k = 0; k < K; k += 8)
                    for (int j = 0; j < 8; ++j) acc[j] += (double)ad[k + j] * (double)b[k + j];
                out[i * N + n] = (float)(((acc[0] + acc[1]) + (acc[2] + acc[3])) +
                                         ((acc[4] + acc[5]) + (acc[6] + acc[7])));
            }
        }
        free(ad);
    }
    free(bd);
}
