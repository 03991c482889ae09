/*
 * qim.h -- C ABI of libqim.so, the MI355X (gfx950) kernels of the per-block
 * transformer hot path of Qwen-Image-2.1-Accel.
 *
 * Every entry point takes raw device pointers, element counts and strides (in
 * elements), and a hipStream_t passed as void* (NULL = the null stream).  It
 * launches asynchronously on that stream and returns a qim_status; nothing is
 * allocated, freed or synchronised, and no device state survives a call.
 * bf16 tensors are uint16 bit patterns, E4M3 codes and E8M0 exponents are
 * bytes, and MXFP8 scales use the 128x4 swizzled layout of the reference: the
 * exponent of (row r, 32-element block kb) of a (rows, K) tensor lives at byte
 *   ((r / 128) * (K / 128) + kb / 4) * 512 + (r % 32) * 16 + ((r % 128) / 32) * 4 + kb % 4
 * (src/qwen_image_accel/kernels/mxfp8.py:53-56).  Quantized tensors are padded
 * to Mp = ceil(M / 128) * 128 rows; padding rows hold code 0 and exponent 0.
 *
 * Each declaration names the reference interface it replaces (file:line under
 * the reference tree src/qwen_image_accel/).
 */
#ifndef QIM_H
#define QIM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qim_status {
    QIM_OK = 0,
    QIM_ERR_ARG = 1,     /* null pointer or invalid argument value            */
    QIM_ERR_SHAPE = 2,   /* shape the kernels do not support                  */
    QIM_ERR_LAYOUT = 3,  /* stride or pointer alignment not supported         */
    QIM_ERR_LAUNCH = 4,  /* the HIP runtime rejected the launch               */
};

/* Flags of qim_adaln / qim_adaln_quantize. */
#define QIM_ADALN_ADD_ONE 1 /* use bf16(1 + scale) instead of scale */
#define QIM_ADALN_TILED 2   /* qim_adaln_quantize: codes in the tiled layout (below) */

/* Epilogues of qim_mxfp8_gemm. */
enum qim_epilogue {
    QIM_EPI_NONE = 0,           /* out = bf16(acc)                                     */
    QIM_EPI_BIAS = 1,           /* out = bf16(acc + bias[n])                           */
    QIM_EPI_GATED_RESIDUAL = 2, /* out = bf16(res + bf16(gate[b, n] * bf16(acc)))      */
    QIM_EPI_SWIGLU = 3,         /* out[m, j] = swiglu(bf16(acc_gate), bf16(acc_up))    */
    QIM_EPI_SWIGLU_QUANT = 4,   /* MXFP8 codes + scales of the QIM_EPI_SWIGLU output   */
    QIM_EPI_QK_NORM_ROPE = 5,   /* QKV projection with per-head RMSNorm + RoPE of Q, K
                                   (qim_mxfp8_gemm_qk_norm_rope only)                  */
};

/* Rows of the gate and of the up projection alternate in groups of this many
 * in a weight fed to the QIM_EPI_SWIGLU* epilogues: rows [2jG, 2jG+G) are gate
 * rows [jG, jG+G) and rows [2jG+G, 2jG+2G) are up rows [jG, jG+G). */
#define QIM_SWIGLU_GROUP 32

/* Message of the last failing call on this host thread ("" if none). */
const char *qim_last_error(void);

/* ABI version of this header. */
int qim_abi_version(void);

/* quantize(x) -- src/qwen_image_accel/kernels/mxfp8.py:59-67 (kernel :30-56).
 * x: bf16 (M, K), row stride ldx.  q: (Mp, K) E4M3 codes.  scales: Mp*K/32
 * E8M0 bytes, swizzled.  K % 128 == 0, ldx % 8 == 0. */
int qim_mx_quantize(const void *x, int64_t ldx, int64_t M, int64_t K,
                    void *q, void *scales, void *stream);

/* qim_mx_quantize writing the codes in the tiled layout (QIM_GEMM_A_TILED /
 * QIM_GEMM_B_TILED operands of qim_mxfp8_gemm_ex).  No reference counterpart. */
int qim_mx_quantize_tiled(const void *x, int64_t ldx, int64_t M, int64_t K,
                          void *q, void *scales, void *stream);

/* layer_norm_scale(x, scale, norm) -- src/qwen_image_accel/kernels/
 * layernorm.py:58-86 (kernel :17-55), extended with the optional MMDiT shift,
 * gate and residual: out = res + gate * (scale * LN(x) + shift) with a bf16
 * rounding after each op.  x, res, out: (rows, D), rows = B * seq;
 * scale, shift, gate: (B, D).  shift, gate, res may be NULL.  D % 8 == 0,
 * D <= 8192. */
int qim_adaln(const void *x, const void *scale, const void *shift, const void *gate,
              const void *res, void *out, int64_t rows, int64_t D, int64_t seq,
              float eps, int flags, void *stream);

/* layer_norm_scale_quantize(x, scale, norm) -- src/qwen_image_accel/kernels/
 * epilogue.py:76-92 (kernel :23-73): qim_adaln's output quantized to MXFP8
 * instead of stored.  q: (Mp, D), row-major or (QIM_ADALN_TILED) tiled;
 * scales: Mp*D/32.  D % 128 == 0. */
int qim_adaln_quantize(const void *x, const void *scale, const void *shift, const void *gate,
                       const void *res, void *q, void *scales, int64_t rows, int64_t D,
                       int64_t seq, float eps, int flags, void *stream);

/* residual(h, x, gate) -- src/qwen_image_accel/kernels/elementwise.py:26-34
 * (kernel :10-23): out = bf16(h + bf16(gate * x)).  h, x, out: (rows, D);
 * gate: (B, D), rows = B * seq.  D % 8 == 0. */
int qim_gated_residual(const void *h, const void *x, const void *gate, void *out,
                       int64_t rows, int64_t D, int64_t seq, void *stream);

/* The per-step modulation terms -- src/qwen_image_accel/optimizations/
 * fusion.py:48-53 (1 + s1, tanh(g1), 1 + s2, tanh(g2) of the modulation
 * chunks, computed there as eager torch ops): mod is (G, period, D) bf16 --
 * G groups of `period` (1..16) rows -- and row i of each group is copied
 * (kind 0), mapped to bf16(1 + x) (kind 1) or to bf16(tanh(x)) (kind 2: tanh
 * in float64, rounded to fp32, then to bf16), kind = (kinds >> (2 * i)) & 3.
 * out is (period, G, D): each term one contiguous block.  rows = G * period;
 * D % 8 == 0. */
int qim_modulation_values(const void *mod, int64_t rows, int64_t D, uint32_t kinds, int period,
                          void *out, void *stream);

/* swiglu(gate, value) -- src/qwen_image_accel/kernels/bf16.py:27-36 (kernel
 * :12-24): out = bf16(bf16(silu(g)) * v).  g, v, out: (M, F) with row strides
 * ldg, ldv, ldo (strided halves of one (M, 2F) tensor are accepted).
 * F % 8 == 0, strides % 8 == 0. */
int qim_swiglu(const void *g, int64_t ldg, const void *v, int64_t ldv, void *out, int64_t ldo,
               int64_t M, int64_t F, void *stream);

/* swiglu_quantize(gate, value) -- src/qwen_image_accel/kernels/epilogue.py:
 * 123-136 (kernel :95-120): swiglu quantized to MXFP8.  q: (Mp, F);
 * scales: Mp*F/32.  F % 128 == 0. */
int qim_swiglu_quantize(const void *g, int64_t ldg, const void *v, int64_t ldv,
                        void *q, void *scales, int64_t M, int64_t F, void *stream);

/* qim_swiglu_quantize writing the codes in the tiled layout.  No reference
 * counterpart. */
int qim_swiglu_quantize_tiled(const void *g, int64_t ldg, const void *v, int64_t ldv,
                              void *q, void *scales, int64_t M, int64_t F, void *stream);

/* rms_norm(x, weight, eps) -- src/qwen_image_accel/kernels/bf16.py:58-63
 * (kernel :46-55): out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w) per row of
 * D.  x, out: (rows, D); w: (D,).  D in {64, 128, 256}. */
int qim_rms_norm(const void *x, const void *w, void *out, int64_t rows, int64_t D,
                 float eps, void *stream);

/* rope_qk(q, k, freqs) -- src/qwen_image_accel/kernels/elementwise.py:63-69
 * (kernel :37-60).  q, k, oq, ok: (B, S, H, D) bf16; freqs: (S, D/2) complex64
 * as interleaved fp32 (cos, sin).  D in {64, 128, 256}. */
int qim_rope_qk(const void *q, const void *k, const void *freqs, void *oq, void *ok,
                int64_t B, int64_t S, int64_t H, int64_t D, void *stream);

/* prepare_attention_inputs(q, k, v, norm_q, norm_k, freqs, cached_k, cached_v)
 * -- src/qwen_image_accel/kernels/attention.py:92-159 (kernel :16-89):
 * oq = rope(RMSNorm_q(q)); ok = cat[ck, rope(RMSNorm_k(k))]; ov = cat[cv, v]
 * along the sequence axis.  q, k, v: (B, S, H, D) with `ldt` elements between
 * consecutive tokens (H*D when contiguous; 3*H*D for the Q/K/V column blocks
 * of a fused QKV projection); oq: (B, S, H, D) contiguous; ck, cv: (B, P, H, D)
 * (NULL when P == 0); ok, ov: (B, P+S, H, D); wq, wk: (D,) bf16.  v/ov may be
 * NULL to skip the V pack (the fused QK-RMSNorm + RoPE of the MMDiT block).
 * D in {64, 128, 256}. */
int qim_qk_norm_rope_pack(const void *q, const void *k, const void *v, const void *ck,
                          const void *cv, const void *wq, const void *wk, const void *freqs,
                          void *oq, void *ok, void *ov, int64_t B, int64_t S, int64_t P,
                          int64_t H, int64_t D, int64_t ldt, float epsq, float epsk,
                          void *stream);

/* MXFP8Linear.matmul(activation) -> torch._scaled_mm --
 * src/qwen_image_accel/optimizations/mxfp8.py:32-36, with fused epilogues.
 * aq: (Mp, K) E4M3 codes + as (swizzled over Mp rows); bq: (N, K) E4M3 codes of
 * the weight (the reference's column-major (K, N) weight_fp8 view is these same
 * bytes) + bs (swizzled over N rows).  fp32 accumulation.  Rows [0, M) are
 * written.  out: bf16 (M, Nout) with row stride ldo, Nout = N (N/2 for the
 * SWIGLU epilogues), or, for QIM_EPI_SWIGLU_QUANT, E4M3 codes (Mp, N/2) with
 * out_scales (Mp*N/64 bytes, swizzled).  bias: (N,) bf16.  gate: (B, N) bf16,
 * res: (M, N) bf16 (row stride N), B = ceil(M / seq).
 * K % 128 == 0, N % 128 == 0 (the reference converts a linear when K and N
 * are multiples of 128, optimizations/mxfp8.py:15-16), N % 512 == 0 for the
 * SWIGLU epilogues. */
int qim_mxfp8_gemm(const void *aq, const void *as, const void *bq, const void *bs,
                   int64_t M, int64_t N, int64_t K, int epilogue, const void *bias,
                   const void *gate, const void *res, int64_t seq, void *out, int64_t ldo,
                   void *out_scales, void *stream);

/* Tiled E4M3 code layout (no reference counterpart: the reference hands
 * row-major codes to torch._scaled_mm).  An (R, K) code matrix, R % 128 == 0,
 * is stored in super-blocks of 256 rows (the last holds R % 256 rows when that
 * is 128).  In a super-block of n rows starting at row r0, the 64-byte K-slab
 * s (codes [64s, 64s + 64) of each row) is n*64 contiguous bytes at
 * r0*K + s*n*64; row r's 64 bytes sit at (r - r0)*64 inside it, with its
 * 16-byte chunk c at chunk position c ^ (((r >> 1) ^ (r >> 2)) & 3).  Every
 * 16-row group of a slab is then the 1 KiB LDS image the GEMM loads with one
 * contiguous DMA instruction.  Scales keep the swizzled layout above. */
#define QIM_GEMM_A_TILED 1   /* aq is tiled over Mp rows                          */
#define QIM_GEMM_B_TILED 2   /* bq is tiled over N rows                           */
#define QIM_GEMM_OUT_TILED 4 /* QIM_EPI_SWIGLU_QUANT codes are written tiled      */
/* Output formats of QIM_EPI_NONE other than bf16 (torch._scaled_mm's out_dtype,
 * optimizations/mxfp8.py:34-35): out is fp32 or fp16 (M, N), row stride ldo
 * elements of that type. */
#define QIM_GEMM_OUT_F32 8
#define QIM_GEMM_OUT_F16 16

/* qim_mxfp8_gemm with operand layouts and output format (an OR of the flags
 * above; 0 = both operands row-major and a bf16 output, which is
 * qim_mxfp8_gemm itself). */
int qim_mxfp8_gemm_ex(const void *aq, const void *as, const void *bq, const void *bs,
                      int64_t M, int64_t N, int64_t K, int epilogue, int layouts,
                      const void *bias, const void *gate, const void *res, int64_t seq,
                      void *out, int64_t ldo, void *out_scales, void *stream);

/* qim_mxfp8_gemm_ex with a caller-provided workspace (no reference
 * counterpart; the same call as optimizations/mxfp8.py:32-36).  When the
 * tile grid's last partial round is a few quarter tiles (at most CUs / 2 of
 * them; e.g. 272 tiles of 256 x 256 on 256 CUs) and the epilogue is
 * QIM_EPI_NONE, QIM_EPI_BIAS or QIM_EPI_GATED_RESIDUAL, each of those quarter
 * tiles is split over K between several workgroups that write fp32 partial
 * sums to ws; a second launch on the same stream adds them in a fixed order
 * and runs the epilogue.  The result is the same function of the inputs
 * within the accumulation order (the partial sums of the tail are added in a
 * different order than one workgroup's MFMA chain).  ws: 16-byte aligned, at
 * least qim_mxfp8_gemm_ws_bytes(M, N, K, epilogue) bytes, not shared by calls
 * that may overlap; with ws = NULL or a smaller ws_bytes the call is
 * qim_mxfp8_gemm_ex. */
int qim_mxfp8_gemm_ws(const void *aq, const void *as, const void *bq, const void *bs,
                      int64_t M, int64_t N, int64_t K, int epilogue, int layouts,
                      const void *bias, const void *gate, const void *res, int64_t seq,
                      void *out, int64_t ldo, void *out_scales, void *ws, int64_t ws_bytes,
                      void *stream);

/* Workspace bytes qim_mxfp8_gemm_ws uses for this problem on the current
 * device; 0 when it splits nothing. */
int64_t qim_mxfp8_gemm_ws_bytes(int64_t M, int64_t N, int64_t K, int epilogue);

/* The fused QKV projection of the MMDiT block: qim_mxfp8_gemm_ex with
 * N = 3 * H * 128 whose output columns [0, H*128) (Q) and [H*128, 2*H*128) (K)
 * leave the GEMM as rope(RMSNorm(bf16(acc))) per 128-wide head, exactly what
 * qim_qk_norm_rope_pack (P = 0, no V) computes on the unfused output; columns
 * [2*H*128, 3*H*128) (V) are bf16(acc).  wq, wk: (128,) bf16; freqs:
 * (seq, 64) complex64 as interleaved fp32, row = output row % seq.  out: bf16
 * (M, N), row stride ldo.  H even.  Fuses kernels/attention.py:16-89 (P = 0)
 * into optimizations/mxfp8.py:32-36. */
int qim_mxfp8_gemm_qk_norm_rope(const void *aq, const void *as, const void *bq, const void *bs,
                                int64_t M, int64_t K, int64_t H, int layouts, const void *wq,
                                const void *wk, const void *freqs, int64_t seq, float epsq,
                                float epsk, void *out, int64_t ldo, void *stream);

/* qim_mxfp8_gemm_qk_norm_rope whose V columns leave as the attention core's
 * V^T tiles instead: written into the first B*H*(seq/64)*16 KiB of a
 * qim_attention workspace for (B = M / seq, S = T = seq, H), which
 * qim_attention / qim_attention_mxfp8 then read when passed v = NULL.  The V
 * columns of out are not written.  seq % 64 == 0, M % seq == 0.  No reference
 * counterpart: it removes the attention's V transpose pass. */
int qim_mxfp8_gemm_qk_norm_rope_vt(const void *aq, const void *as, const void *bq, const void *bs,
                                   int64_t M, int64_t K, int64_t H, int layouts, const void *wq,
                                   const void *wk, const void *freqs, int64_t seq, float epsq,
                                   float epsk, void *out, int64_t ldo, void *vt, void *stream);

/* Attention core, the block's softmax(Q K^T * scale) V per (batch, head) over
 * [prefix + target] keys (SDPA in the reference: optimizations/
 * quantized_decode.py:70-77).  q: (B, S, H, D), k, v: (B, T, H, D), o:
 * (B, S, H, D), bf16, with ldq / ldk / ldv / ldo elements between consecutive
 * tokens (views into a fused QKV output are fine).  D = 128, scale > 0.  fp32
 * scores, softmax and accumulation; P rounded to bf16 for the P V product.
 * workspace: at least qim_attention_workspace_bytes(B, S, T, H, D) bytes,
 * 16-byte aligned, passed with its size (V transposed in 64-key tiles, and
 * the partial results of work items split over key ranges to fill the last
 * round of workgroups; the split depends on the current device's CU count).
 * v = NULL (ldv ignored): the workspace already holds V^T, written by
 * qim_mxfp8_gemm_qk_norm_rope_vt; T % 64 == 0. */
int qim_attention(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                  void *o, int64_t ldo, void *workspace, int64_t workspace_bytes, int64_t B, int64_t S,
                  int64_t T, int64_t H, int64_t D, float scale, void *stream);
int64_t qim_attention_workspace_bytes(int64_t B, int64_t S, int64_t T, int64_t H, int64_t D);

/* qim_attention with its output quantized to MXFP8 in the same pass: exactly
 * the codes and scales qim_mx_quantize (tiled = 0) or qim_mx_quantize_tiled
 * (tiled = 1) would write for qim_attention's bf16 output viewed as a
 * (B*S, H*D) matrix, without that matrix: codes (Mp, H*D) E4M3, Mp =
 * B*S rounded up to 128 (padding rows zero), scales Mp*H*D/32 E8M0 bytes
 * in the swizzled layout; both 16-byte aligned.  The reference quantizes the
 * attention output for the MXFP8 out-projection in a separate pass
 * (optimizations/quantized_decode.py:81-96 with kernels/mxfp8.py:59-67); no
 * reference entry point fuses the two.  Workspace as for qim_attention. */
int qim_attention_mxfp8(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                        void *codes, void *scales, int tiled, void *workspace, int64_t workspace_bytes,
                        int64_t B, int64_t S, int64_t T, int64_t H, int64_t D, float scale, void *stream);

/* qim_attention without a workspace argument and without allocating: the
 * workspace is a device array inside the library of
 * QIM_ATTENTION_NOALLOC_MAX_BYTES, one per device, held from the first call
 * on a device until the process ends.  No reference counterpart: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  Arguments and output as qim_attention
 * with v required (no V^T from a QKV GEMM); a problem whose
 * qim_attention_workspace_bytes exceeds the maximum is rejected with
 * QIM_ERR_SHAPE before anything is launched (S = T = 4352 with 24 heads fits
 * for one batch).  Every call on a device shares its array: calls that
 * overlap on one device race.  The first call on each device resolves the
 * array's device address (hipGetSymbolAddress, which may make the runtime
 * load the library's code object and place the array on that device): make
 * that first call before any graph capture begins, so that a captured call
 * only launches kernels. */
#define QIM_ATTENTION_NOALLOC_MAX_BYTES (64ll << 20)
int qim_attention_noalloc(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                          void *o, int64_t ldo, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                          float scale, void *stream);

/* Test hooks: the device conversions every kernel uses, applied elementwise
 * (fp32 -> E4M3 code; fp32 -> bf16 bits), and one scaled MFMA
 * (32x32x64, E4M3 x E4M3) on a single tile: a (32, 64) codes, b (32, 64) codes
 * (row n of b is column n of the product), sa/sb (32, 2) E8M0 bytes,
 * out (32, 32) fp32 = sum_k a*2^(sa-127) b*2^(sb-127). */
int qim_debug_e4m3_encode(const float *x, void *codes, int64_t n, void *stream);
int qim_debug_bf16_round(const float *x, void *bits, int64_t n, void *stream);
/* bf16 x (n % 4 == 0, 16-byte aligned) -> E4M3 codes of x * 2^(127 - e), 0 <= e <= 254, through the
 * packed scaled conversion (v_cvt_scalef32_pk_fp8_bf16) the quantizers use. */
int qim_debug_e4m3_encode_scaled(const void *x, int e, void *codes, int64_t n, void *stream);
int qim_debug_mfma_tile(const void *a, const void *b, const void *sa, const void *sb,
                        float *out, void *stream);
/* Scale-routing probe of the scaled MFMA (shape 0: 32x32x64, 1: 16x16x128):
 * 4096 one-hot experiments, out: 4096 x 1024 (shape 0) or 4096 x 256 fp32. */
int qim_debug_mfma_probe(int shape, float *out, void *stream);
/* bf16(silu(g)) of n bf16 values with the rounding every SwiGLU kernel uses
 * (reference kernels/bf16.py:17-22: bf16(g / (1 + exp(-g)))). */
int qim_debug_silu(const void *g, void *out, int64_t n, void *stream);
/* The normalisations' reciprocal square root (fp32(1 / sqrt(double(var + eps))),
 * a fast path with an interval check and that expression as fallback) against
 * its definition for var = the fp32 values with bit patterns [first, first +
 * count): bad (2 uint32, the caller sets 0 and 0xffffffff) receives the number
 * of disagreements and the smallest disagreeing pattern. */
int qim_debug_rstd_sweep(uint32_t first, uint32_t count, float eps, void *bad, void *stream);
/* Streaming device copy of nbytes (a multiple of 16, 16-byte aligned): the
 * bandwidth reference of the benchmarks and the calibration kernel of the HBM
 * byte counters.  No reference counterpart. */
int qim_debug_copy(const void *src, void *dst, int64_t nbytes, void *stream);
/* Variants of that copy for the single-launch bandwidth ceiling:
 * vectors_per_lane (1, 2, 4, 8) 16-byte vectors per lane, loads before
 * stores; blocks_per_cu = 0: one-shot grid covering nbytes, else a
 * persistent grid of blocks_per_cu workgroups per CU striding over it. */
int qim_debug_copy_ex(const void *src, void *dst, int64_t nbytes, int vectors_per_lane, int blocks_per_cu,
                      void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QIM_H */
