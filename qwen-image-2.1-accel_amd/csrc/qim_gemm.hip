// MXFP8 GEMM on CDNA4 scaled MFMA with fused epilogues.
//
//   Y[m, n] = sum_k (A[m, k] 2^(sa[m, k/32] - 127)) (B[n, k] 2^(sb[n, k/32] - 127))
//
// A: (Mp, K) E4M3 codes, B: (N, K) E4M3 codes (both K-contiguous), scales in
// the 128x4 swizzled layout.  fp32 accumulation in v_mfma_scale_f32_32x32x64_
// f8f6f4, which applies the E8M0 block scales inside the instruction.  Lane l
// of a 32x32x64 step holds row l%32 of A (column l%32 of B); with h = l/32 its
// bytes 0-15 are K [16h, 16h+16) and bytes 16-31 are K [32+16h, 32+16h+16), so
// bytes 0-15 of both half-waves form scale block 0 and bytes 16-31 block 1, and
// lane l supplies the E8M0 exponent of (row l%32, block h).  (Measured with
// qim_debug_mfma_probe: one-hot operands against per-lane exponents.)
//
// Workgroup tile 256 x 256, K step 128 bytes, 4 waves in a 2 x 2 grid, each
// wave a 128 x 128 block of 4 x 4 MFMA tiles (256 fp32 accumulators per lane).
// A, B and their scale chunks go global -> registers -> LDS with double
// buffering: the loads of stage s+1 are in flight while stage s computes.
// LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at chunk
// c ^ ((r >> 1) & 7), so 16 lanes reading 16 consecutive rows at one chunk
// touch 16 distinct (bank-half, chunk) slots.  The 512-byte scale chunk of a
// (128 rows x 128 K) tile is copied verbatim, and a lane reads the dword of
// its row, which holds the 4 exponents of the stage.
#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int TILE_BYTES = BM * BK;          // 32 KiB per operand per stage
constexpr int SCALE_BYTES = BM / 128 * 512;  // 1 KiB per operand per stage
constexpr int STAGE_BYTES = 2 * TILE_BYTES + 2 * SCALE_BYTES;
constexpr int LDS_BYTES = 2 * STAGE_BYTES;   // 132 KiB

struct GemmArgs {
    const uint8_t *aq, *as, *bq, *bs;
    int64_t M, Mp, N, K;
    const uint16_t *bias, *gate, *res;
    int64_t seq;
    void *out;
    int64_t ldo;
    uint8_t *out_scales;
    int tiles_n;
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Global -> register staging of one K stage.
struct Stage {
    uint4 a[8], b[8];
    uint4 sc;  // threads 0..63: A scale piece; 64..127: B scale piece
};

__device__ __forceinline__ void load_stage(const GemmArgs &p, int64_t m0, int64_t n0, int s, Stage &st) {
    const int tid = threadIdx.x;
    const int64_t kofs = (int64_t)s * BK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int ch = tid + 256 * i, row = ch >> 3, c = ch & 7;
        const int64_t ar = m0 + row;
        st.a[i] = ar < p.Mp ? *reinterpret_cast<const uint4 *>(p.aq + ar * p.K + kofs + c * 16) : make_uint4(0, 0, 0, 0);
        st.b[i] = *reinterpret_cast<const uint4 *>(p.bq + (n0 + row) * p.K + kofs + c * 16);
    }
    const int kt = p.K / BK;
    if (tid < 64) {
        const int g = tid >> 5, piece = tid & 31;  // 128-row group, 16-byte piece of its 512-byte chunk
        const int64_t grow = m0 / 128 + g;
        st.sc = grow * 128 < p.Mp
                    ? reinterpret_cast<const uint4 *>(p.as + (grow * kt + s) * 512)[piece]
                    : make_uint4(0, 0, 0, 0);
    } else if (tid < 128) {
        const int g = (tid - 64) >> 5, piece = tid & 31;
        const int64_t grow = n0 / 128 + g;
        st.sc = reinterpret_cast<const uint4 *>(p.bs + (grow * kt + s) * 512)[piece];
    }
}

__device__ __forceinline__ void store_stage(uint8_t *lds, const Stage &st) {
    const int tid = threadIdx.x;
    uint8_t *la = lds, *lb = lds + TILE_BYTES;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int ch = tid + 256 * i, row = ch >> 3, c = ch & 7;
        *reinterpret_cast<uint4 *>(la + swz(row, c)) = st.a[i];
        *reinterpret_cast<uint4 *>(lb + swz(row, c)) = st.b[i];
    }
    if (tid < 128) reinterpret_cast<uint4 *>(lds + 2 * TILE_BYTES)[tid] = st.sc;
}

// Offset of the scale dword of local row r (0..255) inside a 1 KiB scale tile.
__device__ __forceinline__ int scale_dword(int r) { return (r >> 7) * 512 + (r & 31) * 16 + ((r & 127) >> 5) * 4; }

template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_mx_gemm(GemmArgs p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int stages = (int)(p.K / BK);
    const int lr = lane & 31, kh = lane >> 5;

    f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

    Stage st;
    load_stage(p, m0, n0, 0, st);
    store_stage(lds, st);
    __syncthreads();

    for (int s = 0; s < stages; ++s) {
        uint8_t *cur = lds + (s & 1) * STAGE_BYTES;
        if (s + 1 < stages) load_stage(p, m0, n0, s + 1, st);
        const uint8_t *la = cur, *lb = cur + TILE_BYTES;
        const uint8_t *lsa = cur + 2 * TILE_BYTES, *lsb = lsa + SCALE_BYTES;
        uint32_t sa[4], sb[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sa[t] = *reinterpret_cast<const uint32_t *>(lsa + scale_dword(wm * 128 + t * 32 + lr));
            sb[t] = *reinterpret_cast<const uint32_t *>(lsb + scale_dword(wn * 128 + t * 32 + lr));
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int clo = kk * 4 + kh, chi = kk * 4 + 2 + kh;  // 16-byte chunks of the 128-byte row
            i32x8_t av[4], bv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int ra = wm * 128 + t * 32 + lr, rb = wn * 128 + t * 32 + lr;
                const uint4 a0 = *reinterpret_cast<const uint4 *>(la + swz(ra, clo));
                const uint4 a1 = *reinterpret_cast<const uint4 *>(la + swz(ra, chi));
                const uint4 b0 = *reinterpret_cast<const uint4 *>(lb + swz(rb, clo));
                const uint4 b1 = *reinterpret_cast<const uint4 *>(lb + swz(rb, chi));
                av[t] = i32x8_t{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                bv[t] = i32x8_t{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            }
            const int shift = (kk * 2 + kh) * 8;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ea = (int)((sa[i] >> shift) & 0xffu);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int eb = (int)((sb[j] >> shift) & 0xffu);
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[i], bv[j], acc[i][j], 0, 0, 0, ea,
                                                                                0, eb);
                }
            }
        }
        if (s + 1 < stages) store_stage(lds + ((s + 1) & 1) * STAGE_BYTES, st);
        __syncthreads();
    }

    // ------------------------------------------------------------ epilogue
    // Accumulator i of tile (ti, tj): row 8(i/4) + 4(l/32) + i%4, column l%32.
    const int64_t wrow0 = m0 + wm * 128, wcol0 = n0 + wn * 128;
    if constexpr (EPI == QIM_EPI_NONE || EPI == QIM_EPI_BIAS || EPI == QIM_EPI_GATED_RESIDUAL) {
        uint16_t *out = reinterpret_cast<uint16_t *>(p.out);
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) {
            const int64_t col = wcol0 + tj * 32 + lr;
            float bias = 0.0f;
            if constexpr (EPI == QIM_EPI_BIAS) bias = bf16_to_f32(p.bias[col]);
#pragma unroll
            for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int64_t row = wrow0 + ti * 32 + 8 * (i >> 2) + 4 * kh + (i & 3);
                    if (row >= p.M) continue;
                    float v = acc[ti][tj][i];
                    if constexpr (EPI == QIM_EPI_BIAS) v = v + bias;
                    if constexpr (EPI == QIM_EPI_GATED_RESIDUAL) {
                        const float g = bf16_to_f32(p.gate[(row / p.seq) * p.N + col]);
                        const float h = bf16_to_f32(p.res[row * p.N + col]);
                        v = h + rbf(g * rbf(v));
                    }
                    out[row * p.ldo + col] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
                }
            }
        }
    } else {
        // SwiGLU: tiles tj = 2u (gate) and 2u + 1 (up) hold the same output
        // columns (weight rows interleaved in groups of 32).
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t ocol = wcol0 / 2 + u * 32 + lr;
            const int64_t F = p.N / 2;
#pragma unroll
            for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int64_t row = wrow0 + ti * 32 + 8 * (i >> 2) + 4 * kh + (i & 3);
                    const float y = swiglu1(rbf(acc[ti][2 * u][i]), rbf(acc[ti][2 * u + 1][i]));
                    if constexpr (EPI == QIM_EPI_SWIGLU) {
                        if (row < p.M)
                            reinterpret_cast<uint16_t *>(p.out)[row * p.ldo + ocol] =
                                (uint16_t)(pack_bf16x2(y, 0.0f) & 0xffffu);
                    } else {
                        // One 32-element MX block = the 32 lanes of one half-wave.
                        const uint32_t m = group_umax<32>(__float_as_uint(y) & 0x7fffffffu);
                        const int e = mx_exponent(__uint_as_float(m));
                        const uint8_t code = (uint8_t)(cvt_e4m3x4(y * mx_inverse(e), 0.f, 0.f, 0.f) & 0xffu);
                        if (row < p.Mp) {
                            reinterpret_cast<uint8_t *>(p.out)[row * F + ocol] = code;
                            if (lr == 0) p.out_scales[mx_scale_offset(row, ocol >> 5, F)] = (uint8_t)e;
                        }
                    }
                }
            }
        }
    }
}

template <int EPI>
static int launch_gemm(const GemmArgs &a, int64_t tiles, hipStream_t st) {
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_gemm<EPI>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
        if (e != hipSuccess)
            return fail(QIM_ERR_LAUNCH, "qim_mxfp8_gemm: cannot reserve %d bytes of LDS: %s", LDS_BYTES,
                        hipGetErrorString(e));
        configured = true;
    }
    hipLaunchKernelGGL(k_mx_gemm<EPI>, dim3((unsigned)tiles), dim3(256), LDS_BYTES, st, a);
    return QIM_OK;
}

}  // namespace qim

using namespace qim;

extern "C" int qim_mxfp8_gemm(const void *aq, const void *as, const void *bq, const void *bs, int64_t M, int64_t N,
                              int64_t K, int epilogue, const void *bias, const void *gate, const void *res,
                              int64_t seq, void *out, int64_t ldo, void *out_scales, void *stream) {
    QIM_REQUIRE(aq && as && bq && bs && out, QIM_ERR_ARG, "qim_mxfp8_gemm: null pointer");
    QIM_REQUIRE(M > 0 && N > 0 && K > 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: empty problem");
    QIM_REQUIRE(K % BK == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: K=%lld is not a multiple of 128", (long long)K);
    QIM_REQUIRE(N % BN == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: N=%lld is not a multiple of 256", (long long)N);
    const int64_t Mp = (M + 127) / 128 * 128;
    const int64_t tiles_m = (Mp + BM - 1) / BM, tiles_n = N / BN;
    QIM_REQUIRE(tiles_m * tiles_n < (1ll << 31), QIM_ERR_SHAPE, "qim_mxfp8_gemm: too many tiles");
    QIM_REQUIRE(aligned16(aq) && aligned16(bq) && aligned16(as) && aligned16(bs), QIM_ERR_LAYOUT,
                "qim_mxfp8_gemm: operands must be 16-byte aligned");
    GemmArgs a{(const uint8_t *)aq, (const uint8_t *)as, (const uint8_t *)bq, (const uint8_t *)bs, M, Mp, N, K,
               (const uint16_t *)bias, (const uint16_t *)gate, (const uint16_t *)res, seq > 0 ? seq : M, out, ldo,
               (uint8_t *)out_scales, (int)tiles_n};
    const int64_t tiles = tiles_m * tiles_n;
    int rc;
    switch (epilogue) {
        case QIM_EPI_NONE:
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            rc = launch_gemm<QIM_EPI_NONE>(a, tiles, as_stream(stream));
            break;
        case QIM_EPI_BIAS:
            QIM_REQUIRE(bias, QIM_ERR_ARG, "qim_mxfp8_gemm: bias epilogue without bias");
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            rc = launch_gemm<QIM_EPI_BIAS>(a, tiles, as_stream(stream));
            break;
        case QIM_EPI_GATED_RESIDUAL:
            QIM_REQUIRE(gate && res, QIM_ERR_ARG, "qim_mxfp8_gemm: gated residual needs gate and res");
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            rc = launch_gemm<QIM_EPI_GATED_RESIDUAL>(a, tiles, as_stream(stream));
            break;
        case QIM_EPI_SWIGLU:
            QIM_REQUIRE(N % 512 == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: SwiGLU needs N %% 512 == 0");
            QIM_REQUIRE(ldo >= N / 2, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N/2", (long long)ldo);
            rc = launch_gemm<QIM_EPI_SWIGLU>(a, tiles, as_stream(stream));
            break;
        case QIM_EPI_SWIGLU_QUANT:
            QIM_REQUIRE(N % 512 == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: SwiGLU needs N %% 512 == 0");
            QIM_REQUIRE(out_scales, QIM_ERR_ARG, "qim_mxfp8_gemm: quantized output needs out_scales");
            rc = launch_gemm<QIM_EPI_SWIGLU_QUANT>(a, tiles, as_stream(stream));
            break;
        default:
            return fail(QIM_ERR_ARG, "qim_mxfp8_gemm: unknown epilogue %d", epilogue);
    }
    return rc ? rc : check_launch("qim_mxfp8_gemm");
}
