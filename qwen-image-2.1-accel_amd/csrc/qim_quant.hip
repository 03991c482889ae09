// MXFP8 quantizers: quantize(x) and the fused swiglu_quantize(g, v).
//
// One workgroup quantizes one 128-row x 128-column tile, the unit of the
// reference's scale layout: its 512 E8M0 bytes form one contiguous chunk of
// the swizzled scale array, so they are staged in LDS and written with 32
// 16-byte stores.  Each wave owns 32 rows of the tile; 16 lanes cover one
// 128-column row (8 bf16 = one 16-byte load per lane), 4 rows per pass,
// 8 passes.  A 32-element block is 4 adjacent lanes, reduced with two DPP
// quad permutes.  All 8 loads of a lane are issued before any arithmetic.
// HBM traffic is the algorithmic minimum: every input byte read once, every
// code and scale byte written once.  Codes are written row-major or in the
// GEMM's tiled layout (mxt_offset); an 8-byte store stays contiguous in both.
#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

// Plain bf16 source: quantize(x) (reference kernels/mxfp8.py:30-56).
struct QuantSource {
    const uint16_t *x;
    int64_t ldx;
    __device__ __forceinline__ void load(bool live, int64_t row, int64_t col, uint4 &a, uint4 &b) const {
        a = live ? ld_nt(x + row * ldx + col) : make_uint4(0, 0, 0, 0);
        (void)b;
    }
    __device__ __forceinline__ void values(const uint4 &a, const uint4 &b, float *f) const {
        (void)b;
        unpack8(a, f);
    }
};

// SwiGLU source: swiglu_quantize(g, v) (reference kernels/epilogue.py:
// 95-120): the bf16 value of bf16(silu(g)) * v, exactly what the unfused
// path stores before quantizing.
struct SwigluSource {
    const uint16_t *g;
    int64_t ldg;
    const uint16_t *v;
    int64_t ldv;
    __device__ __forceinline__ void load(bool live, int64_t row, int64_t col, uint4 &a, uint4 &b) const {
        a = live ? ld_nt(g + row * ldg + col) : make_uint4(0, 0, 0, 0);
        b = live ? ld_nt(v + row * ldv + col) : make_uint4(0, 0, 0, 0);
    }
    __device__ __forceinline__ void values(const uint4 &a, const uint4 &b, float *f) const {
        float gg[8], vv[8], s[8];
        unpack8(a, gg);
        unpack8(b, vv);
        silu_bf16_n<8>(gg, s);
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = rbf(s[i] * vv[i]);
    }
};

template <class Source>
__global__ __launch_bounds__(256) void k_quant_tile(Source src, uint8_t *__restrict__ q,
                                                     uint8_t *__restrict__ scales, int64_t M,
                                                     int64_t K, int tiled) {
    __shared__ uint4 s_scale[32];  // the tile's 512 swizzled exponent bytes
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c16 = lane & 15;    // 8-column chunk of the 128-column tile row
    const int rsub = lane >> 4;   // row within a pass of 4 rows
    const int64_t row0 = (int64_t)blockIdx.x * 128;
    const int64_t col = (int64_t)blockIdx.y * 128 + c16 * 8;
    uint8_t *sb = reinterpret_cast<uint8_t *>(s_scale);

    uint4 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = wave * 32 + i * 4 + rsub;
        src.load(row0 + r < M, row0 + r, col, a[i], b[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = wave * 32 + i * 4 + rsub;  // r / 32 == wave
        float f[8];
        src.values(a[i], b[i], f);
        int e;
        uint2 c = quantize8(f, e);
        const int64_t Mp = (int64_t)gridDim.x * 128;
        st_nt(q + (tiled ? mxt_offset(row0 + r, col, Mp, K) : (row0 + r) * K + col), c);
        if ((c16 & 3) == 0) sb[(r & 31) * 16 + wave * 4 + (c16 >> 2)] = (uint8_t)e;
    }
    __syncthreads();
    if (tid < 32) {
        uint4 *dst = reinterpret_cast<uint4 *>(scales + ((int64_t)blockIdx.x * (K >> 7) + blockIdx.y) * 512);
        dst[tid] = s_scale[tid];
    }
}

static int launch_quant_checks(const char *what, int64_t M, int64_t K) {
    QIM_REQUIRE(M > 0 && K > 0, QIM_ERR_SHAPE, "%s: empty input (M=%lld, K=%lld)", what, (long long)M, (long long)K);
    QIM_REQUIRE(K % 128 == 0, QIM_ERR_SHAPE, "%s: K=%lld is not a multiple of 128", what, (long long)K);
    QIM_REQUIRE((M + 127) / 128 < (1ll << 31) && K / 128 < 65536, QIM_ERR_SHAPE, "%s: too large", what);
    return QIM_OK;
}

}  // namespace qim

using namespace qim;

static int mx_quantize(const void *x, int64_t ldx, int64_t M, int64_t K, void *q, void *scales, int tiled,
                       void *stream) {
    QIM_REQUIRE(x && q && scales, QIM_ERR_ARG, "qim_mx_quantize: null pointer");
    int rc = launch_quant_checks("qim_mx_quantize", M, K);
    if (rc) return rc;
    QIM_REQUIRE(ldx >= K && ldx % 8 == 0 && aligned16(x) && aligned16(q) && aligned16(scales), QIM_ERR_LAYOUT,
                "qim_mx_quantize: x must be 16-byte aligned with ldx %% 8 == 0 (ldx=%lld)", (long long)ldx);
    dim3 grid((unsigned)((M + 127) / 128), (unsigned)(K / 128));
    QuantSource src{(const uint16_t *)x, ldx};
    launch(k_quant_tile<QuantSource>, grid, dim3(256), 0, as_stream(stream), src, (uint8_t *)q,
                       (uint8_t *)scales, M, K, tiled);
    return check_launch("qim_mx_quantize");
}

static int swiglu_quantize(const void *g, int64_t ldg, const void *v, int64_t ldv, void *q, void *scales,
                           int64_t M, int64_t F, int tiled, void *stream) {
    QIM_REQUIRE(g && v && q && scales, QIM_ERR_ARG, "qim_swiglu_quantize: null pointer");
    int rc = launch_quant_checks("qim_swiglu_quantize", M, F);
    if (rc) return rc;
    QIM_REQUIRE(ldg >= F && ldv >= F && ldg % 8 == 0 && ldv % 8 == 0 && aligned16(g) && aligned16(v) &&
                    aligned16(q) && aligned16(scales),
                QIM_ERR_LAYOUT, "qim_swiglu_quantize: inputs must be 16-byte aligned with strides %% 8 == 0");
    dim3 grid((unsigned)((M + 127) / 128), (unsigned)(F / 128));
    SwigluSource src{(const uint16_t *)g, ldg, (const uint16_t *)v, ldv};
    launch(k_quant_tile<SwigluSource>, grid, dim3(256), 0, as_stream(stream), src, (uint8_t *)q,
                       (uint8_t *)scales, M, F, tiled);
    return check_launch("qim_swiglu_quantize");
}

extern "C" int qim_mx_quantize(const void *x, int64_t ldx, int64_t M, int64_t K, void *q, void *scales,
                               void *stream) {
    return mx_quantize(x, ldx, M, K, q, scales, 0, stream);
}

extern "C" int qim_mx_quantize_tiled(const void *x, int64_t ldx, int64_t M, int64_t K, void *q, void *scales,
                                     void *stream) {
    return mx_quantize(x, ldx, M, K, q, scales, 1, stream);
}

extern "C" int qim_swiglu_quantize(const void *g, int64_t ldg, const void *v, int64_t ldv, void *q,
                                   void *scales, int64_t M, int64_t F, void *stream) {
    return swiglu_quantize(g, ldg, v, ldv, q, scales, M, F, 0, stream);
}

extern "C" int qim_swiglu_quantize_tiled(const void *g, int64_t ldg, const void *v, int64_t ldv, void *q,
                                         void *scales, int64_t M, int64_t F, void *stream) {
    return swiglu_quantize(g, ldg, v, ldv, q, scales, M, F, 1, stream);
}
