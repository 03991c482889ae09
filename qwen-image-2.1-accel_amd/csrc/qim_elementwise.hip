// Bandwidth-bound elementwise kernels: gated residual and SwiGLU.
//
// One lane handles one 16-byte vector (8 bf16) per operand: coalesced
// dwordx4 loads and stores, one read of every input byte and one write of
// every output byte.  Row and batch indices come from 32-bit divides done
// once per lane.
#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

// residual(h, x, gate): out = bf16(h + bf16(gate * x)), gate broadcast over
// each batch's rows (reference kernels/elementwise.py:10-23).
__global__ __launch_bounds__(256) void k_gated_residual(const uint16_t *__restrict__ h,
                                                         const uint16_t *__restrict__ x,
                                                         const uint16_t *__restrict__ gate,
                                                         uint16_t *__restrict__ out, uint32_t nvec,
                                                         uint32_t d8, uint32_t batch_vec) {
    const uint32_t v = blockIdx.x * 256u + threadIdx.x;
    if (v >= nvec) return;
    const uint32_t b = v / batch_vec, c = v % d8;
    const uint4 hv = ld_nt(reinterpret_cast<const uint4 *>(h) + v);
    const uint4 xv = ld_nt(reinterpret_cast<const uint4 *>(x) + v);
    const uint4 gv = reinterpret_cast<const uint4 *>(gate)[b * d8 + c];
    float hf[8], xf[8], gf[8], o[8];
    unpack8(hv, hf);
    unpack8(xv, xf);
    unpack8(gv, gf);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = hf[i] + rbf(gf[i] * xf[i]);
    st_nt(reinterpret_cast<uint4 *>(out) + v, pack8(o));
}

// swiglu(g, v) over strided rows (reference kernels/bf16.py:12-24).
__global__ __launch_bounds__(256) void k_swiglu(const uint16_t *__restrict__ g, int64_t ldg,
                                                 const uint16_t *__restrict__ v, int64_t ldv,
                                                 uint16_t *__restrict__ out, int64_t ldo, uint32_t f8) {
    const uint32_t c = blockIdx.x * 256u + threadIdx.x;
    if (c >= f8) return;
    const int64_t row = blockIdx.y;
    const uint4 gv = ld_nt(g + row * ldg + c * 8);
    const uint4 vv = ld_nt(v + row * ldv + c * 8);
    float gf[8], vf[8], o[8];
    unpack8(gv, gf);
    unpack8(vv, vf);
    silu_bf16_n<8>(gf, o);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= vf[i];
    st_nt(out + row * ldo + c * 8, pack8(o));
}

// The per-step modulation terms (reference optimizations/fusion.py:48-53:
// 1 + s and tanh(g) of the modulation chunks, as bf16 tensors): rows of D
// values, row r = g P + i (term i of group g) copied (kind 0), mapped to
// bf16(1 + x) (kind 1) or to bf16(tanh(x)) (kind 2: tanh in float64, rounded
// to fp32 and then to bf16); kind = (kinds >> 2 i) & 3.  Written term-major,
// to row i G + g of out (G groups), so that each term is one contiguous block.
// One value per lane: the launch is a few thousand values, and its time is
// one lane's float64 tanh.
__global__ __launch_bounds__(256) void k_modulation_values(const uint16_t *__restrict__ mod,
                                                            uint16_t *__restrict__ out, uint32_t n,
                                                            uint32_t d, uint32_t kinds, uint32_t period,
                                                            uint32_t groups) {
    const uint32_t v = blockIdx.x * 256u + threadIdx.x;
    if (v >= n) return;
    const uint32_t r = v / d, c = v - r * d, grp = r / period, term = r - grp * period;
    const uint32_t kind = (kinds >> (2u * term)) & 3u;
    uint16_t u = mod[v];
    if (kind != 0) {
        const float f = bf16_to_f32(u);
        u = (uint16_t)pack_bf16x2(kind == 1 ? f + 1.0f : (float)tanh((double)f), 0.0f);
    }
    out[(term * groups + grp) * d + c] = u;
}

}  // namespace qim

using namespace qim;

extern "C" int qim_modulation_values(const void *mod, int64_t rows, int64_t D, uint32_t kinds, int period,
                                     void *out, void *stream) {
    QIM_REQUIRE(mod && out, QIM_ERR_ARG, "qim_modulation_values: null pointer");
    QIM_REQUIRE(rows > 0 && D > 0, QIM_ERR_SHAPE, "qim_modulation_values: empty input");
    QIM_REQUIRE(D % 8 == 0, QIM_ERR_SHAPE, "qim_modulation_values: D=%lld is not a multiple of 8", (long long)D);
    QIM_REQUIRE(period >= 1 && period <= 16, QIM_ERR_ARG, "qim_modulation_values: period %d not in [1, 16]",
                period);
    for (int r = 0; r < period; ++r)
        QIM_REQUIRE(((kinds >> (2 * r)) & 3u) != 3u, QIM_ERR_ARG, "qim_modulation_values: kind 3 for row %d", r);
    QIM_REQUIRE(rows % period == 0, QIM_ERR_SHAPE, "qim_modulation_values: rows=%lld not a multiple of %d",
                (long long)rows, period);
    QIM_REQUIRE(rows * D < (1ll << 31), QIM_ERR_SHAPE, "qim_modulation_values: too large");
    QIM_REQUIRE(aligned16(mod) && aligned16(out), QIM_ERR_LAYOUT,
                "qim_modulation_values: operands must be 16-byte aligned");
    const uint32_t n = (uint32_t)(rows * D);
    launch(k_modulation_values, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), (const uint16_t *)mod,
           (uint16_t *)out, n, (uint32_t)D, kinds, (uint32_t)period, (uint32_t)(rows / period));
    return check_launch("qim_modulation_values");
}

extern "C" int qim_gated_residual(const void *h, const void *x, const void *gate, void *out, int64_t rows,
                                  int64_t D, int64_t seq, void *stream) {
    QIM_REQUIRE(h && x && gate && out, QIM_ERR_ARG, "qim_gated_residual: null pointer");
    QIM_REQUIRE(rows > 0 && D > 0 && seq > 0, QIM_ERR_SHAPE, "qim_gated_residual: empty input");
    QIM_REQUIRE(D % 8 == 0, QIM_ERR_SHAPE, "qim_gated_residual: D=%lld is not a multiple of 8", (long long)D);
    QIM_REQUIRE(rows * D / 8 < (1ll << 31) && seq * D / 8 < (1ll << 31), QIM_ERR_SHAPE,
                "qim_gated_residual: too large");
    QIM_REQUIRE(aligned16(h) && aligned16(x) && aligned16(gate) && aligned16(out), QIM_ERR_LAYOUT,
                "qim_gated_residual: operands must be 16-byte aligned");
    const uint32_t nvec = (uint32_t)(rows * D / 8);
    launch(k_gated_residual, dim3((nvec + 255) / 256), dim3(256), 0, as_stream(stream),
                       (const uint16_t *)h, (const uint16_t *)x, (const uint16_t *)gate, (uint16_t *)out, nvec,
                       (uint32_t)(D / 8), (uint32_t)(seq * D / 8));
    return check_launch("qim_gated_residual");
}

extern "C" int qim_swiglu(const void *g, int64_t ldg, const void *v, int64_t ldv, void *out, int64_t ldo,
                          int64_t M, int64_t F, void *stream) {
    QIM_REQUIRE(g && v && out, QIM_ERR_ARG, "qim_swiglu: null pointer");
    QIM_REQUIRE(M > 0 && F > 0, QIM_ERR_SHAPE, "qim_swiglu: empty input");
    QIM_REQUIRE(F % 8 == 0, QIM_ERR_SHAPE, "qim_swiglu: F=%lld is not a multiple of 8", (long long)F);
    QIM_REQUIRE(M < 65536ll * 65536ll && M <= 0x7fffffffll, QIM_ERR_SHAPE, "qim_swiglu: too many rows");
    QIM_REQUIRE(ldg >= F && ldv >= F && ldo >= F && ldg % 8 == 0 && ldv % 8 == 0 && ldo % 8 == 0 &&
                    aligned16(g) && aligned16(v) && aligned16(out),
                QIM_ERR_LAYOUT, "qim_swiglu: operands must be 16-byte aligned with strides %% 8 == 0");
    const uint32_t f8 = (uint32_t)(F / 8);
    // grid.y is limited to 65535: fold extra rows into repeated launches.
    for (int64_t r0 = 0; r0 < M; r0 += 65535) {
        const int64_t n = M - r0 < 65535 ? M - r0 : 65535;
        launch(k_swiglu, dim3((f8 + 255) / 256, (unsigned)n), dim3(256), 0, as_stream(stream),
                           (const uint16_t *)g + r0 * ldg, ldg, (const uint16_t *)v + r0 * ldv, ldv,
                           (uint16_t *)out + r0 * ldo, ldo, f8);
        int rc = check_launch("qim_swiglu");
        if (rc) return rc;
    }
    return QIM_OK;
}
