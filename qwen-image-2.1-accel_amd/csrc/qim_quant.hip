// MXFP8 quantizers: quantize(x) and the fused swiglu_quantize(g, v).
//
// quantize(x) (k_quant_tile): the unit of work is a 128-row x 128-column tile, the unit of the
// reference's scale layout: its 512 E8M0 bytes form one contiguous chunk of
// the swizzled scale array, row r's 4 exponents at (r % 32) * 16 + (r / 32) * 4.
// A wave owns 32 rows of a tile: rows 8w .. 8w + 7 of each 32-row quarter
// (w = the wave's role), so its 32 exponent dwords are 8 whole 16-byte groups,
// one contiguous 128-byte store.  (Owning 32 consecutive rows made each wave
// write one dword of every 16 bytes of the chunk: 4 partial writes per 32-byte
// sector, 1.2 MB of extra HBM writes at config 4a.)  16 lanes cover one
// 128-column row (8 bf16 = one 16-byte load per lane), 4 rows per pass, 8
// passes, loads two passes at a time.  A 32-element block is 4 adjacent
// lanes, reduced with two DPP quad permutes; the codes come from the packed
// bf16 values through the scaled conversion (no unpacking, no multiply).
// Workgroups are one wave (a quarter tile; measured fastest at config 4a).
// HBM traffic is the algorithmic minimum: every input byte read once, every
// code and scale byte written once.  Codes are written row-major or in the
// GEMM's tiled layout (mxt_offset); an 8-byte store stays contiguous in both.
// swiglu_quantize (k_quant_rows): the same codes, exponents and layouts from
// one vector per lane and one 4-row group of a tile per wave (below).
#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

// Plain bf16 source: quantize(x) (reference kernels/mxfp8.py:30-56).
struct QuantSource {
    const uint16_t *x;
    int64_t ldx;
    // Loads of rows row + pass_row(i) (i = 0..7) at column col: pointer and
    // the two row steps set once.
    const uint16_t *px;
    int64_t s4, s32;
    __device__ __forceinline__ void start(int64_t row, int64_t col) {
        px = x + row * ldx + col;
        s4 = 4 * ldx;
        s32 = 32 * ldx;
    }
    __device__ __forceinline__ void load(bool live, int i, uint4 &a, uint4 &b) const {
        a = live ? ld_nt(px + (i >> 1) * s32 + (i & 1) * s4) : make_uint4(0, 0, 0, 0);
        (void)b;
    }
    // The 8 bf16 values as they are: converted packed, no unpacking.
    __device__ __forceinline__ uint2 quantize(const uint4 &a, const uint4 &b, int &e) const {
        (void)b;
        return quantize8_bf16(a, e);
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
    const uint16_t *pg, *pv;
    int64_t sg4, sg32, sv4, sv32;
    __device__ __forceinline__ void start(int64_t row, int64_t col) {
        pg = g + row * ldg + col;
        pv = v + row * ldv + col;
        sg4 = 4 * ldg;
        sg32 = 32 * ldg;
        sv4 = 4 * ldv;
        sv32 = 32 * ldv;
    }
    __device__ __forceinline__ void load(bool live, int i, uint4 &a, uint4 &b) const {
        a = live ? ld_nt(pg + (i >> 1) * sg32 + (i & 1) * sg4) : make_uint4(0, 0, 0, 0);
        b = live ? ld_nt(pv + (i >> 1) * sv32 + (i & 1) * sv4) : make_uint4(0, 0, 0, 0);
    }
    // One vector of each at row row0 + 32 j, column col (k_quant_rows;
    // row0 is wave-uniform, so its products stay scalar).
    __device__ __forceinline__ void load_at(int64_t row0, int j, int64_t col, bool live, uint4 &a, uint4 &b) const {
        const uint16_t *g0 = g + row0 * ldg, *v0 = v + row0 * ldv;
        a = live ? ld_nt(g0 + (int64_t)(32 * j) * ldg + col) : make_uint4(0, 0, 0, 0);
        b = live ? ld_nt(v0 + (int64_t)(32 * j) * ldv + col) : make_uint4(0, 0, 0, 0);
    }
    // The products are rounded to bf16 in pairs, packed, and quantized as
    // packed bf16 (quantize8_bf16: the codes and exponent of quantize8 on the
    // same values).
    __device__ __forceinline__ uint2 quantize(const uint4 &a, const uint4 &b, int &e) const {
        float gg[8], vv[8], s[8];
        unpack8(a, gg);
        unpack8(b, vv);
        silu_bf16_n<8>(gg, s);
        const uint4 p = make_uint4(pack_bf16x2(s[0] * vv[0], s[1] * vv[1]), pack_bf16x2(s[2] * vv[2], s[3] * vv[3]),
                                   pack_bf16x2(s[4] * vv[4], s[5] * vv[5]), pack_bf16x2(s[6] * vv[6], s[7] * vv[7]));
        return quantize8_bf16(p, e);
    }
};

// W waves per workgroup.  W = 4: one workgroup per 128 x 128 tile; W = 1:
// one per 32-row quarter of it (wave role = blockIdx.x % 4), so a launch has
// four times as many workgroups and the last round of the CUs is fuller.
// Row of pass i (0..7) relative to the lane's base row 8w + rsub: passes
// 2q and 2q + 1 cover rows 8w .. 8w + 7 of quarter q.
__device__ __forceinline__ int pass_row(int i) { return 32 * (i >> 1) + 4 * (i & 1); }

// W waves per workgroup.  W = 4: one workgroup per 128 x 128 tile; W = 1:
// one per quarter of its rows (wave role = blockIdx.x % 4), so a launch has
// four times as many workgroups and the last round of the CUs is fuller.
template <class Source, int W>
__global__ __launch_bounds__(64 * W) void k_quant_tile(Source src, uint8_t *__restrict__ q,
                                                        uint8_t *__restrict__ scales, int64_t M,
                                                        int64_t K, int tiled) {
    // Per wave: its 32 exponent dwords in the order of the scale chunk, row
    // j (0..7 of the 8w + j rows) of quarter q at dword j * 4 + q.
    __shared__ uint32_t s_scale[W][32];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = W == 1 ? (int)(blockIdx.x & 3) : tid >> 6;
    const int c16 = lane & 15;    // 8-column chunk of the 128-column tile row
    const int rsub = lane >> 4;   // row within a pass of 4 rows
    const int64_t row0 = (int64_t)(W == 1 ? blockIdx.x >> 2 : blockIdx.x) * 128;
    const int64_t col = (int64_t)blockIdx.y * 128 + c16 * 8;
    uint8_t *sb = reinterpret_cast<uint8_t *>(s_scale[W == 1 ? 0 : wave]);
    // This lane's rows are rb + pass_row(i) (i = 0..7) of the tile; their
    // addresses advance by fixed steps, computed once.
    const int rb = wave * 8 + rsub;
    Source in = src;
    in.start(row0 + rb, col);

    // Loads in flight per lane: two or four rows (all eight at once crowds
    // the L1 miss queue: measured slower).
    uint4 a[8], b[8];
    // Code offsets: row-major (row0 + r) * K + col; tiled (mxt_offset) the
    // 256-row super-block's slab of col plus 64 bytes per row and the row's
    // chunk swizzle -- the tile's 128 rows share the super-block.
    const int64_t Mp = (int64_t)gridDim.x * (W == 1 ? 32 : 128);
    const int64_t r0 = row0 & ~int64_t(255);
    const int64_t n = Mp - r0 < 256 ? Mp - r0 : 256;
    const int64_t out0 = tiled ? r0 * K + (col >> 6) * n * 64 + (col & 15) : (row0 + rb) * K + col;
    const int rl = (int)(row0 + rb - r0), chunk = (int)((col >> 4) & 3);
    // Rows two at a time; the next pair's loads are issued after this pair's
    // arithmetic and before its stores, so that waiting for them never means
    // waiting for stores (the vector-memory counter drains in issue order and
    // counts stores too).
    in.load(row0 + rb + pass_row(0) < M, 0, a[0], b[0]);
    in.load(row0 + rb + pass_row(1) < M, 1, a[1], b[1]);
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        int e[2];
        uint2 c[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) c[u] = in.quantize(a[i + u], b[i + u], e[u]);
        if (i + 2 < 8) {
            in.load(row0 + rb + pass_row(i + 2) < M, i + 2, a[i + 2], b[i + 2]);
            in.load(row0 + rb + pass_row(i + 3) < M, i + 3, a[i + 3], b[i + 3]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int rr = rl + pass_row(i + u);
            st_nt(q + out0 + (tiled ? (int64_t)(rr * 64 + ((chunk ^ mx_chunk_swizzle(rr)) << 4))
                                    : (int64_t)pass_row(i + u) * K),
                  c[u]);
            // Row j = 4 * ((i + u) & 1) + rsub of quarter (i + u) >> 1.
            if ((c16 & 3) == 0) sb[(4 * ((i + u) & 1) + rsub) * 16 + ((i + u) >> 1) * 4 + (c16 >> 2)] = (uint8_t)e[u];
        }
    }
    __syncthreads();
    // This wave's 128 contiguous bytes of the tile's 512-byte scale chunk:
    // rows 8w .. 8w + 7 of every quarter.
    uint8_t *chunk0 = scales + ((int64_t)(row0 >> 7) * (K >> 7) + blockIdx.y) * 512 + wave * 128;
    if (lane < 8)
        *reinterpret_cast<uint4 *>(chunk0 + lane * 16) = reinterpret_cast<const uint4 *>(sb)[lane];
}

// The SwiGLU quantizer's kernel: U 16-byte vectors of g and of v per lane
// (U = 2, or 1 for an odd chunk count), all loads issued first.  A wave owns
// rows r, r + 32, r + 64, r + 96 of a 128-row tile (r < 32) over U adjacent
// 128-column chunks, lanes 16j .. 16j + 15 holding row r + 32j, 8 columns of
// each chunk.  Per chunk its 16 exponents (4 rows x 4 blocks of 32) are the
// 16 contiguous bytes r * 16 .. r * 16 + 15 of that tile's 512-byte scale
// chunk: lane 16j gathers row j's four by DPP row shifts, and the four dword
// stores of one instruction cover the 16 bytes.  The four waves of a
// workgroup take four adjacent U-chunk groups of the same rows, and
// consecutive workgroups the next four.  Rows in [M, Mp) read as zeros
// (codes 0, the exponent of 0), as in k_quant_tile.  The 32 groups of a
// scale chunk come from 32 workgroups, and the scale bytes reach HBM about
// twice (3 % of the launch's writes).  The SiLU makes this
// source arithmetic-heavy (~24 vector instructions per element), and many
// short waves overlap it with the loads better than k_quant_tile's eight rows
// per lane: [4352, 12288] 54.7 -> 46.1 us, [16640, 12288] 212 -> 162 us (same
// box; addresses, tile and row in scalar registers, no division, U = 2; one
// chunk per lane measured 47.5 / 175 us, four 47.5 / 172 us).  The plain
// quantizer stays on k_quant_tile (8.53 against 9.0-10.0 us in this form).
template <class Source, int U>
__global__ __launch_bounds__(256) void k_quant_rows(Source src, uint8_t *__restrict__ q,
                                                    uint8_t *__restrict__ scales, int64_t M, int64_t K,
                                                    int64_t Mp, uint32_t nk, int tiled, int64_t g0) {
    const int lane = threadIdx.x & 63, j = lane >> 4, c16 = lane & 15;
    // Wave-uniform position (scalar registers): the four waves of a workgroup
    // take column-chunk groups tcu = 4 blockIdx.x .. + 3 (chunks U tcu ..
    // U tcu + U - 1) of the same rows, and consecutive workgroups the next
    // groups (walking along the rows, as a copy would); row r32 of each
    // quarter of tile tr from g0 + blockIdx.y.
    const uint32_t tcu = blockIdx.x * 4 + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if ((tcu + 1) * U > nk) return;  // past the last group of a row (wave-uniform, no barrier)
    const int64_t grp = g0 + blockIdx.y;
    const int64_t tr = grp >> 5;
    const int r32 = (int)(grp & 31);
    const int64_t row0 = tr * 128 + r32;           // the wave's first row; lane rows row0 + 32 j
    const int64_t row = row0 + j * 32;
    uint4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) src.load_at(row0, j, (int64_t)(tcu * U + u) * 128 + c16 * 8, row < M, a[u], b[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t tc = tcu * U + u;
        int e;
        const uint2 c = src.quantize(a[u], b[u], e);
        // Code offset: row-major row * K + col, or mxt_offset(row, col, Mp,
        // K), whose 256-row super-block (r0, n rows) and chunk swizzle (bits
        // 1-3 of the row: those of r32) are the wave's.
        int64_t off;
        if (tiled) {
            const int64_t r0 = (tr * 128) & ~int64_t(255);
            const int64_t n = Mp - r0 < 256 ? Mp - r0 : 256;
            const int sw = mx_chunk_swizzle(row0);
            off = r0 * K + ((int64_t)tc * 2 + (c16 >> 3)) * n * 64 + (row - r0) * 64 +
                  ((((c16 >> 1) & 3) ^ sw) << 4) + (c16 & 1) * 8;
        } else {
            off = row * K + (int64_t)tc * 128 + c16 * 8;
        }
        st_nt(q + off, c);
        const uint32_t e1 = dpp_mov<DPP_ROW_SHL4>((uint32_t)e);
        const uint32_t e2 = dpp_mov<DPP_ROW_SHL8>((uint32_t)e);
        const uint32_t e3 = dpp_mov<DPP_ROW_SHL12>((uint32_t)e);
        if (c16 == 0)
            *reinterpret_cast<uint32_t *>(scales + (tr * nk + tc) * 512 + r32 * 16 + j * 4) =
                (uint32_t)e | (e1 << 8) | (e2 << 16) | (e3 << 24);
    }
}

// Grid of k_quant_rows: ceil(K / (512 U)) groups of four U-chunk groups x
// (Mp / 128) * 32 row groups, workgroups of four waves; grid y is at most
// 65535, so larger row counts take several launches.  U = 2 (two chunks per
// lane, both loads issued first) when the chunk count is even, else 1.
template <class Source, int U>
static void launch_quant_rows_u(const Source &src, uint8_t *q, uint8_t *scales, int64_t M, int64_t K, int tiled,
                                hipStream_t st) {
    const int64_t Mp = (M + 127) / 128 * 128;
    const uint32_t nk = (uint32_t)(K / 128);
    const int64_t groups = Mp / 128 * 32;
    for (int64_t g0 = 0; g0 < groups; g0 += 65535) {
        const int64_t n = groups - g0 < 65535 ? groups - g0 : 65535;
        launch(k_quant_rows<Source, U>, dim3((nk / U + 3) / 4, (unsigned)n), dim3(256), 0, st, src, q, scales, M, K,
               Mp, nk, tiled, g0);
    }
}
template <class Source>
static void launch_quant_rows(const Source &src, uint8_t *q, uint8_t *scales, int64_t M, int64_t K, int tiled,
                              hipStream_t st) {
    if ((K / 128) % 2 == 0)
        launch_quant_rows_u<Source, 2>(src, q, scales, M, K, tiled, st);
    else
        launch_quant_rows_u<Source, 1>(src, q, scales, M, K, tiled, st);
}

// Workgroups of one wave (W = 1) or four (W = 4): the launch shape of the
// quantizers.
constexpr int QUANT_WAVES = 1;

static int launch_quant_checks(const char *what, int64_t M, int64_t K) {
    QIM_REQUIRE(M > 0 && K > 0, QIM_ERR_SHAPE, "%s: empty input (M=%lld, K=%lld)", what, (long long)M, (long long)K);
    QIM_REQUIRE(K % 128 == 0, QIM_ERR_SHAPE, "%s: K=%lld is not a multiple of 128", what, (long long)K);
    QIM_REQUIRE((M + 127) / 128 * 8 * (K / 128) < (1ll << 31) && K / 128 < 65536, QIM_ERR_SHAPE, "%s: too large",
                what);
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
    dim3 grid((unsigned)((M + 127) / 128 * (4 / QUANT_WAVES)), (unsigned)(K / 128));
    QuantSource src{(const uint16_t *)x, ldx};
    launch(k_quant_tile<QuantSource, QUANT_WAVES>, grid, dim3(64 * QUANT_WAVES), 0, as_stream(stream), src, (uint8_t *)q,
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
    SwigluSource src{(const uint16_t *)g, ldg, (const uint16_t *)v, ldv};
    launch_quant_rows(src, (uint8_t *)q, (uint8_t *)scales, M, F, tiled, as_stream(stream));
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
