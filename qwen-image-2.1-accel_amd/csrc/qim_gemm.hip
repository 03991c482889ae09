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
// Workgroup tile 256 x 256, 4 waves in a 2 x 2 grid, each wave a 128 x 128
// block of 4 x 4 MFMA tiles (256 fp32 accumulators per lane, in AGPRs).
// K advances 64 bytes per stage through a 4-deep LDS ring (34 KiB per stage:
// A 256 x 64, B 256 x 64, and the 1 KiB A / B scale chunks of the stage's
// 128-K group).  Operands move global -> LDS with global_load_lds_dwordx4
// (no register staging): lane i of an instruction writes LDS bytes
// [16i, 16i+16) of a 1 KiB segment, so the bank swizzle is applied to the
// source address instead -- LDS holds logical 16-byte chunk c of tile row r at
// chunk c ^ (((r >> 1) ^ (r >> 2)) & 3), which makes 8 (and 16) lanes reading
// 8 (16) consecutive rows at one chunk hit distinct banks.  Stage s+4 is
// issued at the top of stage s, right after the barrier that proves every wave
// has consumed ring slot s % 4; the fragments of stage s+1 are read from LDS
// while the 16 MFMAs of stage s run.
#include <type_traits>

#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

constexpr int BM = 256, BN = 256, BK = 64, NSTAGE = 4;
constexpr int TILE_BYTES = BM * BK;                          // 16 KiB per operand per stage
constexpr int SCALE_BYTES = 1024;                            // two 512-byte chunks per operand
constexpr int STAGE_BYTES = 2 * TILE_BYTES + 2 * SCALE_BYTES;  // 34 KiB
constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;              // 136 KiB
// Loads per wave per stage: 4 A + 4 B (16 B each), plus 2 of 4 B for the
// scales in even stages only: a 128-K scale group spans two stages, and odd
// stages reuse the even stage's scales from registers.
constexpr int LOADS_EVEN = 10, LOADS_ODD = 8;

struct GemmArgs {
    const uint8_t *aq, *as, *bq, *bs;
    int64_t M, Mp, N, K;
    const uint16_t *bias, *gate, *res;
    int64_t seq;
    void *out;
    int64_t ldo;
    uint8_t *out_scales;
    int tiles_m, tiles_n;  // 256 x 256 tiles (tiles_n: whole 256-column blocks)
    int main_tiles;  // whole tiles; workgroups past them compute quarter tiles of the rest
    int quarters;    // quarter tiles of whole tiles; the ones after them cover a last
                     // 128-column block (N % 256 == 128), 128 rows each
    int a_tiled, b_tiled, out_tiled;  // code layouts (mxt_offset) of A, B and a quantized output
    // QIM_EPI_QK_NORM_ROPE: head weights, RoPE table (seq rows of 128 fp32),
    // and the column ends of Q (H * 128) and K (2 * H * 128).
    const uint16_t *wq, *wk;
    const float *freqs;
    float epsq, epsk;
    int64_t q_cols, qk_cols;
    // With vt set, the V columns leave as the attention's V^T tiles instead:
    // tile (batch, head, key block) of 128 rows (d) x 64 keys at
    // ((batch * H + head) * vt_nkb + key block) * 8192 elements, vt_nkb =
    // seq / 64 (seq % 64 == 0).
    uint16_t *vt;
    int64_t vt_nkb;
    // Split-K tail (qim_mxfp8_gemm_ws): with ksplit > 1 each quarter tile of
    // the last partial round is computed by ksplit workgroups over disjoint
    // ranges of K, which write their fp32 accumulators to ws; k_mx_gemm_tail
    // then sums them in a fixed order and runs the epilogue.
    float *ws;
    int ksplit;
};

// qim_mxfp8_gemm_qk_norm_rope_vt: the QK-norm + RoPE epilogue whose V columns
// leave as V^T tiles (an instantiation of its own, so the plain QKV kernel
// carries none of it).  Its outputs are read next by the attention core, so
// it stores through the caches (block @1024^2 with attention: 881 -> 874 us)
// where every other epilogue streams its output past them.
constexpr int EPI_QKV_VT = 6;
template <int EPI>
constexpr bool is_qk_epi() { return EPI == QIM_EPI_QK_NORM_ROPE || EPI == EPI_QKV_VT; }
// QIM_EPI_NONE with an fp32 or fp16 output (QIM_GEMM_OUT_F32 / _F16): the
// reference's out_dtype of torch._scaled_mm.
constexpr int EPI_F32 = 7, EPI_F16 = 8;

template <typename V>
__device__ __forceinline__ void st_out(bool cached, void *ptr, const V &v) {
    if (cached)
        *reinterpret_cast<V *>(ptr) = v;
    else
        st_nt(ptr, v);
}

__device__ __forceinline__ int kswz(int row) { return mx_chunk_swizzle(row); }
// LDS byte offset of logical 16-byte chunk c of tile row `row` (64-byte rows).
__device__ __forceinline__ int lds_off(int row, int c) { return row * BK + ((c ^ kswz(row)) << 4); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Stage-0 source offset of this lane's 16 bytes in the DMA of the 16 tile
// rows [grp, grp + 16) of an (R, K) code matrix whose tile starts at row m0:
// lane i lands at row grp + i/4, physical LDS chunk i%4.  Row-major codes:
// the lane's logical chunk of its row.  Tiled codes (mxt_offset): the group is
// already the LDS image, 1 KiB contiguous.  Rows past R are clamped into the
// matrix; they only feed output rows that are never stored.
__device__ __forceinline__ uint32_t opnd_offset(int64_t m0, int grp, int lane, int64_t R, int64_t K, bool tiled) {
    if (!tiled) {
        const int row = grp + (lane >> 2);
        int64_t r = m0 + row;
        r = r < R ? r : R - 1;
        return (uint32_t)(r * K + (((lane & 3) ^ kswz(row)) << 4));
    }
    int64_t rg = m0 + grp;
    rg = rg <= R - 16 ? rg : R - 16;
    const int64_t r0 = rg & ~int64_t(255);
    return (uint32_t)(r0 * K + (rg - r0) * 64 + lane * 16);
}
// Advance of those offsets per 64-byte K stage (wave-uniform).
__device__ __forceinline__ uint32_t opnd_step(int64_t m0, int64_t R, bool tiled) {
    if (!tiled) return BK;
    const int64_t r0 = m0 & ~int64_t(255);
    return (uint32_t)((R - r0 < 256 ? R - r0 : 256) * 64);
}

// Per-lane source offsets of the 10 load instructions of a stage (stage 0);
// stage s adds s * astep / s * bstep (operands) or (s / 2) * 512 (scales).
struct LoadPlan {
    uint32_t a[4], b[4];      // byte offsets into aq / bq
    uint32_t sc[2];           // byte offsets into sc_base
    const uint8_t *sc_base[2];  // as (A scale quarter) or bs (B scale quarter); wave-uniform
    uint32_t astep, bstep;
    int wave;
};

__device__ __forceinline__ LoadPlan make_plan(const GemmArgs &p, int64_t m0, int64_t n0) {
    LoadPlan L;
    const int lane = threadIdx.x & 63;
    L.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int grp = (L.wave * 4 + j) * 16;
        L.a[j] = opnd_offset(m0, grp, lane, p.Mp, p.K, p.a_tiled);
        L.b[j] = opnd_offset(n0, grp, lane, p.N, p.K, p.b_tiled);
    }
    L.astep = opnd_step(m0, p.Mp, p.a_tiled);
    L.bstep = opnd_step(n0, p.N, p.b_tiled);
    const int64_t kt = p.K / 128;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int idx = L.wave * 2 + j;          // 0..3: A scale quarter, 4..7: B scale quarter
        const int off = (idx & 3) * 256 + lane * 4;
        const int g = off >> 9, o = off & 511;
        L.sc_base[j] = idx >= 4 ? p.bs : p.as;
        int64_t grow;
        if (idx < 4) {
            grow = m0 / 128 + g;
            grow = grow < p.Mp / 128 ? grow : p.Mp / 128 - 1;
        } else {
            grow = n0 / 128 + g;
        }
        L.sc[j] = (uint32_t)(grow * kt * 512 + o);
    }
    return L;
}

// LDS DMA through inline asm: the compiler does not see these as LDS writes,
// so it does not force vmcnt(0) before every LDS read (it cannot prove the
// ring slots disjoint); the ring's own vmcnt waits and s_barrier order them.
// M0 holds the wave-uniform LDS destination; lane i lands at M0 + 16i (4i for
// the dword form).  The destination is an "{m0}" operand, so the compiler
// writes M0 itself and knows its value at every statement; the s_nop covers
// the wait state between that write and the DMA's read of M0.
__device__ __forceinline__ void dma16(const uint8_t *base, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
                 "{m0}"(lds_addr)
                 : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *base, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base),
                 "{m0}"(lds_addr)
                 : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

template <bool SCALES>
__device__ __forceinline__ void issue_stage(const GemmArgs &p, const LoadPlan &L, uint8_t *slot, int s) {
    const uint32_t ka = (uint32_t)s * L.astep, kb = (uint32_t)s * L.bstep;
    const uint32_t base = lds_addr(slot);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(p.aq, L.a[j] + ka, base + (L.wave * 4 + j) * 1024);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(p.bq, L.b[j] + kb, base + TILE_BYTES + (L.wave * 4 + j) * 1024);
    if constexpr (SCALES) {
        const uint32_t gofs = (uint32_t)(s >> 1) * 512;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            dma4(L.sc_base[j], L.sc[j] + gofs, base + 2 * TILE_BYTES + (L.wave * 2 + j) * 256);
    }
}

struct Frags {
    i32x8_t a[4], b[4];
    uint4 sa, sb;  // scale dwords of row tiles 0..3 (exponents of the 128-K group's 4 blocks)
};

// Fragment reads of one ring slot (stage), one operand tile at a time.
__device__ __forceinline__ i32x8_t read_tile(const uint8_t *base, int row, int kh) {
    const uint4 lo = *reinterpret_cast<const uint4 *>(base + lds_off(row, kh));
    const uint4 hi = *reinterpret_cast<const uint4 *>(base + lds_off(row, 2 + kh));
    return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}
// The four scale dwords of a wave's row tiles t = 0..3 (local rows
// r = h*128 + t*32 + lr of a 1 KiB scale tile, whose dword for row r sits at
// (r/128)*512 + (r%32)*16 + ((r%128)/32)*4 = h*512 + lr*16 + t*4): contiguous,
// so one 16-byte read.
__device__ __forceinline__ uint4 read_scales(const uint8_t *base, int h, int lr) {
    return *reinterpret_cast<const uint4 *>(base + h * 512 + lr * 16);
}

__device__ __forceinline__ void read_frags(const uint8_t *slot, int wm, int wn, int lr, int kh, Frags &f) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        f.a[t] = read_tile(slot, wm * 128 + t * 32 + lr, kh);
        f.b[t] = read_tile(slot + TILE_BYTES, wn * 128 + t * 32 + lr, kh);
    }
    f.sa = read_scales(slot + 2 * TILE_BYTES, wm, lr);
    f.sb = read_scales(slot + 2 * TILE_BYTES + SCALE_BYTES, wn, lr);
}

// Every stage issues its loads unconditionally (past the end of K they
// re-read the last stage into a ring slot that is never read again), so at
// the top of stage s the outstanding loads are always those of stages s+1,
// s+2, s+3, and "stage s+1 landed" is always vmcnt(LOADS_EVEN + LOADS_ODD).  Keeping the stage
// free of branches keeps it one basic block, which the explicit schedule
// below needs.

#define QIM_SCHED() __builtin_amdgcn_sched_barrier(0)

// One pipeline step with an explicit instruction order (the scheduler may not
// move anything across QIM_SCHED()).  With one wave per SIMD the MFMA pipe
// idles whenever the wave stalls, so the 16 MFMAs of stage s (operands in
// `cur`) are spread around everything else the stage has to do:
//   MFMA 0 | wait for stage s+1's DMA, barrier | MFMA 1-3, each followed by a
//   third of the 10 DMA issues of stage s+4 | MFMA 4-15, each followed by two
//   of the 24 LDS reads of stage s+1's operands into `nxt`.
// The scale dwords hold the exponents of K blocks 0..3 of the stage's 128-K
// group; the upper half-wave's are shifted down one byte so that byte
// (s % 2) * 2 is every lane's own block and op_sel can select it uniformly.
template <int PAR>
__device__ __forceinline__ void pipeline_step(const GemmArgs &p, const LoadPlan &L, uint8_t *lds, int s, int S,
                                              f32x16_t (&acc)[4][4], const Frags &cur, Frags &nxt, int wm,
                                              int wn, int lr, int kh) {
    int sa[4], sb[4];
    const uint32_t ca[4] = {cur.sa.x, cur.sa.y, cur.sa.z, cur.sa.w}, cb[4] = {cur.sb.x, cur.sb.y, cur.sb.z, cur.sb.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        sa[t] = (int)(ca[t] >> (8 * kh));
        sb[t] = (int)(cb[t] >> (8 * kh));
    }
#define QIM_MF(i, j)                                                                                          \
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(cur.a[i], cur.b[j], acc[i][j], 0, 0, PAR * 2, \
                                                                sa[i], PAR * 2, sb[j])
    uint8_t *fill = lds + (s & 3) * STAGE_BYTES;
    const uint8_t *next = lds + ((s + 1) & 3) * STAGE_BYTES;  // stale at the last stage; unused then
    const int sl = s + 4 < S ? s + 4 : S - 1;                 // stage to load (clamped)
    const uint32_t ka = (uint32_t)sl * L.astep, kb = (uint32_t)sl * L.bstep, gofs = (uint32_t)(sl >> 1) * 512;
    const uint32_t fb = lds_addr(fill);
    const int ra0 = wm * 128 + lr, rb0 = wn * 128 + lr;

    const uint8_t *nsa = next + 2 * TILE_BYTES, *nsb = nsa + SCALE_BYTES;
    const uint8_t *scb0 = L.sc_base[0], *scb1 = L.sc_base[1];
    const uint32_t w4 = L.wave * 4;
#define QIM_STEP(mi, mj, work) QIM_MF(mi, mj); QIM_SCHED(); work; QIM_SCHED()
    QIM_MF(0, 0);
    QIM_SCHED();
    wait_vmcnt<LOADS_EVEN + LOADS_ODD>();
    block_barrier();
    QIM_SCHED();
    QIM_STEP(0, 1, dma16(p.aq, L.a[0] + ka, fb + (w4 + 0) * 1024));
    // The next stage's scales: the same 128-K group after an even stage (kept
    // in registers), a new group after an odd one (one 16-byte read each).
    QIM_STEP(0, 2, dma16(p.aq, L.a[1] + ka, fb + (w4 + 1) * 1024);
             if constexpr (PAR == 0) nxt.sa = cur.sa; else nxt.sa = read_scales(nsa, wm, lr));
    QIM_STEP(0, 3, dma16(p.aq, L.a[2] + ka, fb + (w4 + 2) * 1024);
             if constexpr (PAR == 0) nxt.sb = cur.sb; else nxt.sb = read_scales(nsb, wn, lr));
    QIM_STEP(1, 0, dma16(p.aq, L.a[3] + ka, fb + (w4 + 3) * 1024); nxt.a[0] = read_tile(next, ra0, kh));
    QIM_STEP(1, 1, dma16(p.bq, L.b[0] + kb, fb + TILE_BYTES + (w4 + 0) * 1024);
             nxt.b[0] = read_tile(next + TILE_BYTES, rb0, kh));
    QIM_STEP(1, 2, dma16(p.bq, L.b[1] + kb, fb + TILE_BYTES + (w4 + 1) * 1024);
             nxt.b[1] = read_tile(next + TILE_BYTES, rb0 + 32, kh));
    QIM_STEP(1, 3, dma16(p.bq, L.b[2] + kb, fb + TILE_BYTES + (w4 + 2) * 1024);
             nxt.b[2] = read_tile(next + TILE_BYTES, rb0 + 64, kh));
    QIM_STEP(2, 0, dma16(p.bq, L.b[3] + kb, fb + TILE_BYTES + (w4 + 3) * 1024);
             nxt.b[3] = read_tile(next + TILE_BYTES, rb0 + 96, kh));
    // Logical stage s + 4 has this stage's parity: scales in even stages only.
    QIM_STEP(2, 1, if constexpr (PAR == 0) dma4(scb0, L.sc[0] + gofs, fb + 2 * TILE_BYTES + (L.wave * 2 + 0) * 256);
             nxt.a[1] = read_tile(next, ra0 + 32, kh));
    QIM_STEP(2, 2, if constexpr (PAR == 0) dma4(scb1, L.sc[1] + gofs, fb + 2 * TILE_BYTES + (L.wave * 2 + 1) * 256);
             nxt.a[2] = read_tile(next, ra0 + 64, kh));
    QIM_STEP(2, 3, nxt.a[3] = read_tile(next, ra0 + 96, kh));
    QIM_MF(3, 0);
    QIM_MF(3, 1);
    QIM_MF(3, 2);
    QIM_MF(3, 3);
    QIM_SCHED();
#undef QIM_STEP
#undef QIM_MF
}

// Tile id -> (tile row, tile column): groups of 4 tile-rows, column-major
// inside a group, so consecutive tiles share B columns and, within a group, A
// rows in L2.
__device__ __forceinline__ void tile_coords(const GemmArgs &p, int t, int &tm, int &tn) {
    constexpr int GM = 4;
    const int per_group = GM * p.tiles_n;
    const int group = t / per_group, first = group * GM;
    const int gm = p.tiles_m - first < GM ? p.tiles_m - first : GM;
    const int r = t - group * per_group;
    tm = first + r % gm;
    tn = r / gm;
}

// Workgroup -> tile.  Workgroups are dispatched round-robin over the 8 XCDs,
// so workgroup w runs on XCD w % 8; tile ids are remapped so that each XCD
// owns one contiguous range, walked in groups of 4 tile-rows (column-major
// inside a group) so the tiles resident on one XCD share A rows and B columns
// in that XCD's L2.
__device__ __forceinline__ void tile_of(const GemmArgs &p, int &tm, int &tn) {
    const int nt = p.main_tiles;
    int t = blockIdx.x;
    if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
    tile_coords(p, t, tm, tn);
}

// ------------------------------------------------------------ SiLU table --
// The SwiGLU epilogues look bf16(silu(g)) up instead of computing it (the
// estimate, its band test and the rounding cost ~14 vector instructions per
// output, on one wave per SIMD with nothing to hide them).  The table holds
// every bf16 g with biased exponent 101..132 (2^-26 <= |g| < 64): entry i of
// a sign is g = bits 0x3280 + i, positive at byte 2i, negative at 8192 + 2i,
// so for the packed bf16 pair G the two byte addresses come from
// P = G - 0x3280 (per half) as (P << 1) for bits 0..12 and (P >> 2) for the
// sign at bit 13; a value is in the table when bits 12..14 of P are clear.
// Entries are computed with silu_bf16 (bit-identical to the reference's
// rounding) by each workgroup while its first stages' loads are in flight;
// the rest (|g| < 2^-26, |g| >= 64, NaN) takes silu_bf16 itself.
constexpr int SILU_TAB_BYTES = 16384;
constexpr uint16_t SILU_TAB_BASE = 0x3280;
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

template <int EPI>
constexpr int ring_offset() { return (EPI == QIM_EPI_SWIGLU || EPI == QIM_EPI_SWIGLU_QUANT) ? SILU_TAB_BYTES : 0; }

__device__ __forceinline__ void fill_silu_table(uint8_t *tab) {
    // 256 threads x 16 dwords (two entries each), dword d = c * 256 + t.
#pragma unroll
    for (int c0 = 0; c0 < 16; c0 += 4) {
        float g[8], y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t e = 2 * ((c0 + j / 2) * 256 + threadIdx.x) + (j & 1);  // entry 0..8191
            const uint32_t b = SILU_TAB_BASE + (e & 4095) + ((e >> 12) << 15);
            g[j] = __uint_as_float(b << 16);
        }
        silu_bf16_n<8>(g, y);
#pragma unroll
        for (int j = 0; j < 8; j += 2)
            *reinterpret_cast<uint32_t *>(tab + 4 * ((c0 + j / 2) * 256 + threadIdx.x)) = pack_bf16x2(y[j], y[j + 1]);
    }
}

// bf16(silu(g)) for the two bf16 values of gp (low half first), from the
// table, as bf16 bits; `bad` collects the bits that mark a value outside it.
__device__ __forceinline__ void silu_lookup2(const uint8_t *tab, uint32_t gp, uint32_t &y0, uint32_t &y1,
                                             uint32_t &bad) {
    const u16x2_t P = __builtin_bit_cast(u16x2_t, gp) - (u16x2_t){SILU_TAB_BASE, SILU_TAB_BASE};
    bad |= __builtin_bit_cast(uint32_t, P) & 0x70007000u;
    const uint32_t a = __builtin_bit_cast(uint32_t, (u16x2_t)(P << (u16x2_t){1, 1}));
    const uint32_t b = __builtin_bit_cast(uint32_t, (u16x2_t)(P >> (u16x2_t){2, 2}));
    uint32_t w;  // bits 0..12 of each half from a, bit 13 (and the zero bits above it) from b
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(w) : "s"(0x1fff1fffu), "v"(a), "v"(b));
    y0 = *reinterpret_cast<const uint16_t *>(tab + (w & 0xffffu));
    y1 = *reinterpret_cast<const uint16_t *>(tab + (w >> 16));
}

// ------------------------------------------------------------- epilogue --
// Two passes per 64 rows (two MFMA row tiles) of the wave's block, through a
// wave-private LDS region (the ring is free once the main loop has drained):
//  1. registers -> LDS: the per-element part of the epilogue (bias add, or
//     SwiGLU of the gate/up tile pair), then bf16.  Accumulators i = 4g'..4g'+3
//     of an MFMA tile are 4 consecutive rows of one column, so they are packed
//     two rows per dword (v_cvt_pk_bf16_f32) and stored with one 8-byte write:
//     the region holds, per group of 4 rows and per column, the column's 4
//     values (8 bytes).
//  2. LDS -> global: each lane reads the 4 x 8 block of 4 rows x 8 columns
//     (4 x 16 bytes), regroups it into the 4 rows' 16-byte vectors with byte
//     permutes, applies the per-row part (gated residual with coalesced
//     res/gate loads, or MXFP8 quantization of 32-column blocks = 4 lanes) and
//     stores each row vector (8 bytes for codes).
// Accumulator i of MFMA tile (ti, tj) is row 32ti + 8(i/4) + 4(l/32) + i%4,
// column 32tj + l%32 of the wave's block of TI x TJ MFMA tiles, whose first
// row is row0 and first GEMM column gcol0.  Within a row group, column c sits
// at 8c + 16(c/8) bytes: the pass-2 lanes of a 16-lane read group start 80
// bytes apart, on disjoint banks.
template <int W>
__device__ __forceinline__ int epi_col_offset(int c) { return c * 8 + (c >> 3) * 16; }

template <int EPI, int TI, int TJ>
__device__ __forceinline__ void epilogue(const GemmArgs &p, f32x16_t (&acc)[TI][TJ], uint8_t *lds,
                                         [[maybe_unused]] const uint8_t *tab, int64_t row0, int64_t gcol0, int lane,
                                         int wave) {
    if constexpr (EPI == EPI_F32 || EPI == EPI_F16) {
        // Straight from the accumulators: for each register, 32 lanes store
        // 32 consecutive columns of one row (128 or 64 contiguous bytes).
        const int lr = lane & 31, kh = lane >> 5;
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t row = row0 + 32 * ti + 8 * (i / 4) + 4 * kh + (i % 4);
                if (row >= p.M) continue;
#pragma unroll
                for (int tj = 0; tj < TJ; ++tj) {
                    const int64_t o = row * p.ldo + gcol0 + 32 * tj + lr;
                    if constexpr (EPI == EPI_F32)
                        __builtin_nontemporal_store(acc[ti][tj][i], reinterpret_cast<float *>(p.out) + o);
                    else
                        __builtin_nontemporal_store((_Float16)acc[ti][tj][i], reinterpret_cast<_Float16 *>(p.out) + o);
                }
            }
        return;
    } else {
    constexpr bool SWI = EPI == QIM_EPI_SWIGLU || EPI == QIM_EPI_SWIGLU_QUANT;
    constexpr int W = SWI ? 16 * TJ : 32 * TJ;  // output columns of this wave
    constexpr int RGS = W * 8 + (W / 8) * 16;   // bytes per group of 4 rows
    constexpr int LPR = W / 8;                  // lanes per row group in pass 2
    constexpr int GPI = 64 / LPR;               // row groups per pass-2 step
    const int lr = lane & 31, kh = lane >> 5;
    uint8_t *reg = lds + wave * (16 * RGS);
    const int64_t col0 = SWI ? gcol0 / 2 : gcol0;  // first output column
    // SwiGLU -> MXFP8 in a whole tile (TI = 4): the two waves of a 128-row
    // block (wave & 1 = 0, 1) together produce its 512-byte scale chunk (128
    // rows x the tile's 4 blocks of 32 output columns).  Their exponent bytes
    // are staged in LDS, after every wave's staging region, and the chunk
    // leaves as 32 whole 16-byte stores: byte stores straight to memory wrote
    // each 64-byte segment of the scales in many partial writes (+45 % of the
    // kernel's HBM writes at 4352 x 24576 x 3072).
    constexpr bool STAGE_SC = EPI == QIM_EPI_SWIGLU_QUANT && TI == 4;
    [[maybe_unused]] uint8_t *const sc_stage = lds + 4 * 16 * RGS + (wave >> 1) * 512;
    const int64_t F = p.N / 2;
    // QKV projection with vt: this wave's V columns are staged per column (64
    // keys, VT_COL bytes apart; the odd stride spreads the pass-1 writes of a
    // 32-lane group over all banks) and leave as V^T tiles.
    [[maybe_unused]] constexpr int VT_COL = 136;
    static_assert(W * VT_COL <= 16 * RGS, "V^T staging fits the wave's region");
    const bool vtw = EPI == EPI_QKV_VT && col0 >= p.qk_cols;
    float bias[TJ] = {};
    if constexpr (EPI == QIM_EPI_BIAS) {
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) bias[tj] = bf16_to_f32(p.bias[gcol0 + tj * 32 + lr]);
    }
#pragma unroll
    for (int half = 0; half < TI / 2; ++half) {
        // The residual rows of this half's pass 2, loaded before pass 1 so that
        // their latency overlaps it (rows past M: clamped, not stored).
        [[maybe_unused]] uint4 rpre[16 / GPI][4];
        // The gate vector of this half's rows when they are one batch's (a
        // per-row load in pass 2 would sit between stores: see pass 2).
        [[maybe_unused]] uint4 gpre = make_uint4(0, 0, 0, 0);
        [[maybe_unused]] bool gate_once = false;
        if constexpr (EPI == QIM_EPI_GATED_RESIDUAL) {
            const int cl = lane % LPR, gl = lane / LPR;
            // Row h0 + lr, clamped to M - 1: a uniform base row hc and
            // min(lr, M - 1 - hc) rows past it (32-bit per row).
            const int64_t h0 = row0 + half * 64, hc = h0 < p.M ? h0 : p.M - 1;
            const uint16_t *rb = p.res + hc * p.N;
            const uint32_t lmax = (uint32_t)(p.M - 1 - hc), rcol = (uint32_t)(col0 + cl * 8);
#pragma unroll
            for (int it = 0; it < 16 / GPI; ++it)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t lr = (uint32_t)(4 * (it * GPI + gl) + r);
                    rpre[it][r] = ld_nt(rb + ((lr < lmax ? lr : lmax) * (uint32_t)p.N + rcol));
                }
            const int64_t h1 = h0 + 63 < p.M ? h0 + 63 : p.M - 1;
            const uint32_t b0 = (uint32_t)hc / (uint32_t)p.seq;
            gate_once = b0 == (uint32_t)h1 / (uint32_t)p.seq;
            gpre = *reinterpret_cast<const uint4 *>(p.gate + (int64_t)b0 * p.N + col0 + cl * 8);
        }
        // pass 1
        if constexpr (SWI) {
            // bf16(bf16(silu(g)) * v) for the half's 8 row groups: g and v
            // rounded to bf16 in pairs, every table read of the half issued
            // before the first is used (their latency overlaps the rest), one
            // rarely taken branch for values outside the table (recomputed
            // from the accumulators), then the products; the store's bf16
            // packing is the final rounding.
            constexpr int NP = TJ;  // pairs per row group: TJ / 2 column pairs x 2 row pairs
            uint32_t up[2][4][NP], bad = 0;
            uint32_t y[2][4][2 * NP];  // bf16 bits
#pragma unroll
            for (int tl = 0; tl < 2; ++tl)
#pragma unroll
                for (int ig = 0; ig < 4; ++ig)
#pragma unroll
                    for (int u = 0; u < TJ / 2; ++u)
#pragma unroll
                        for (int e = 0; e < 4; e += 2) {
                            const int ti = half * 2 + tl, k = 2 * u + e / 2;
                            const uint32_t gp = pack_bf16x2(acc[ti][2 * u][4 * ig + e], acc[ti][2 * u][4 * ig + e + 1]);
                            up[tl][ig][k] =
                                pack_bf16x2(acc[ti][2 * u + 1][4 * ig + e], acc[ti][2 * u + 1][4 * ig + e + 1]);
                            silu_lookup2(tab, gp, y[tl][ig][2 * k], y[tl][ig][2 * k + 1], bad);
                        }
            // Keep the conversions below from being scheduled up against
            // their reads.
            __builtin_amdgcn_sched_barrier(0);
            if (__builtin_expect(bad != 0, 0)) {
#pragma unroll
                for (int tl = 0; tl < 2; ++tl)
#pragma unroll
                    for (int ig = 0; ig < 4; ++ig)
#pragma unroll
                        for (int u = 0; u < TJ / 2; ++u)
#pragma unroll
                            for (int e = 0; e < 4; e += 2) {
                                const int ti = half * 2 + tl, k = 2 * u + e / 2;
                                const uint32_t gp =
                                    pack_bf16x2(acc[ti][2 * u][4 * ig + e], acc[ti][2 * u][4 * ig + e + 1]);
#pragma unroll
                                for (int h = 0; h < 2; ++h) {
                                    const uint32_t gb = (gp >> (16 * h)) & 0xffffu;
                                    if (((gb - SILU_TAB_BASE) & 0x7000u) != 0)
                                        y[tl][ig][2 * k + h] = __float_as_uint(silu_bf16(__uint_as_float(gb << 16))) >> 16;
                                }
                            }
            }
#pragma unroll
            for (int tl = 0; tl < 2; ++tl)
#pragma unroll
                for (int ig = 0; ig < 4; ++ig) {
                    uint8_t *grp = reg + (tl * 8 + ig * 2 + kh) * RGS;  // rows 32tl + 8ig + 4kh + 0..3
                    float yy[2 * NP];
#pragma unroll
                    for (int i = 0; i < 2 * NP; ++i) yy[i] = __uint_as_float(y[tl][ig][i] << 16);
#pragma unroll
                    for (int u = 0; u < TJ / 2; ++u) {
                        const uint32_t v0 = up[tl][ig][2 * u], v1 = up[tl][ig][2 * u + 1];
                        *reinterpret_cast<uint2 *>(grp + epi_col_offset<W>(u * 32 + lr)) =
                            make_uint2(pack_bf16x2(yy[4 * u] * __uint_as_float(v0 << 16),
                                                   yy[4 * u + 1] * __uint_as_float(v0 & 0xffff0000u)),
                                       pack_bf16x2(yy[4 * u + 2] * __uint_as_float(v1 << 16),
                                                   yy[4 * u + 3] * __uint_as_float(v1 & 0xffff0000u)));
                    }
                }
        } else
#pragma unroll
        for (int tl = 0; tl < 2; ++tl) {
            const int ti = half * 2 + tl;
#pragma unroll
            for (int ig = 0; ig < 4; ++ig) {
                uint8_t *grp = reg + (tl * 8 + ig * 2 + kh) * RGS;  // rows 32tl + 8ig + 4kh + 0..3
                if (vtw) {
#pragma unroll
                    for (int tj = 0; tj < TJ; ++tj)
                        *reinterpret_cast<uint2 *>(reg + (tj * 32 + lr) * VT_COL + (32 * tl + 8 * ig + 4 * kh) * 2) =
                            make_uint2(pack_bf16x2(acc[ti][tj][4 * ig + 0], acc[ti][tj][4 * ig + 1]),
                                       pack_bf16x2(acc[ti][tj][4 * ig + 2], acc[ti][tj][4 * ig + 3]));
                } else {
#pragma unroll
                    for (int tj = 0; tj < TJ; ++tj) {
                        float y[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            y[e] = acc[ti][tj][4 * ig + e];
                            if constexpr (EPI == QIM_EPI_BIAS) y[e] = y[e] + bias[tj];
                        }
                        *reinterpret_cast<uint2 *>(grp + epi_col_offset<W>(tj * 32 + lr)) =
                            make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
                    }
                }
            }
        }
        // pass 2 (LDS operations of one wave complete in order: no wait needed)
        if (vtw) {
            // V^T tiles: this half's 64 rows are one key block (seq % 64 ==
            // 0).  Tile row d is 8 chunks of 16 bytes; physical chunk pc holds
            // logical chunk c = pc ^ ((d >> 1) & 7): keys 16(c/2) + 4(c%2) +
            // 0..3, then the same 8 keys later.  Eight lanes per row: each
            // store instruction writes 1 KiB contiguous.
            const int64_t R = row0 + half * 64;
            if (R < p.M) {
                const int64_t bt = R / p.seq, kb = (R - bt * p.seq) / 64, vc = col0 - p.qk_cols;
                uint16_t *tile = p.vt + ((bt * (p.q_cols / 128) + vc / 128) * p.vt_nkb + kb) * (64 * 128);
#pragma unroll
                for (int it = 0; it < W / 8; ++it) {
                    const int dl = it * 8 + (lane >> 3), pc = lane & 7, d = (int)(vc & 127) + dl;
                    const int c = pc ^ ((d >> 1) & 7), k0 = 16 * (c >> 1) + 4 * (c & 1);
                    const uint2 lo = *reinterpret_cast<const uint2 *>(reg + dl * VT_COL + k0 * 2);
                    const uint2 hi = *reinterpret_cast<const uint2 *>(reg + dl * VT_COL + (k0 + 8) * 2);
                    *reinterpret_cast<uint4 *>(tile + d * 64 + pc * 8) = make_uint4(lo.x, lo.y, hi.x, hi.y);
                }
            }
            continue;
        }
        // Pass 2.  Loads issued between one row group's stores and the next
        // group's use would make the compiler wait for those stores too (the
        // vector-memory counter drains in issue order and counts stores), and
        // a per-row "row < M" branch makes every wait after it assume the
        // fewest outstanding operations.  So: the per-half gate vector and the
        // head weights are loaded before the loop, the QK epilogue's RoPE
        // rows one row group ahead (before the current group's stores), and a
        // half whose 64 rows are all below M takes a version of the loop
        // without per-row checks (every half, when M % 64 == 0).
        const int cl = lane % LPR, gl = lane / LPR;
        const int64_t col = col0 + cl * 8;
        [[maybe_unused]] const bool isq = col0 < p.q_cols;
        [[maybe_unused]] const int hc = (int)(col0 & 127) + cl * 8;  // column within the head
        [[maybe_unused]] float wt[8];
        [[maybe_unused]] float4 fr[2][4][2];  // RoPE (cos, sin) of 4 rows: this group's and the next's
        [[maybe_unused]] const bool qk_cols = is_qk_epi<EPI>() && col0 < p.qk_cols;
        auto load_freqs = [&](int it, float4 (&f)[4][2]) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = (uint32_t)(row0 + half * 64 + 4 * (it * GPI + gl) + r) % (uint32_t)p.seq;
                const float4 *fp = reinterpret_cast<const float4 *>(p.freqs + (int64_t)tok * 128 + hc);
                f[r][0] = fp[0];
                f[r][1] = fp[1];
            }
        };
        if constexpr (is_qk_epi<EPI>()) {
            if (qk_cols) {
                unpack8(*reinterpret_cast<const uint4 *>((isq ? p.wq : p.wk) + hc), wt);
                load_freqs(0, fr[0]);
            }
        }
        // MXFP8 output: the half's 64 rows lie in one 256-row group of the
        // tiled layout and one 128-row block of the scales, so each row's
        // code and scale offsets are a uniform base plus a per-lane 32-bit
        // offset plus a compile-time row term (times a uniform row step for
        // the codes): no 64-bit arithmetic per row.  Local row
        // lr = 4 (it GPI + gl) + r; with GPI % 4 == 0 its chunk swizzle
        // ((lr >> 1) ^ (lr >> 2)) & 3 is ((2 gl + r / 2) ^ gl) & 3.  Mp is a
        // multiple of 128, so a half is stored whole or not at all.
        // bf16 output rows: the same split, row h0 + lr at obase + ooff + lr * ldo.
        [[maybe_unused]] uint16_t *const obase = reinterpret_cast<uint16_t *>(p.out) + (row0 + half * 64) * p.ldo;
        [[maybe_unused]] const uint32_t ooff = (uint32_t)(col + 4 * gl * p.ldo);
        [[maybe_unused]] uint8_t *qbase = nullptr, *sbase = nullptr;
        [[maybe_unused]] uint32_t qoff[2] = {0, 0}, soff = 0, sst = 0, qstep = 0;
        [[maybe_unused]] bool qlive = false;
        if constexpr (EPI == QIM_EPI_SWIGLU_QUANT) {
            static_assert(GPI % 8 == 0, "row terms below assume whole groups of 8 row groups");
            const int64_t h0 = row0 + half * 64, kb = col >> 5;
            qlive = h0 < p.Mp;
            sbase = p.out_scales + (h0 >> 7) * (F >> 7) * 512 + ((h0 & 127) >> 5) * 4;
            soff = (uint32_t)((kb >> 2) * 512 + (kb & 3) + (gl & 7) * 64 + (gl >> 3) * 4);
            sst = (uint32_t)((kb & 3) + (gl & 7) * 64 + (gl >> 3) * 4 + ((h0 & 127) >> 5) * 4);
            if (p.out_tiled) {
                const int64_t r0 = h0 & ~int64_t(255);
                const int64_t n = p.Mp - r0 < 256 ? p.Mp - r0 : 256;
                qbase = reinterpret_cast<uint8_t *>(p.out) + r0 * F + (h0 - r0) * 64;
                qstep = 64;
                const uint32_t lo = (uint32_t)((col >> 6) * n * 64 + (col & 15) + gl * 4 * 64);
                const int ch = (int)(col >> 4) & 3;
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) qoff[hb] = lo + ((ch ^ (((2 * gl + hb) ^ gl) & 3)) << 4);
            } else {
                qbase = reinterpret_cast<uint8_t *>(p.out) + h0 * F;
                qstep = (uint32_t)F;
                qoff[0] = qoff[1] = (uint32_t)(col + gl * 4 * F);
            }
        }
        auto pass2 = [&](auto all_rows, auto one_gate) {
            constexpr bool ALL_ROWS = decltype(all_rows)::value, ONE_GATE = decltype(one_gate)::value;
#pragma unroll
        for (int it = 0; it < 16 / GPI; ++it) {
            const int g = it * GPI + gl;  // row group: rows 4g .. 4g+3 of this half
            const uint8_t *src = reg + g * RGS + epi_col_offset<W>(cl * 8);
            uint4 q[4];  // q[k]: columns 8cl + 2k, 2k+1; .x/.y rows 0-1/2-3 of the first, .z/.w of the second
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = *reinterpret_cast<const uint4 *>(src + k * 16);
            uint4 rowv[4];
            {
                uint32_t w[4][4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    w[0][k] = __builtin_amdgcn_perm(q[k].z, q[k].x, 0x05040100u);  // row 0: low halves
                    w[1][k] = __builtin_amdgcn_perm(q[k].z, q[k].x, 0x07060302u);  // row 1: high halves
                    w[2][k] = __builtin_amdgcn_perm(q[k].w, q[k].y, 0x05040100u);
                    w[3][k] = __builtin_amdgcn_perm(q[k].w, q[k].y, 0x07060302u);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) rowv[r] = make_uint4(w[r][0], w[r][1], w[r][2], w[r][3]);
            }
            if constexpr (is_qk_epi<EPI>()) {
                // Q and K head columns: RMSNorm + RoPE of each row's 128-wide
                // head, as k_norm_rope computes it on the stored output.  A
                // wave holds W columns of the head; with W = 64 (quarter tiles)
                // the other half is the partner wave's (wave ^ 1, same rows),
                // whose row sums come through LDS.  The Q/K/V class is uniform
                // over a quarter tile's four waves (one head), so its barriers
                // are too.
                if (qk_cols) {
                    float x[4][8];
                    double ss[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        unpack8(rowv[r], x[r]);
                        ss[r] = group_sum<LPR>(head_sumsq8(x[r]));
                    }
                    if constexpr (W < 128) {
                        static_assert(W == 64, "a head spans two waves at most");
                        double *xs = reinterpret_cast<double *>(lds + 4 * 16 * RGS) + (it & 1) * (4 * GPI * 4);
                        if (cl == 0) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) xs[(wave * GPI + gl) * 4 + r] = ss[r];
                        }
                        __syncthreads();
#pragma unroll
                        for (int r = 0; r < 4; ++r) ss[r] += xs[((wave ^ 1) * GPI + gl) * 4 + r];
                    }
                    const float eps = isq ? p.epsq : p.epsk;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        head_rmsnorm8(x[r], ss[r], 128, eps, wt);
                        head_rope8(x[r], fr[it & 1][r][0], fr[it & 1][r][1]);
                        rowv[r] = pack8(x[r]);
                    }
                    if (it + 1 < 16 / GPI) load_freqs(it + 1, fr[(it + 1) & 1]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t grow = row0 + half * 64 + 4 * g + r;
                const uint4 v = rowv[r];
                if constexpr (EPI == QIM_EPI_SWIGLU_QUANT) {
                    int e;
                    const uint2 c = quantize8_bf16(v, e);
                    // Cached, not streaming: a store instruction covers half of
                    // each 128-byte line (rows 4 apart), and streamed half-line
                    // writes reached memory as 1.5x the code bytes (WRITE_SIZE
                    // 78207 vs 53952 KiB at 4352 x 24576 x 3072); through the
                    // cache the two halves merge.
                    *reinterpret_cast<uint2 *>(qbase + (qoff[r >> 1] + (uint32_t)(4 * it * GPI + r) * qstep)) = c;
                    if ((cl & 3) == 0) {
                        if constexpr (STAGE_SC)
                            sc_stage[sst + (uint32_t)(16 * r + it * (GPI / 8) * 4)] = (uint8_t)e;
                        else
                            sbase[soff + (uint32_t)(16 * r + it * (GPI / 8) * 4)] = (uint8_t)e;
                    }
                } else {
                    if (!ALL_ROWS && grow >= p.M) continue;
                    uint4 o = v;
                    if constexpr (EPI == QIM_EPI_GATED_RESIDUAL) {
                        const uint4 hv = rpre[it][r];
                        const uint4 gv = ONE_GATE ? gpre
                                                  : *reinterpret_cast<const uint4 *>(p.gate + (grow / p.seq) * p.N + col);
                        float y[8], h[8], gg[8], z[8];
                        unpack8(v, y);
                        unpack8(hv, h);
                        unpack8(gv, gg);
#pragma unroll
                        for (int t = 0; t < 8; ++t) z[t] = h[t] + rbf(gg[t] * y[t]);
                        o = pack8(z);
                    }
                    st_out(EPI == EPI_QKV_VT, obase + (ooff + (uint32_t)(4 * it * GPI + r) * (uint32_t)p.ldo), o);
                }
            }
        }
        };
        // Two versions only where pass 2 loads (gated residual, QK): the
        // epilogues without loads wait for nothing there, and a second copy of
        // their loop only lengthens live ranges across the main loop.
        const bool all_rows = row0 + half * 64 + 64 <= p.M;  // uniform
        if constexpr (EPI == QIM_EPI_GATED_RESIDUAL) {
            if (all_rows && gate_once)
                pass2(std::true_type{}, std::true_type{});
            else
                pass2(std::false_type{}, std::false_type{});
        } else if constexpr (is_qk_epi<EPI>()) {
            if (all_rows)
                pass2(std::true_type{}, std::false_type{});
            else
                pass2(std::false_type{}, std::false_type{});
        } else if constexpr (EPI == QIM_EPI_SWIGLU_QUANT) {
            if (qlive) pass2(std::false_type{}, std::false_type{});
        } else {
            pass2(std::false_type{}, std::false_type{});
        }
    }
    if constexpr (STAGE_SC) {
        // Both halves of both waves of each 128-row block staged (a block
        // below Mp is live in both halves: Mp % 128 == 0).
        __syncthreads();
        if ((wave & 1) == 0 && lane < 32 && row0 < p.Mp) {
            uint8_t *chunk = p.out_scales + ((row0 >> 7) * (F >> 7) + (col0 >> 7)) * 512;
            *reinterpret_cast<uint4 *>(chunk + lane * 16) = *reinterpret_cast<const uint4 *>(sc_stage + lane * 16);
        }
    }
    }
}

// ------------------------------------------------------------ tail tiles --
// The tile grid is rarely a whole number of rounds of the CUs (4352 x 12288:
// 816 tiles = 3.19 rounds of 256).  The last r tiles (r <= CUs / 2) are then
// computed as 4r quarter tiles of 128 x 128 by as many extra workgroups, so
// the last round takes about a quarter of a tile's time instead of a whole
// one.  A quarter tile: 4 waves in a 2 x 2 grid, each a 64 x 64 block of 2 x 2
// MFMA tiles, on the same 4-stage LDS ring (half of each operand area used)
// with the same schedule rules.
constexpr int QLOADS_EVEN = 5, QLOADS_ODD = 4;  // per wave per stage: 2 A + 2 B (16 B) + 1 scale (4 B, even stages)

struct QPlan {
    uint32_t a[2], b[2];   // byte offsets into aq / bq (stage 0)
    uint32_t sc;           // byte offset of this wave's 256 scale bytes (stage 0)
    const uint8_t *sc_base;
    uint32_t astep, bstep;
    int wave;
};

__device__ __forceinline__ QPlan make_qplan(const GemmArgs &p, int64_t m0, int64_t n0) {
    QPlan Q;
    const int lane = threadIdx.x & 63;
    Q.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int grp = (Q.wave * 2 + j) * 16;
        Q.a[j] = opnd_offset(m0, grp, lane, p.Mp, p.K, p.a_tiled);
        Q.b[j] = opnd_offset(n0, grp, lane, p.N, p.K, p.b_tiled);
    }
    Q.astep = opnd_step(m0, p.Mp, p.a_tiled);
    Q.bstep = opnd_step(n0, p.N, p.b_tiled);
    // Waves 0, 1 load the A scale chunk of rows [m0, m0 + 128), waves 2, 3 the B chunk.
    const int64_t kt = p.K / 128;
    const int64_t grow = Q.wave < 2 ? m0 / 128 : n0 / 128;
    Q.sc_base = Q.wave < 2 ? p.as : p.bs;
    Q.sc = (uint32_t)(grow * kt * 512 + (Q.wave & 1) * 256 + lane * 4);
    return Q;
}

template <bool SCALES>
__device__ __forceinline__ void issue_qstage(const GemmArgs &p, const QPlan &Q, uint8_t *slot, int s) {
    const uint32_t ka = (uint32_t)s * Q.astep, kb = (uint32_t)s * Q.bstep, base = lds_addr(slot), w2 = Q.wave * 2;
    dma16(p.aq, Q.a[0] + ka, base + (w2 + 0) * 1024);
    dma16(p.aq, Q.a[1] + ka, base + (w2 + 1) * 1024);
    dma16(p.bq, Q.b[0] + kb, base + TILE_BYTES + (w2 + 0) * 1024);
    dma16(p.bq, Q.b[1] + kb, base + TILE_BYTES + (w2 + 1) * 1024);
    if constexpr (SCALES)
        dma4(Q.sc_base, Q.sc + (uint32_t)(s >> 1) * 512,
             base + 2 * TILE_BYTES + (Q.wave < 2 ? 0 : SCALE_BYTES) + (Q.wave & 1) * 256);
}

struct QFrags {
    i32x8_t a[2], b[2];
    uint2 sa, sb;  // scale dwords of row tiles 0, 1
};

// Rows h*64 + t*32 + lr (t = 0, 1) of a 128-row scale chunk: dwords at
// lr*16 + (2h + t)*4, contiguous.
__device__ __forceinline__ uint2 read_qscales(const uint8_t *base, int h, int lr) {
    return *reinterpret_cast<const uint2 *>(base + lr * 16 + h * 8);
}

__device__ __forceinline__ void read_qfrags(const uint8_t *slot, int wm, int wn, int lr, int kh, QFrags &f, bool scales) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        f.a[t] = read_tile(slot, wm * 64 + t * 32 + lr, kh);
        f.b[t] = read_tile(slot + TILE_BYTES, wn * 64 + t * 32 + lr, kh);
    }
    if (scales) {
        f.sa = read_qscales(slot + 2 * TILE_BYTES, wm, lr);
        f.sb = read_qscales(slot + 2 * TILE_BYTES + SCALE_BYTES, wn, lr);
    }
}

template <int PAR>
__device__ __forceinline__ void qstep(const GemmArgs &p, const QPlan &Q, uint8_t *lds, int s, int S,
                                      f32x16_t (&acc)[2][2], const QFrags &cur, QFrags &nxt, int wm, int wn, int lr,
                                      int kh) {
    const int sa[2] = {(int)(cur.sa.x >> (8 * kh)), (int)(cur.sa.y >> (8 * kh))};
    const int sb[2] = {(int)(cur.sb.x >> (8 * kh)), (int)(cur.sb.y >> (8 * kh))};
#define QIM_QMF(i, j)                                                                                          \
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(cur.a[i], cur.b[j], acc[i][j], 0, 0, PAR * 2, \
                                                                sa[i], PAR * 2, sb[j])
    QIM_QMF(0, 0);
    QIM_SCHED();
    wait_vmcnt<QLOADS_EVEN + QLOADS_ODD>();
    block_barrier();
    QIM_SCHED();
    issue_qstage<PAR == 0>(p, Q, lds + (s & 3) * STAGE_BYTES, s + 4 < S ? s + 4 : S - 1);
    QIM_SCHED();
    QIM_QMF(0, 1);
    QIM_SCHED();
    if constexpr (PAR == 0) {
        read_qfrags(lds + ((s + 1) & 3) * STAGE_BYTES, wm, wn, lr, kh, nxt, false);
        nxt.sa = cur.sa;
        nxt.sb = cur.sb;
    } else {
        read_qfrags(lds + ((s + 1) & 3) * STAGE_BYTES, wm, wn, lr, kh, nxt, true);
    }
    QIM_SCHED();
    QIM_QMF(1, 0);
    QIM_QMF(1, 1);
    QIM_SCHED();
#undef QIM_QMF
}

// fp32 words of one split-K partial: a quarter tile's 4 waves x 2 x 2 MFMA
// tiles x 16 accumulators x 64 lanes.  Each MFMA tile's 16 accumulators are
// four groups of 4 (r = 4 g .. 4 g + 3), a group stored as 64 lanes x 16 bytes,
// so each 16-byte store and load instruction covers 1 KiB contiguous.
constexpr int QPART_WORDS = 4 * 2 * 2 * 16 * 64;

// Group 0 of the lane's accumulators of MFMA tile (i, j) of a wave; group g
// is at [64 * g].
__device__ __forceinline__ float4 *qpart(const GemmArgs &p, int unit, int wave, int i, int j, int lane) {
    return reinterpret_cast<float4 *>(p.ws + (int64_t)unit * QPART_WORDS) + ((wave * 2 + i) * 2 + j) * 256 + lane;
}

// Corner of quarter tile q (of the last whole tiles, or a 128-row piece of a
// last 128-column block).
__device__ __forceinline__ void quarter_origin(const GemmArgs &p, int q, int64_t &m0, int64_t &n0) {
    if (q < p.quarters) {  // a quarter of one of the last whole tiles
        const int tile = p.main_tiles + q / 4, quarter = q & 3;
        int tm, tn;
        tile_coords(p, tile, tm, tn);
        m0 = (int64_t)tm * BM + (quarter >> 1) * 128;
        n0 = (int64_t)tn * BN + (quarter & 1) * 128;
    } else {               // 128 rows of the last 128-column block
        m0 = (int64_t)(q - p.quarters) * 128;
        n0 = (int64_t)p.tiles_n * BN;
    }
}

// Quarter-tile unit u: quarter tile u % quarters over K-stage pairs
// [kp * P / ksplit, (kp + 1) * P / ksplit), kp = u / quarters, P = K / 128 (the
// whole of K when ksplit == 1).  Stages keep their ring slot (s & 3) and
// their parity (even stages carry the 128-K scale group).
template <int EPI>
__device__ __forceinline__ void quarter_tile(const GemmArgs &p, uint8_t *lds, uint8_t *tab, int u) {
    const int split = p.ksplit > 1 ? p.ksplit : 1;
    const int q = split > 1 ? u % p.quarters : u, kp = split > 1 ? u / p.quarters : 0;
    int64_t m0, n0;
    quarter_origin(p, q, m0, n0);
    if (m0 >= p.Mp) return;  // padding rows only (whole workgroup)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, kh = lane >> 5;
    const int P = (int)(p.K / (2 * BK));
    const int sb = 2 * (kp * P / split), se = 2 * ((kp + 1) * P / split);
    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16_t{};
    const QPlan Q = make_qplan(p, m0, n0);
    issue_qstage<true>(p, Q, lds + (sb & 3) * STAGE_BYTES, sb);
    issue_qstage<false>(p, Q, lds + ((sb + 1) & 3) * STAGE_BYTES, sb + 1);
    issue_qstage<true>(p, Q, lds + ((sb + 2) & 3) * STAGE_BYTES, sb + 2 < se ? sb + 2 : se - 1);
    issue_qstage<false>(p, Q, lds + ((sb + 3) & 3) * STAGE_BYTES, sb + 3 < se ? sb + 3 : se - 1);
    if constexpr (ring_offset<EPI>() > 0) fill_silu_table(tab);
    wait_vmcnt<QLOADS_ODD + QLOADS_EVEN + QLOADS_ODD>();  // stage sb landed
    block_barrier();
    QFrags fa, fb;
    read_qfrags(lds + (sb & 3) * STAGE_BYTES, wm, wn, lr, kh, fa, true);
    for (int s = sb; s < se; s += 2) {
        qstep<0>(p, Q, lds, s, se, acc, fa, fb, wm, wn, lr, kh);
        qstep<1>(p, Q, lds, s + 1, se, acc, fb, fa, wm, wn, lr, kh);
    }
    wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (split > 1) {  // a partial sum: to the workspace, the epilogue runs in k_mx_gemm_tail
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float4 *w = qpart(p, u, wave, i, j, lane);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    w[64 * g] = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                            acc[i][j][4 * g + 3]);
            }
        return;
    }
    block_barrier();
    epilogue<EPI, 2, 2>(p, acc, lds, tab, m0 + wm * 64, n0 + wn * 64, lane, wave);
}

template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_mx_gemm(GemmArgs p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    // The SwiGLU kernels keep their SiLU table in the first 16 KiB; the ring
    // (and the epilogue's staging) follows it.
    uint8_t *const tab = smem, *const lds = smem + ring_offset<EPI>();
    if ((int)blockIdx.x >= p.main_tiles) {  // a quarter tile of the last partial round
        quarter_tile<EPI>(p, lds, tab, (int)blockIdx.x - p.main_tiles);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    tile_of(p, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int S = (int)(p.K / BK);
    const int lr = lane & 31, kh = lane >> 5;

    f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

    const LoadPlan L = make_plan(p, m0, n0);
    issue_stage<true>(p, L, lds, 0);
    issue_stage<false>(p, L, lds + STAGE_BYTES, 1 < S ? 1 : S - 1);
    issue_stage<true>(p, L, lds + 2 * STAGE_BYTES, 2 < S ? 2 : S - 1);
    issue_stage<false>(p, L, lds + 3 * STAGE_BYTES, 3 < S ? 3 : S - 1);
    if constexpr (ring_offset<EPI>() > 0) fill_silu_table(tab);
    wait_vmcnt<LOADS_ODD + LOADS_EVEN + LOADS_ODD>();  // stage 0 landed
    block_barrier();
    Frags fa, fb;
    read_frags(lds, wm, wn, lr, kh, fa);

    // S = K / 64 is even (K % 128 == 0): stages come in (even, odd) pairs.
    for (int s = 0; s < S; s += 2) {
        pipeline_step<0>(p, L, lds, s, S, acc, fa, fb, wm, wn, lr, kh);
        pipeline_step<1>(p, L, lds, s + 1, S, acc, fb, fa, wm, wn, lr, kh);
    }
    wait_vmcnt<0>();  // the clamped tail loads must land before LDS is reused
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    block_barrier();

    epilogue<EPI, 4, 4>(p, acc, lds, tab, m0 + wm * 128, n0 + wn * 128, lane, wave);
}

// The split-K tail's second launch: one one-wave workgroup per 64 x 64 block
// of a quarter tile (workgroup 4 q + w does wave w's block of quarter q) sums
// its ksplit partials in order kp = 0, 1, ... (the register layout the
// quarter tile's wave wrote, each partial's 16 loads in flight together) and
// runs that block's epilogue.  At 64 quarter tiles x 4 splits this takes
// 6.8 us, against 7.8 us with one four-wave workgroup per quarter tile.
constexpr int TAIL_LDS_BYTES = 16 * (64 * 8 + 8 * 16);  // epilogue<EPI, 2, 2>'s staging of one wave (TJ = 2, bf16 rows)

template <int EPI>
__global__ __launch_bounds__(64) void k_mx_gemm_tail(GemmArgs p) {
    static_assert(ring_offset<EPI>() == 0, "the split tail runs the plain, bias and gated-residual epilogues");
    __shared__ __attribute__((aligned(16))) uint8_t lds[TAIL_LDS_BYTES];
    const int q = (int)(blockIdx.x >> 2);
    int64_t m0, n0;
    quarter_origin(p, q, m0, n0);
    if (m0 >= p.Mp) return;
    const int lane = threadIdx.x, wave = (int)(blockIdx.x & 3);
    const int wm = wave >> 1, wn = wave & 1;
    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float4 *w = qpart(p, q, wave, i, j, lane);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 v = w[64 * g];
                acc[i][j][4 * g] = v.x;
                acc[i][j][4 * g + 1] = v.y;
                acc[i][j][4 * g + 2] = v.z;
                acc[i][j][4 * g + 3] = v.w;
            }
        }
    for (int kp = 1; kp < p.ksplit; ++kp) {
        // all 16 loads of a partial in flight before its adds
        const int u = kp * p.quarters + q;
        float4 v[2][2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float4 *w = qpart(p, u, wave, i, j, lane);
#pragma unroll
                for (int g = 0; g < 4; ++g) v[i][j][g] = w[64 * g];
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    acc[i][j][4 * g] += v[i][j][g].x;
                    acc[i][j][4 * g + 1] += v[i][j][g].y;
                    acc[i][j][4 * g + 2] += v[i][j][g].z;
                    acc[i][j][4 * g + 3] += v[i][j][g].w;
                }
    }
    epilogue<EPI, 2, 2>(p, acc, lds, nullptr, m0 + wm * 64, n0 + wn * 64, lane, 0);  // LDS region 0: its own
}

// CUs the work split plans for: the current device's, or MI355X's 256 when no
// device answers (sizes queried without a GPU).
static int64_t plan_cus() {
    const int c = device_cus();
    return c > 0 ? c : 256;
}

// Whole tiles to launch: all of them, or all but the last r when the last
// round of the CUs would hold r <= CUs / 2 tiles (those become 4r quarters).
static int64_t main_tile_count(int64_t tiles) {
    const int64_t cus = plan_cus();
    if (tiles <= cus) return tiles;
    const int64_t r = tiles % cus;
    return (r > 0 && 2 * r <= cus) ? tiles - r : tiles;
}

template <int EPI>
static int launch_gemm(const GemmArgs &a, hipStream_t st) {
    static std::atomic<bool> configured[QIM_MAX_DEVICES] = {};
    constexpr int lds_bytes = LDS_BYTES + ring_offset<EPI>();
    if (const int rc = reserve_lds(reinterpret_cast<const void *>(&k_mx_gemm<EPI>), lds_bytes, configured,
                                   "qim_mxfp8_gemm"))
        return rc;
    const int64_t half_column = a.tiles_n * BN < a.N ? (a.Mp + 127) / 128 : 0;
    const int64_t split = a.ksplit > 1 ? a.ksplit : 1;
    const int64_t grid = a.main_tiles + a.quarters * split + half_column;
    launch(k_mx_gemm<EPI>, dim3((unsigned)grid), dim3(256), lds_bytes, st, a);
    if constexpr (ring_offset<EPI>() == 0 && EPI != QIM_EPI_QK_NORM_ROPE && EPI != EPI_QKV_VT) {
        if (split > 1) launch(k_mx_gemm_tail<EPI>, dim3((unsigned)a.quarters * 4), dim3(64), 0, st, a);
    }
    return QIM_OK;
}

// K-splits of the tail's quarter tiles: as many as fill the CUs' one round
// (quarters * ksplit <= CUs), at most one stage pair each and at most 8; 1
// (no split) when the quarters alone hold more than half the CUs, when a last
// 128-column block is there, or for an epilogue other than the plain, bias
// and gated-residual ones.
static int tail_ksplit(int64_t quarters, bool half_column, int epilogue, int64_t K) {
    const int64_t cus = plan_cus();
    if (quarters <= 0 || half_column) return 1;
    if (epilogue != QIM_EPI_NONE && epilogue != QIM_EPI_BIAS && epilogue != QIM_EPI_GATED_RESIDUAL) return 1;
    int64_t k = cus / quarters;
    const int64_t pairs = K / (2 * BK);
    if (k > pairs) k = pairs;
    if (k > 8) k = 8;
    return k >= 2 ? (int)k : 1;
}

}  // namespace qim

using namespace qim;

// Operands of the QK-norm-RoPE epilogue (qim_mxfp8_gemm_qk_norm_rope).
struct QKNormRope {
    const void *wq, *wk, *freqs;
    float epsq, epsk;
    int64_t heads;
    void *vt;  // V^T tiles instead of the V columns of out, or null
};

// Quarter tiles and K-splits of the tail for a problem shape (tail_ksplit).
static void tail_plan(int64_t M, int64_t N, int64_t K, int epilogue, int64_t &quarters, int &ksplit) {
    const int64_t Mp = (M + 127) / 128 * 128, tiles_m = (Mp + BM - 1) / BM, tiles_n = N / BN;
    const int64_t tiles = tiles_m * tiles_n;
    quarters = 4 * (tiles - main_tile_count(tiles));
    ksplit = tail_ksplit(quarters, tiles_n * BN < N, epilogue, K);
}

static int gemm_run(const void *aq, const void *as, const void *bq, const void *bs, int64_t M, int64_t N, int64_t K,
                    int epilogue, int layouts, const void *bias, const void *gate, const void *res, int64_t seq,
                    void *out, int64_t ldo, void *out_scales, const QKNormRope *qk, void *stream,
                    void *ws = nullptr, int64_t ws_bytes = 0) {
    QIM_REQUIRE(aq && as && bq && bs && out, QIM_ERR_ARG, "qim_mxfp8_gemm: null pointer");
    constexpr int KNOWN = QIM_GEMM_A_TILED | QIM_GEMM_B_TILED | QIM_GEMM_OUT_TILED | QIM_GEMM_OUT_F32 | QIM_GEMM_OUT_F16;
    QIM_REQUIRE((layouts & ~KNOWN) == 0, QIM_ERR_ARG, "qim_mxfp8_gemm: unknown layout flags 0x%x", layouts);
    const int out_format = layouts & (QIM_GEMM_OUT_F32 | QIM_GEMM_OUT_F16);
    QIM_REQUIRE(out_format != (QIM_GEMM_OUT_F32 | QIM_GEMM_OUT_F16), QIM_ERR_ARG,
                "qim_mxfp8_gemm: QIM_GEMM_OUT_F32 and QIM_GEMM_OUT_F16 exclude each other");
    QIM_REQUIRE(!out_format || epilogue == QIM_EPI_NONE, QIM_ERR_ARG,
                "qim_mxfp8_gemm: an fp32 / fp16 output is available with QIM_EPI_NONE only");
    QIM_REQUIRE(!(layouts & QIM_GEMM_OUT_TILED) || epilogue == QIM_EPI_SWIGLU_QUANT, QIM_ERR_ARG,
                "qim_mxfp8_gemm: a tiled output needs the quantized SwiGLU epilogue");
    QIM_REQUIRE(M > 0 && N > 0 && K > 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: empty problem");
    QIM_REQUIRE(K % 128 == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: K=%lld is not a multiple of 128", (long long)K);
    QIM_REQUIRE(N % 128 == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: N=%lld is not a multiple of 128", (long long)N);
    const int64_t Mp = (M + 127) / 128 * 128;
    const int64_t tiles_m = (Mp + BM - 1) / BM, tiles_n = N / BN;
    QIM_REQUIRE(4 * tiles_m * tiles_n < (1ll << 31), QIM_ERR_SHAPE, "qim_mxfp8_gemm: too many tiles");
    QIM_REQUIRE(aligned16(aq) && aligned16(bq) && aligned16(as) && aligned16(bs) && aligned16(out) &&
                    (!res || aligned16(res)) && (!gate || aligned16(gate)) && (!out_scales || aligned16(out_scales)),
                QIM_ERR_LAYOUT, "qim_mxfp8_gemm: operands must be 16-byte aligned");
    QIM_REQUIRE(epilogue == QIM_EPI_SWIGLU_QUANT || ldo % 8 == 0, QIM_ERR_LAYOUT,
                "qim_mxfp8_gemm: ldo=%lld is not a multiple of 8", (long long)ldo);
    // The epilogues address a 64-row half's outputs with 32-bit offsets.
    QIM_REQUIRE(ldo < (1ll << 25), QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld too large", (long long)ldo);
    QIM_REQUIRE(Mp / 128 < (1ll << 30), QIM_ERR_SHAPE, "qim_mxfp8_gemm: M=%lld too large", (long long)M);
    QIM_REQUIRE(Mp * K < (1ll << 31) && N * K < (1ll << 31), QIM_ERR_SHAPE,
                "qim_mxfp8_gemm: operands above 2 GiB are not supported");
    GemmArgs a{(const uint8_t *)aq, (const uint8_t *)as, (const uint8_t *)bq, (const uint8_t *)bs, M, Mp, N, K,
               (const uint16_t *)bias, (const uint16_t *)gate, (const uint16_t *)res, seq > 0 ? seq : M, out, ldo,
               (uint8_t *)out_scales, (int)tiles_m, (int)tiles_n, 0, 0,
               (layouts & QIM_GEMM_A_TILED) != 0, (layouts & QIM_GEMM_B_TILED) != 0,
               (layouts & QIM_GEMM_OUT_TILED) != 0,
               nullptr, nullptr, nullptr, 0.0f, 0.0f, 0, 0, nullptr, 0};
    if (qk) {
        a.wq = (const uint16_t *)qk->wq;
        a.wk = (const uint16_t *)qk->wk;
        a.freqs = (const float *)qk->freqs;
        a.epsq = qk->epsq;
        a.epsk = qk->epsk;
        a.q_cols = qk->heads * 128;
        a.qk_cols = 2 * qk->heads * 128;
        a.vt = static_cast<uint16_t *>(qk->vt);
        a.vt_nkb = seq / 64;
    }
    const int64_t tiles = tiles_m * tiles_n;
    a.main_tiles = (int)main_tile_count(tiles);
    a.quarters = (int)(4 * (tiles - a.main_tiles));
    if (ws && !qk) {
        int64_t quarters;
        int ksplit;
        tail_plan(M, N, K, epilogue, quarters, ksplit);
        QIM_REQUIRE(aligned16(ws), QIM_ERR_LAYOUT, "qim_mxfp8_gemm_ws: ws must be 16-byte aligned");
        if (ksplit > 1 && ws_bytes >= quarters * ksplit * (int64_t)QPART_WORDS * 4) {
            a.ws = static_cast<float *>(ws);
            a.ksplit = ksplit;
        }
    }
    int rc;
    switch (epilogue) {
        case QIM_EPI_NONE:
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            if (out_format == QIM_GEMM_OUT_F32)
                rc = launch_gemm<EPI_F32>(a, as_stream(stream));
            else if (out_format == QIM_GEMM_OUT_F16)
                rc = launch_gemm<EPI_F16>(a, as_stream(stream));
            else
                rc = launch_gemm<QIM_EPI_NONE>(a, as_stream(stream));
            break;
        case QIM_EPI_BIAS:
            QIM_REQUIRE(bias, QIM_ERR_ARG, "qim_mxfp8_gemm: bias epilogue without bias");
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            rc = launch_gemm<QIM_EPI_BIAS>(a, as_stream(stream));
            break;
        case QIM_EPI_GATED_RESIDUAL:
            QIM_REQUIRE(gate && res, QIM_ERR_ARG, "qim_mxfp8_gemm: gated residual needs gate and res");
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            rc = launch_gemm<QIM_EPI_GATED_RESIDUAL>(a, as_stream(stream));
            break;
        case QIM_EPI_SWIGLU:
            QIM_REQUIRE(N % 512 == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: SwiGLU needs N %% 512 == 0");
            QIM_REQUIRE(ldo >= N / 2, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N/2", (long long)ldo);
            rc = launch_gemm<QIM_EPI_SWIGLU>(a, as_stream(stream));
            break;
        case QIM_EPI_SWIGLU_QUANT:
            QIM_REQUIRE(N % 512 == 0, QIM_ERR_SHAPE, "qim_mxfp8_gemm: SwiGLU needs N %% 512 == 0");
            QIM_REQUIRE(out_scales, QIM_ERR_ARG, "qim_mxfp8_gemm: quantized output needs out_scales");
            rc = launch_gemm<QIM_EPI_SWIGLU_QUANT>(a, as_stream(stream));
            break;
        case QIM_EPI_QK_NORM_ROPE:
            QIM_REQUIRE(qk, QIM_ERR_ARG, "qim_mxfp8_gemm: the QK epilogue is qim_mxfp8_gemm_qk_norm_rope's");
            QIM_REQUIRE(ldo >= N, QIM_ERR_LAYOUT, "qim_mxfp8_gemm: ldo=%lld < N", (long long)ldo);
            rc = qk->vt ? launch_gemm<EPI_QKV_VT>(a, as_stream(stream))
                        : launch_gemm<QIM_EPI_QK_NORM_ROPE>(a, as_stream(stream));
            break;
        default:
            return fail(QIM_ERR_ARG, "qim_mxfp8_gemm: unknown epilogue %d", epilogue);
    }
    return rc ? rc : check_launch("qim_mxfp8_gemm");
}

extern "C" int qim_mxfp8_gemm(const void *aq, const void *as, const void *bq, const void *bs, int64_t M, int64_t N,
                              int64_t K, int epilogue, const void *bias, const void *gate, const void *res,
                              int64_t seq, void *out, int64_t ldo, void *out_scales, void *stream) {
    return qim_mxfp8_gemm_ex(aq, as, bq, bs, M, N, K, epilogue, 0, bias, gate, res, seq, out, ldo, out_scales,
                             stream);
}

extern "C" int qim_mxfp8_gemm_ex(const void *aq, const void *as, const void *bq, const void *bs, int64_t M,
                                 int64_t N, int64_t K, int epilogue, int layouts, const void *bias, const void *gate,
                                 const void *res, int64_t seq, void *out, int64_t ldo, void *out_scales,
                                 void *stream) {
    return gemm_run(aq, as, bq, bs, M, N, K, epilogue, layouts, bias, gate, res, seq, out, ldo, out_scales, nullptr,
                    stream);
}

extern "C" int64_t qim_mxfp8_gemm_ws_bytes(int64_t M, int64_t N, int64_t K, int epilogue) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 || N % 128) return 0;
    int64_t quarters;
    int ksplit;
    tail_plan(M, N, K, epilogue, quarters, ksplit);
    return ksplit > 1 ? quarters * ksplit * (int64_t)QPART_WORDS * 4 : 0;
}

extern "C" int qim_mxfp8_gemm_ws(const void *aq, const void *as, const void *bq, const void *bs, int64_t M,
                                 int64_t N, int64_t K, int epilogue, int layouts, const void *bias, const void *gate,
                                 const void *res, int64_t seq, void *out, int64_t ldo, void *out_scales, void *ws,
                                 int64_t ws_bytes, void *stream) {
    return gemm_run(aq, as, bq, bs, M, N, K, epilogue, layouts, bias, gate, res, seq, out, ldo, out_scales, nullptr,
                    stream, ws, ws_bytes);
}

static int qk_norm_rope_run(const char *who, const void *aq, const void *as, const void *bq, const void *bs, int64_t M,
                            int64_t K, int64_t H, int layouts, const void *wq, const void *wk, const void *freqs,
                            int64_t seq, float epsq, float epsk, void *out, int64_t ldo, void *vt, void *stream) {
    QIM_REQUIRE(wq && wk && freqs, QIM_ERR_ARG, "%s: null pointer", who);
    QIM_REQUIRE(H > 0 && H % 2 == 0 && H < (1 << 20), QIM_ERR_SHAPE,
                "%s: H=%lld must be even (N = 3 H 128 %% 256 == 0)", who, (long long)H);
    QIM_REQUIRE(seq > 0 && seq < (1ll << 31) && M < (1ll << 31), QIM_ERR_SHAPE, "%s: seq=%lld / M=%lld out of range",
                who, (long long)seq, (long long)M);
    QIM_REQUIRE(aligned16(wq) && aligned16(wk) && aligned16(freqs) && aligned16(vt), QIM_ERR_LAYOUT,
                "%s: wq, wk, freqs (and vt) must be 16-byte aligned", who);
    QIM_REQUIRE((layouts & QIM_GEMM_OUT_TILED) == 0, QIM_ERR_ARG, "%s: the output is bf16 (no tiled output)", who);
    const QKNormRope qk{wq, wk, freqs, epsq, epsk, H, vt};
    return gemm_run(aq, as, bq, bs, M, 3 * H * 128, K, QIM_EPI_QK_NORM_ROPE, layouts, nullptr, nullptr, nullptr, seq,
                    out, ldo, nullptr, &qk, stream);
}

extern "C" int qim_mxfp8_gemm_qk_norm_rope(const void *aq, const void *as, const void *bq, const void *bs,
                                           int64_t M, int64_t K, int64_t H, int layouts, const void *wq,
                                           const void *wk, const void *freqs, int64_t seq, float epsq, float epsk,
                                           void *out, int64_t ldo, void *stream) {
    return qk_norm_rope_run("qim_mxfp8_gemm_qk_norm_rope", aq, as, bq, bs, M, K, H, layouts, wq, wk, freqs, seq, epsq,
                            epsk, out, ldo, nullptr, stream);
}

extern "C" int qim_mxfp8_gemm_qk_norm_rope_vt(const void *aq, const void *as, const void *bq, const void *bs,
                                              int64_t M, int64_t K, int64_t H, int layouts, const void *wq,
                                              const void *wk, const void *freqs, int64_t seq, float epsq,
                                              float epsk, void *out, int64_t ldo, void *vt, void *stream) {
    QIM_REQUIRE(vt, QIM_ERR_ARG, "qim_mxfp8_gemm_qk_norm_rope_vt: null vt");
    QIM_REQUIRE(seq > 0 && seq % 64 == 0 && M % seq == 0, QIM_ERR_SHAPE,
                "qim_mxfp8_gemm_qk_norm_rope_vt: seq=%lld must be a multiple of 64 dividing M=%lld", (long long)seq,
                (long long)M);
    return qk_norm_rope_run("qim_mxfp8_gemm_qk_norm_rope_vt", aq, as, bq, bs, M, K, H, layouts, wq, wk, freqs, seq,
                            epsq, epsk, out, ldo, vt, stream);
}
