// Attention core of the MMDiT block: O = softmax(Q K^T * scale) V per (batch,
// head), head dim 128, bf16 in and out, fp32 scores, softmax statistics and
// accumulation, in the online-softmax (flash) form: K/V are streamed in blocks
// of 64 keys and never materialise the score matrix.  No mask (bidirectional
// attention over [prefix + target] keys, the reference's SDPA call of
// optimizations/quantized_decode.py:70-77).
//
// Transposed formulation on v_mfma_f32_32x32x16_bf16: S^T = K Q^T (32 keys x 32
// queries per MFMA tile) and O^T = V^T P^T (32 head dims x 32 queries), so
// lane l owns query l % 32 in both: the running max and sum and the rescale
// of O are lane-local; the two half-waves, which hold different keys of one
// query, exchange one value per block.  An S^T accumulator is already the B
// operand of the P V product: lane (q, h = l / 32) holds keys
// {8(i/4) + 4h + i%4}, i = 0..15, of its 32-key tile, so values 0-7 are its 8
// keys of the first 16-key MFMA step and 8-15 of the second.  V^T is stored
// with each 16-key group in that order ([0-3, 8-11 | 4-7, 12-15]), so the A
// operand of lane (d, h) is one contiguous 16-byte read.  (An MFMA pairs the
// K slots of A and B by position, so any key order works as long as A and B
// agree.)
//
// V^T comes from a transpose pass (k_attn_vt) into a workspace: one 16 KiB
// tile per (batch, head, 64-key block), 128 rows (d) of 64 keys, with the
// 16-byte chunk c of row d at chunk c ^ ((d >> 1) & 7) (conflict-free reads of
// 16 lanes with consecutive d).  K is loaded straight from the K tensor, with
// chunk c of key r at chunk c ^ (r & 15) in LDS.
#include "qim_attention.h"
#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16a_t __attribute__((ext_vector_type(16)));

constexpr int ATT_D = 128;          // head dim
constexpr int ATT_KB = 64;          // keys per block
constexpr int ATT_BQ = 256;         // queries per workgroup: 4 waves x 2 tiles of 32
constexpr int ATT_TILE = ATT_KB * ATT_D * 2;  // 16 KiB: one K block or one V^T block
constexpr int ATT_STAGE = 2 * ATT_TILE;       // K + V^T
constexpr int ATT_NSTAGE = 4;
constexpr int ATT_LDS = ATT_NSTAGE * ATT_STAGE;  // 128 KiB

struct AttnArgs {
    const uint16_t *q, *k;
    const uint16_t *vt;  // V^T tiles
    uint16_t *o;
    int64_t ldq, ldk, ldo;  // elements between consecutive tokens
    int S, T, H, nkb;       // queries, keys, heads, key blocks
    int nq;                 // query blocks per (batch, head)
    // Work split (att_plan): workgroups [0, nfull) each run one whole work item
    // (query block, head, batch); the remaining ntail items run as nsplit
    // chunks of kbc key blocks each, writing partial results (part_o: each
    // chunk's normalised output rows O_c / l_c in bf16, part_ml: (m, l) per
    // query in fp32) that k_attn_merge combines.
    int nfull, ntail, nsplit, kbc;
    uint16_t *part_o;
    float *part_ml;
    float scale_log2e;
    // MXFP8 output (qim_attention_mxfp8) instead of o: E4M3 codes of the
    // (B*S, H*128) output, row-major or in the GEMM's tiled layout over Mp
    // rows (mxt_offset), and its swizzled E8M0 scales.
    uint8_t *qcodes, *qscales;
    int64_t Mp;
    int tiled;
};

// One query row's 4-column group of an MXFP8 output: code byte offset.
__device__ __forceinline__ int64_t att_code_offset(const AttnArgs &p, int64_t row, int64_t k) {
    const int64_t K = (int64_t)p.H * ATT_D;
    return p.tiled ? mxt_offset(row, k, p.Mp, K) : row * K + k;
}

// ---------------------------------------------------------- V transpose --
// One workgroup per (batch, head, key block): 64 keys x 128 d through LDS.
__global__ __launch_bounds__(256) void k_attn_vt(const uint16_t *__restrict__ v, int64_t ldv, uint16_t *__restrict__ vt,
                                                 int T, int H, int nkb) {
    __shared__ uint16_t s[ATT_KB][ATT_D + 8];  // +8: stagger rows across banks
    const int kb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    // Load: 64 keys x 16 chunks of 16 bytes; zeros past the last key.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + tid, key = idx >> 4, c = idx & 15;
        const int t = kb * ATT_KB + key;
        uint4 x = make_uint4(0, 0, 0, 0);
        if (t < T) x = ld_nt(v + ((int64_t)b * T + t) * ldv + (int64_t)h * ATT_D + c * 8);
        *reinterpret_cast<uint4 *>(&s[key][c * 8]) = x;
    }
    __syncthreads();
    // Store: 128 rows (d) x 8 chunks; physical chunk pc of row d holds logical
    // chunk c = pc ^ ((d >> 1) & 7): keys 16g + [4hh, 4hh+4) and 16g + 8 + [4hh, 4hh+4)
    // with g = c / 2, hh = c % 2.
    uint16_t *tile = vt + (((int64_t)b * H + h) * nkb + kb) * (ATT_KB * ATT_D);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + tid, d = idx >> 3, pc = idx & 7;
        const int c = pc ^ ((d >> 1) & 7), g = c >> 1, hh = c & 1;
        const int k0 = 16 * g + 4 * hh;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int key_lo = (e < 2) ? k0 + 2 * e : k0 + 8 + 2 * (e - 2);
            w[e] = (uint32_t)s[key_lo][d] | ((uint32_t)s[key_lo + 1][d] << 16);
        }
        *reinterpret_cast<uint4 *>(tile + d * ATT_KB + pc * 8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// ------------------------------------------------------------- forward --
__device__ __forceinline__ void att_dma16(const void *base, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds_addr)
                 : "memory");
}
__device__ __forceinline__ uint32_t att_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <int N>
__device__ __forceinline__ void att_wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4 &u) { return __builtin_bit_cast(bf16x8_t, u); }

// DMA addressing of one wave's share of a key block: 4 instructions of K and
// 4 of V^T (1 KiB each).  K instruction j (n = 4 wave + j) covers keys
// 4n..4n+3 of the block: lane i lands at LDS row r = 4n + i/16, physical chunk
// i % 16, whose source is the key's logical chunk (i % 16) ^ (r & 15).  Per
// block only the (wave-uniform) base address moves; the per-lane offsets are
// fixed, with a second set for the last block whose rows past T - 1 are
// clamped to T - 1 (their scores are masked).  V^T tiles are copied as they are.
struct AttLoader {
    const uint8_t *k0;            // K row 0 of this (batch, head)
    const uint8_t *vt0;           // V^T tile 0 of this (batch, head)
    int64_t kstep;                // bytes of K per key block
    uint32_t koff[4], klast[4];   // per-lane K offsets: full blocks, the last block
    uint32_t voff;                // per-lane V^T offset
    int lastb;
};

__device__ __forceinline__ AttLoader att_loader(const AttnArgs &p, int b, int h, int wave, int lane) {
    AttLoader L;
    L.k0 = reinterpret_cast<const uint8_t *>(p.k + (int64_t)b * p.T * p.ldk + (int64_t)h * ATT_D);
    L.vt0 = reinterpret_cast<const uint8_t *>(p.vt + ((int64_t)b * p.H + h) * p.nkb * (ATT_KB * ATT_D));
    L.kstep = (int64_t)ATT_KB * p.ldk * 2;
    L.lastb = p.nkb - 1;
    const int rmax = p.T - 1 - L.lastb * ATT_KB;  // last valid row of the last block
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * (wave * 4 + j) + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        const int rl = r < rmax ? r : rmax;
        L.koff[j] = (uint32_t)(((int64_t)r * p.ldk + c * 8) * 2);
        L.klast[j] = (uint32_t)(((int64_t)rl * p.ldk + c * 8) * 2);
    }
    L.voff = (uint32_t)(wave * 4096 + lane * 16);
    return L;
}

// Issue key block kb (clamped by the caller to the last block) into an LDS slot.
__device__ __forceinline__ void att_issue(const AttLoader &L, int wave, uint8_t *slot, int kb) {
    const uint32_t base = att_lds_addr(slot) + wave * 4096;
    const uint8_t *kp = L.k0 + kb * L.kstep;
    if (kb == L.lastb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) att_dma16(kp, L.klast[j], base + j * 1024);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) att_dma16(kp, L.koff[j], base + j * 1024);
    }
    const uint8_t *tile = L.vt0 + (int64_t)kb * ATT_TILE;
#pragma unroll
    for (int j = 0; j < 4; ++j) att_dma16(tile, L.voff + j * 1024, base + ATT_TILE + j * 1024);
}

// K fragments of one 32-key sub-block (half hb of an LDS key block), all 8
// head-dim steps: lane (r = key % 32, hf) reads d [16j + 8hf, +8) of key r.
__device__ __forceinline__ void att_read_k(uint4 (&kf)[8], const uint8_t *kt_lds, int hb, int lq, int hf) {
    const int r = 32 * hb + lq;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        kf[j] = *reinterpret_cast<const uint4 *>(kt_lds + r * 256 + (((2 * j + hf) ^ (r & 15)) * 16));
}

// V^T fragments of one 32-key sub-block: lane (d % 32, hf) reads the 8 keys of
// 16-key step kk = 2hb + u that pair with its P^T operand, head dims 32dt + d % 32.
__device__ __forceinline__ void att_read_v(uint4 (&vf)[2][4], const uint8_t *vt_lds, int hb, int lq, int hf) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d = 32 * dt + lq, kk = 2 * hb + u;
            vf[u][dt] = *reinterpret_cast<const uint4 *>(vt_lds + d * (ATT_KB * 2) + (((2 * kk + hf) ^ ((d >> 1) & 7)) * 16));
        }
}

// S^T of one 32-query tile over one 32-key sub-block: 8 MFMAs.
__device__ __forceinline__ void att_scores(f32x16a_t &s, const uint4 (&kf)[8], const uint4 (&qf)[8]) {
    s = f32x16a_t{};
#pragma unroll
    for (int j = 0; j < 8; ++j) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[j]), as_bf16x8(qf[j]), s, 0, 0, 0);
}

// O^T += V^T P^T for one 32-query tile over one 32-key sub-block: 8 MFMAs.
__device__ __forceinline__ void att_pv(f32x16a_t (&o)[4], const uint4 (&vf)[2][4], const uint4 (&pf)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(vf[u][dt]), as_bf16x8(pf[u]), o[dt], 0, 0, 0);
}

// Keys at or past T (the partial last sub-block) get a score of -inf.
__device__ __forceinline__ void att_mask(f32x16a_t &s, int kbase, int T, int hf) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int key = kbase + 8 * (i >> 2) + 4 * hf + (i & 3);
        if (key >= T) s[i] = -__builtin_inff();
    }
}

__device__ __forceinline__ float att_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Keep a softmax inside the region whose MFMAs it runs beside: the compiler
// would otherwise sink it past the branch that ends the region.
__device__ __forceinline__ void att_pin(uint4 (&pf)[2], float &x) {
    u32x4_t v0 = {pf[0].x, pf[0].y, pf[0].z, pf[0].w}, v1 = {pf[1].x, pf[1].y, pf[1].z, pf[1].w};
    asm volatile("" : "+v"(v0), "+v"(v1), "+v"(x));
    pf[0] = make_uint4(v0.x, v0.y, v0.z, v0.w);
    pf[1] = make_uint4(v1.x, v1.y, v1.z, v1.w);
}

// P = 2^(s c - m) for this lane's 16 keys of query lq, written as the bf16 B
// operands of the P V product; returns their sum (of the bf16 values used).
__device__ __forceinline__ float att_exp_pack(const f32x16a_t &s, float m, uint4 (&pf)[2], float c) {
    const bf16x2_t ones = {(__bf16)1.0f, (__bf16)1.0f};
    float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * u + 2 * e], c, -m));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * u + 2 * e + 1], c, -m));
            w[e] = pack_bf16x2(p0, p1);
        }
        pf[u] = make_uint4(w[0], w[1], w[2], w[3]);
        sum0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[0]), ones, sum0, false);
        sum1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[1]), ones, sum1, false);
        sum0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[2]), ones, sum0, false);
        sum1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[3]), ones, sum1, false);
    }
    return sum0 + sum1;
}

// The (unscaled) row max of a score tile over both half-waves (the other
// half-wave holds the other 16 keys of the same query).
__device__ __forceinline__ float att_rowmax(const f32x16a_t &s) {
    float a0 = att_max(s[0], s[1]), a1 = att_max(s[2], s[3]);
#pragma unroll
    for (int i = 4; i < 16; i += 4) {
        a0 = att_max(a0, att_max(s[i], s[i + 1]));
        a1 = att_max(a1, att_max(s[i + 2], s[i + 3]));
    }
    const float mx0 = att_max(a0, a1);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx0), __float_as_uint(mx0), false, false);
    return att_max(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

// Online softmax with a running max (the safe form).  Scores above the
// reference max m by at most ATT_RESCALE (log2 units) are exponentiated
// against m as they are (P <= 2^ATT_RESCALE); a sub-block whose max exceeds
// that moves m to its max.  Updates m and the partial sum l (this lane's keys;
// the half-waves' sums are added at the end) and returns the factor O must be
// multiplied by before this sub-block's P V.
constexpr float ATT_RESCALE = 8.0f;

__device__ __forceinline__ float att_softmax(const f32x16a_t &s, float &m, float &l, uint4 (&pf)[2], float c) {
    const float mx = att_rowmax(s) * c;
    const float mnew = mx > m + ATT_RESCALE ? mx : m;
    float alpha = __builtin_amdgcn_exp2f(m - mnew);  // 1 if m stays, 0 on the first sub-block
    m = mnew;
    l = l * alpha + att_exp_pack(s, mnew, pf, c);
    att_pin(pf, alpha);
    return alpha;
}

// o *= alpha, skipped (wave-uniform) when no query of the wave moved its max.
__device__ __forceinline__ void att_rescale(f32x16a_t (&o)[4], float alpha) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
    }
}

// The softmax of one region.  FIXED: against the reference max m fixed by
// the tile's first sub-block (no max, no rescale: l += sum, nothing to branch
// on); otherwise the safe form above.  att_sm_end runs at the region's end,
// after its LDS reads are issued.
template <bool FIXED>
__device__ __forceinline__ float att_sm(const f32x16a_t &s, float &m, float &l, uint4 (&pf)[2], float c) {
    if constexpr (FIXED) {
        float sum = att_exp_pack(s, m, pf, c);
        att_pin(pf, sum);
        return sum;
    } else {
        return att_softmax(s, m, l, pf, c);
    }
}
template <bool FIXED>
__device__ __forceinline__ void att_sm_end(f32x16a_t (&o)[4], float &l, float r) {
    if constexpr (FIXED) l += r;
    else att_rescale(o, r);
}

// One pass over all keys for this wave's 64 queries: two 32-query tiles
// (0, 1), keys in 32-key sub-blocks u (two per 64-key LDS block).  Per
// sub-block the work is S_t = K Q_t^T, the softmax SM_t and O_t += V^T P_t^T;
// it runs software-pipelined in two steps so that each softmax runs on the
// vector ALU beside 16 MFMAs that do not depend on it:
//   X(u): MFMA S_1(u), PV_1(u-1)   | VALU SM_0(u) | LDS reads of V^T(u), K(u+1)
//   Y(u): MFMA PV_0(u), S_0(u+1)   | VALU SM_1(u)
// Every K and V^T fragment is read from LDS once and used for both query
// tiles; the fragments alternate between two register sets by the parity of u.
// LDS holds four 64-key blocks: block n + 2 is issued into the slot of block
// n - 2 at the barrier before X(2n - 1), after the last read of that slot.
//
// FAST: after each tile's first sub-block (which sets m to its max) the
// reference max stays fixed, so a region has no max, no rescale and no branch.
// P may then exceed 1 by the growth of the scores past the first sub-block's
// max; the caller checks that l stayed below ATT_FAST_LMAX (so that P, l and O
// stayed finite) and otherwise reruns the pass with FAST = false.
template <bool FAST>
__device__ __forceinline__ void att_pass(const AttnArgs &p, const AttLoader &ld, uint8_t *lds, const uint4 (&qf)[2][8],
                                         int wave, int lq, int hf, int kb0, int nkb, f32x16a_t (&o0)[4],
                                         f32x16a_t (&o1)[4], float &m0, float &m1, float &l0, float &l1) {
    // Key blocks [kb0, kb0 + nkb); n below counts from kb0.  Keys past T exist
    // only in the last block of T; a sub-block there may be all masked, which
    // gives P = 0 and leaves m, l and O as they are.
    const int lastb = nkb - 1;
    const bool ragged = kb0 + nkb == p.nkb && (p.T & (ATT_KB - 1)) != 0;
    const int key0 = kb0 * ATT_KB;
    const float c = p.scale_log2e;
#pragma unroll
    for (int i = 0; i < 3; ++i) att_issue(ld, wave, lds + i * ATT_STAGE, kb0 + (i < nkb ? i : lastb));

#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o0[dt] = o1[dt] = f32x16a_t{};
    m0 = m1 = -__builtin_inff();
    l0 = l1 = 0.f;
    uint4 kfa[8], kfb[8], vfa[2][4], vfb[2][4], pf0[2], pf1[2];
    f32x16a_t s0, s1;
    auto slot = [&](int n) { return lds + (n & 3) * ATT_STAGE; };

    // Block 0 landed for every wave.  S_0(0); X(0) without a P V, whose
    // softmax (the safe form) sets tile 0's reference max; in a FAST pass
    // tile 1's is set here from S_1(0) as well.
    att_wait_vmcnt<16>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    att_read_k(kfa, lds, 0, lq, hf);
    att_scores(s0, kfa, qf[0]);
    if (lastb == 0 && ragged) att_mask(s0, key0, p.T, hf);
    {
        att_scores(s1, kfa, qf[1]);
        const float r = att_sm<false>(s0, m0, l0, pf0, c);
        att_read_v(vfa, slot(0) + ATT_TILE, 0, lq, hf);
        att_read_k(kfb, slot(0), 1, lq, hf);
        att_sm_end<false>(o0, l0, r);
    }
    if (FAST) {
        if (lastb == 0 && ragged) att_mask(s1, key0, p.T, hf);
        m1 = att_rowmax(s1) * c;
    }
    // Block n: sub-blocks u = 2n (fragments in the "a" registers) and 2n + 1 ("b").
    for (int n = 0; n < lastb; ++n) {
        // ---- Y(2n): P V with vfa, next scores with kfb
        {
            att_pv(o0, vfa, pf0);
            att_scores(s0, kfb, qf[0]);
            const float r = att_sm<FAST>(s1, m1, l1, pf1, c);
            att_sm_end<FAST>(o1, l1, r);
        }
        // Block n + 1 (K of sub-block 2n + 2, read in X(2n + 1)) landed for
        // every wave; the slot of block n - 1 is free: issue block n + 3 there.
        att_wait_vmcnt<8>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        att_issue(ld, wave, slot(n + 3), kb0 + (n + 3 < nkb ? n + 3 : lastb));
        // ---- X(2n + 1): scores with kfb, P V with vfa; reads vfb, kfa
        {
            att_scores(s1, kfb, qf[1]);
            att_pv(o1, vfa, pf1);
            const float r = att_sm<FAST>(s0, m0, l0, pf0, c);
            att_read_v(vfb, slot(n) + ATT_TILE, 1, lq, hf);
            att_read_k(kfa, slot(n + 1), 0, lq, hf);
            att_sm_end<FAST>(o0, l0, r);
        }
        // ---- Y(2n + 1): P V with vfb, next scores with kfa
        {
            att_pv(o0, vfb, pf0);
            att_scores(s0, kfa, qf[0]);
            const float r = att_sm<FAST>(s1, m1, l1, pf1, c);
            att_sm_end<FAST>(o1, l1, r);
        }
        if (n + 1 == lastb && ragged) att_mask(s0, key0 + (n + 1) * ATT_KB, p.T, hf);
        // ---- X(2n + 2): scores with kfa, P V with vfb; reads vfa, kfb
        {
            att_scores(s1, kfa, qf[1]);
            att_pv(o1, vfb, pf1);
            const float r = att_sm<FAST>(s0, m0, l0, pf0, c);
            att_read_v(vfa, slot(n + 1) + ATT_TILE, 0, lq, hf);
            att_read_k(kfb, slot(n + 1), 1, lq, hf);
            att_sm_end<FAST>(o0, l0, r);
        }
    }
    // Last block L: Y(2L), X(2L + 1), Y(2L + 1) and PV_1(2L + 1); its data
    // landed at the last barrier (or the first), no further loads.
    if (ragged) att_mask(s1, key0 + lastb * ATT_KB, p.T, hf);
    {
        att_pv(o0, vfa, pf0);
        att_scores(s0, kfb, qf[0]);
        const float r = att_sm<FAST>(s1, m1, l1, pf1, c);
        att_sm_end<FAST>(o1, l1, r);
    }
    if (ragged) att_mask(s0, key0 + lastb * ATT_KB + 32, p.T, hf);
    {
        att_scores(s1, kfb, qf[1]);
        att_pv(o1, vfa, pf1);
        const float r = att_sm<FAST>(s0, m0, l0, pf0, c);
        att_read_v(vfb, slot(lastb) + ATT_TILE, 1, lq, hf);
        att_sm_end<FAST>(o0, l0, r);
    }
    if (ragged) att_mask(s1, key0 + lastb * ATT_KB + 32, p.T, hf);
    {
        att_pv(o0, vfb, pf0);
        const float r = att_sm<FAST>(s1, m1, l1, pf1, c);
        att_sm_end<FAST>(o1, l1, r);
    }
    att_pv(o1, vfb, pf1);
    att_wait_vmcnt<0>();  // the clamped tail loads land before the LDS is reused or released
}

// Bound on a lane's partial sum l after a FAST pass: below it, every P and
// every |O| (for |V| < 2^63) stayed finite.
constexpr float ATT_FAST_LMAX = 18446744073709551616.0f;  // 2^64

template <bool QOUT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_attn_fwd(AttnArgs p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    __shared__ int redo[4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lq = lane & 31, hf = lane >> 5;

    // Work item (query block, head, batch) and key-block range.  Workgroup ids
    // go to the XCDs round-robin (over 8); each range of workgroups (the whole
    // items, then the tail chunks) is remapped so that each XCD runs a
    // contiguous range of it: the query blocks of few heads at a time, which
    // share K and V^T in that XCD's L2.  Tail chunks are ordered chunk-major.
    int item, kb0 = 0, nkb = p.nkb, tail = -1;
    {
        int lin = blockIdx.x, nw = p.nfull;
        if (lin >= p.nfull) {
            lin -= p.nfull;
            nw = p.ntail * p.nsplit;
        }
        const int xcd = lin & 7, base = nw >> 3, rem = nw & 7;
        const int w = xcd * base + (xcd < rem ? xcd : rem) + (lin >> 3);
        if (blockIdx.x < (unsigned)p.nfull) {
            item = w;
        } else {
            const int chunk = w / p.ntail, ti = w % p.ntail;
            item = p.nfull + ti;
            kb0 = chunk * p.kbc;
            nkb = p.nkb - kb0 < p.kbc ? p.nkb - kb0 : p.kbc;
            tail = ti * p.nsplit + chunk;
        }
    }
    const int qblk = item % p.nq, h = (item / p.nq) % p.H, b = item / (p.nq * p.H);
    const int q0 = qblk * ATT_BQ + wave * 64;

    // Q^T operands: lane (q, hf) holds d [16j + 8hf, +8) of query q0 + 32t + q.
    uint4 qf[2][8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        int qi = q0 + 32 * t + lq;
        qi = qi < p.S ? qi : p.S - 1;  // rows past the end: computed, not stored
        const uint16_t *qrow = p.q + ((int64_t)b * p.S + qi) * p.ldq + (int64_t)h * ATT_D + hf * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) qf[t][j] = *reinterpret_cast<const uint4 *>(qrow + 16 * j);
    }
    // Q^T is only ever an MFMA operand: keep it in accumulation registers, which
    // leaves the architectural ones to O, the scores, P and the softmax.
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u32x4_t v = {qf[t][j].x, qf[t][j].y, qf[t][j].z, qf[t][j].w};
            asm volatile("" : "+a"(v));
            qf[t][j] = make_uint4(v.x, v.y, v.z, v.w);
        }

    const AttLoader ld = att_loader(p, b, h, wave, lane);
    f32x16a_t o0[4], o1[4];
    float m0, m1, l0, l1;
    att_pass<true>(p, ld, lds, qf, wave, lq, hf, kb0, nkb, o0, o1, m0, m1, l0, l1);
    // Rerun the whole workgroup in the safe form when any wave's sums left
    // the range the fixed reference max guarantees (scores that grew by more
    // than ~64 in log2 units past their first sub-block's max).
    if (threadIdx.x % 64 == 0) redo[wave] = 0;
    const bool bad = !(l0 < ATT_FAST_LMAX && l1 < ATT_FAST_LMAX);
    if (__builtin_amdgcn_ballot_w64(bad) && lane == 0) redo[wave] = 1;
    __syncthreads();
    if (redo[0] | redo[1] | redo[2] | redo[3])
        att_pass<false>(p, ld, lds, qf, wave, lq, hf, kb0, nkb, o0, o1, m0, m1, l0, l1);

    // O = O^T / l: lane (q, hf) holds dims 32dt + 8(i/4) + 4hf + i%4 of its query.
    // A tail chunk writes the same bf16 rows into its part_o slot (256 x 128)
    // and (m, l) of each query into part_ml, for k_attn_merge.
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const f32x16a_t(&o)[4] = t ? o1 : o0;
        const float lf = t ? l1 : l0;
        const float lt = lf + __shfl_xor(lf, 32, 64);
        const float inv = 1.0f / lt;
        const int qi = q0 + 32 * t + lq;
        if (qi >= p.S) continue;
        if (QOUT && tail < 0) {
            // MXFP8: the bf16 values the plain output would hold, quantized as
            // qim_mx_quantize does.  A 32-column block (dt) is this lane's 16
            // values and its partner's (lane ^ 32).
            const int64_t row = (int64_t)b * p.S + qi;
            uint32_t sc = 0;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                float f[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) f[i] = rbf(o[dt][i] * inv);
                uint32_t m = absmax_bits8(f);
                const uint32_t m2 = absmax_bits8(f + 8);
                m = m2 > m ? m2 : m;
                const uint32_t mp = (uint32_t)__shfl_xor((int)m, 32, 64);
                m = mp > m ? mp : m;
                const int e = mx_exponent(__uint_as_float(m));
                const float s = mx_scale_operand(e);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int64_t k = (int64_t)h * ATT_D + 32 * dt + 8 * g + 4 * hf;
                    *reinterpret_cast<uint32_t *>(p.qcodes + att_code_offset(p, row, k)) =
                        cvt_e4m3x4_scaled(f[4 * g], f[4 * g + 1], f[4 * g + 2], f[4 * g + 3], s);
                }
                sc |= (uint32_t)e << (8 * dt);
            }
            if (hf == 0)
                *reinterpret_cast<uint32_t *>(p.qscales + mx_scale_offset(row, 4 * h, (int64_t)p.H * ATT_D)) = sc;
            continue;
        }
        uint16_t *orow = p.o + ((int64_t)b * p.S + qi) * p.ldo + (int64_t)h * ATT_D;
        if (tail >= 0) {
            const int ql = wave * 64 + 32 * t + lq;
            orow = p.part_o + ((int64_t)tail * ATT_BQ + ql) * ATT_D;
            if (hf == 0)
                *reinterpret_cast<float2 *>(p.part_ml + ((int64_t)tail * ATT_BQ + ql) * 2) =
                    make_float2(t ? m1 : m0, lt);
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * dt + 8 * g + 4 * hf;
                const uint2 w = make_uint2(pack_bf16x2(o[dt][4 * g + 0] * inv, o[dt][4 * g + 1] * inv),
                                           pack_bf16x2(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv));
                *reinterpret_cast<uint2 *>(orow + d) = w;
            }
    }
}

// Combine the chunks of each tail item from their normalised rows
// R_c = O_c / l_c: O = sum_c w_c R_c / sum_c w_c with w_c = 2^(m_c - M) l_c,
// M = max_c m_c (accumulated with a running max).  One thread per (item,
// query, 8 d).
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs p) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int dg = (int)(g & 15), ql = (int)((g >> 4) & (ATT_BQ - 1));
    const int ti = (int)(g >> 12);  // 16 x 256 threads per item
    if (ti >= p.ntail) return;
    const int item = p.nfull + ti;
    const int qblk = item % p.nq, h = (item / p.nq) % p.H, b = item / (p.nq * p.H);
    const int qi = qblk * ATT_BQ + ql;
    if (qi >= p.S) return;
    // One pass, rescaling the running sums when the max grows, so that each
    // chunk's loads do not wait for the previous chunks' arithmetic.
    const int nc = p.nsplit;
    float M = -__builtin_inff(), wsum = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (int c = 0; c < nc; ++c) {
        const int64_t tc = (int64_t)(ti * p.nsplit + c);
        const float2 ml = *reinterpret_cast<const float2 *>(p.part_ml + (tc * ATT_BQ + ql) * 2);
        float r[8];
        unpack8(*reinterpret_cast<const uint4 *>(p.part_o + (tc * ATT_BQ + ql) * ATT_D + dg * 8), r);
        const float Mn = ml.x > M ? ml.x : M;
        const float sc = __builtin_amdgcn_exp2f(M - Mn);  // 0 on the first chunk (M = -inf)
        const float w = __builtin_amdgcn_exp2f(ml.x - Mn) * ml.y;
        wsum = wsum * sc + w;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = acc[e] * sc + w * r[e];
        M = Mn;
    }
    const float inv = 1.0f / wsum;
    if (p.qcodes) {
        // MXFP8 output: a 32-column block is 4 adjacent threads (dg 4j .. 4j+3).
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = rbf(acc[e] * inv);
        int e;
        const uint2 c = quantize8(f, e);
        const int64_t row = (int64_t)b * p.S + qi;
        *reinterpret_cast<uint2 *>(p.qcodes + att_code_offset(p, row, (int64_t)h * ATT_D + dg * 8)) = c;
        if ((dg & 3) == 0) p.qscales[mx_scale_offset(row, 4 * h + (dg >> 2), (int64_t)p.H * ATT_D)] = (uint8_t)e;
        return;
    }
    uint16_t *orow = p.o + ((int64_t)b * p.S + qi) * p.ldo + (int64_t)h * ATT_D + dg * 8;
    // 8-byte stores: ldo need only be a multiple of 4 elements.
    *reinterpret_cast<uint2 *>(orow) = make_uint2(pack_bf16x2(acc[0] * inv, acc[1] * inv),
                                                  pack_bf16x2(acc[2] * inv, acc[3] * inv));
    *reinterpret_cast<uint2 *>(orow + 4) = make_uint2(pack_bf16x2(acc[4] * inv, acc[5] * inv),
                                                      pack_bf16x2(acc[6] * inv, acc[7] * inv));
}

// MXFP8 output rows [M, Mp) (the padding of the last 128-row scale block):
// zero codes and scales, as qim_mx_quantize writes them.  One thread per
// 16-byte code chunk.
__global__ __launch_bounds__(256) void k_attn_qpad(AttnArgs p, int64_t M) {
    const int64_t K = (int64_t)p.H * ATT_D, per_row = K / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t r = M + i / per_row, c = i % per_row;
    if (r >= p.Mp) return;
    *reinterpret_cast<uint4 *>(p.qcodes + att_code_offset(p, r, c * 16)) = make_uint4(0, 0, 0, 0);
    if (c < K / 128) *reinterpret_cast<uint32_t *>(p.qscales + mx_scale_offset(r, 4 * c, K)) = 0;
}

}  // namespace qim

using namespace qim;

// Work split.  Every workgroup of k_attn_fwd runs for about the same time and
// one fits per CU, so W whole items take ceil(W / CUs) rounds; when the last
// round is partial, its items may run instead as chunks of kbc key blocks plus
// a merge pass.  Cost model, in units of one workgroup's time per 64-key
// block (measured ~1.75 us at 24 heads): whole rounds * nkb + chunk rounds *
// kbc + the partials' HBM traffic (written once, read once by the merge, at
// ~5 TB/s) + ~3 for the merge launch.  A split is taken when it saves >= 5 %;
// chunks have at least ATT_MIN_CHUNK blocks.  Partials are bf16 rows and
// fp32 (m, l): 66 KiB per chunk.  (At S = T = 16640 and 24 heads the 24 tail
// items run as 10 chunks each, ~10 % faster; at S = T = 4352 the 152 tail
// items of one image run as 3 chunks each, ~1 % faster.)
namespace qim {

constexpr int ATT_MIN_CHUNK = 8;

AttPlan att_plan(int64_t B, int64_t S, int64_t T, int64_t H) {
    const int64_t nq = (S + ATT_BQ - 1) / ATT_BQ, nkb = (T + ATT_KB - 1) / ATT_KB, W = B * H * nq;
    const int64_t C = device_cus() > 0 ? device_cus() : 256;
    AttPlan pl{W, 0, 1, nkb, B * H * nkb * ATT_TILE, 0, 0};
    const int64_t R = W / C, Wr = W - R * C;
    if (Wr == 0) return pl;
    const double per_chunk_bytes = 2.0 * (ATT_BQ * ATT_D * 2 + ATT_BQ * 2 * 4);  // written + read
    const double bytes_per_block = 5e12 * 1.75e-6;
    double best = 0.95 * (double)((R + 1) * nkb);
    for (int64_t k = 2; k <= 16; ++k) {
        const int64_t kbc = (nkb + k - 1) / k;
        if (kbc < ATT_MIN_CHUNK) break;
        const int64_t keff = (nkb + kbc - 1) / kbc;
        const int64_t rounds = (Wr * keff + C - 1) / C;
        const double cost = (double)(R * nkb + rounds * kbc) + (double)(Wr * keff) * per_chunk_bytes / bytes_per_block + 3.0;
        if (cost < best) {
            best = cost;
            pl.nfull = R * C;
            pl.ntail = Wr;
            pl.nsplit = keff;
            pl.kbc = kbc;
        }
    }
    if (pl.ntail) {
        pl.part_o_bytes = pl.ntail * pl.nsplit * ATT_BQ * ATT_D * 2;
        pl.part_ml_bytes = pl.ntail * pl.nsplit * ATT_BQ * 2 * 4;
    }
    return pl;
}

// The checks and launches the attention entry points share.  Output: bf16 rows
// of o (ldo elements apart), or MXFP8 codes and scales when qcodes is set.
// v null: the workspace already holds V^T (qim_mxfp8_gemm_qk_norm_rope_vt),
// T % 64 == 0.
int attention_run(const char *who, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                         int64_t ldv, void *o, int64_t ldo, void *qcodes, void *qscales, int tiled, void *workspace,
                         int64_t workspace_bytes, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D, float scale,
                         void *stream) {
    QIM_REQUIRE(q && k && (o || (qcodes && qscales)) && workspace, QIM_ERR_ARG, "%s: null pointer", who);
    QIM_REQUIRE(D == ATT_D, QIM_ERR_SHAPE, "%s: head dim %lld (128 only)", who, (long long)D);
    QIM_REQUIRE(scale > 0.0f && scale < 1e30f, QIM_ERR_ARG, "%s: scale must be positive and finite", who);
    QIM_REQUIRE(B > 0 && S > 0 && T > 0 && H > 0, QIM_ERR_SHAPE, "%s: empty problem", who);
    QIM_REQUIRE(B < 65536 && H < 65536 && S < (1 << 30) && T < (1 << 30) && B * H * ((S + ATT_BQ - 1) / ATT_BQ) < (1 << 30),
                QIM_ERR_SHAPE, "%s: too large", who);
    QIM_REQUIRE(v || T % ATT_KB == 0, QIM_ERR_SHAPE, "%s: V^T from the workspace (v null) needs T %% 64 == 0", who);
    QIM_REQUIRE(ldq >= H * D && ldk >= H * D && (!v || (ldv >= H * D && ldv % 8 == 0)) && ldq % 8 == 0 &&
                    ldk % 8 == 0 &&
                    (qcodes || (ldo >= H * D && ldo % 4 == 0)),
                QIM_ERR_LAYOUT, "%s: token strides must cover H*D and be multiples of 8 (ldo: 4)", who);
    QIM_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(workspace) &&
                    (qcodes ? aligned16(qcodes) && aligned16(qscales) : (reinterpret_cast<uintptr_t>(o) & 7u) == 0),
                QIM_ERR_LAYOUT, "%s: q, k, v, workspace (and codes, scales) 16-byte aligned, o 8-byte aligned", who);
    QIM_REQUIRE(tiled == 0 || tiled == 1, QIM_ERR_ARG, "%s: tiled must be 0 or 1", who);
    const int64_t nkb = (T + ATT_KB - 1) / ATT_KB;
    QIM_REQUIRE(B * T * ldk < (1ll << 31), QIM_ERR_SHAPE, "%s: K above 4 GiB of offsets", who);
    const AttPlan pl = att_plan(B, S, T, H);
    QIM_REQUIRE(workspace_bytes >= pl.total(), QIM_ERR_ARG,
                "%s: workspace of %lld bytes, this problem needs %lld (qim_attention_workspace_bytes)", who,
                (long long)workspace_bytes, (long long)pl.total());
    static std::atomic<bool> configured[2][QIM_MAX_DEVICES] = {};
    const void *fwd = qcodes ? reinterpret_cast<const void *>(&k_attn_fwd<true>)
                             : reinterpret_cast<const void *>(&k_attn_fwd<false>);
    if (const int rc = reserve_lds(fwd, ATT_LDS, configured[qcodes ? 1 : 0], who)) return rc;
    hipStream_t st = as_stream(stream);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    if (v)
        launch(k_attn_vt, dim3((unsigned)nkb, (unsigned)H, (unsigned)B), dim3(256), 0, st,
                           (const uint16_t *)v, ldv, (uint16_t *)ws, (int)T, (int)H, (int)nkb);
    AttnArgs a{};
    a.q = (const uint16_t *)q;
    a.k = (const uint16_t *)k;
    a.vt = (const uint16_t *)ws;
    a.o = (uint16_t *)o;
    a.ldq = ldq;
    a.ldk = ldk;
    a.ldo = ldo;
    a.S = (int)S;
    a.T = (int)T;
    a.H = (int)H;
    a.nkb = (int)nkb;
    a.nq = (int)((S + ATT_BQ - 1) / ATT_BQ);
    a.nfull = (int)pl.nfull;
    a.ntail = (int)pl.ntail;
    a.nsplit = (int)pl.nsplit;
    a.kbc = (int)pl.kbc;
    a.part_o = reinterpret_cast<uint16_t *>(ws + pl.vt_bytes);
    a.part_ml = reinterpret_cast<float *>(ws + pl.vt_bytes + pl.part_o_bytes);
    a.scale_log2e = scale * 1.4426950408889634f;
    const int64_t M = B * S;
    a.qcodes = static_cast<uint8_t *>(qcodes);
    a.qscales = static_cast<uint8_t *>(qscales);
    a.Mp = (M + 127) / 128 * 128;
    a.tiled = tiled;
    const int64_t nwg = pl.nfull + pl.ntail * pl.nsplit;
    if (qcodes)
        launch(k_attn_fwd<true>, dim3((unsigned)nwg), dim3(256), ATT_LDS, st, a);
    else
        launch(k_attn_fwd<false>, dim3((unsigned)nwg), dim3(256), ATT_LDS, st, a);
    if (pl.ntail) {
        const int64_t threads = pl.ntail * ATT_BQ * (ATT_D / 8);
        launch(k_attn_merge, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, a);
    }
    if (qcodes && a.Mp > M) {
        const int64_t threads = (a.Mp - M) * H * ATT_D / 16;
        launch(k_attn_qpad, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, a, M);
    }
    return check_launch(who);
}

}  // namespace qim

extern "C" int qim_attention(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                             void *o, int64_t ldo, void *workspace, int64_t workspace_bytes, int64_t B, int64_t S,
                             int64_t T, int64_t H, int64_t D, float scale, void *stream) {
    if (!o) return qim::fail(QIM_ERR_ARG, "qim_attention: null pointer");
    return attention_run("qim_attention", q, ldq, k, ldk, v, ldv, o, ldo, nullptr, nullptr, 0, workspace,
                         workspace_bytes, B, S, T, H, D, scale, stream);
}

extern "C" int qim_attention_mxfp8(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                                   int64_t ldv, void *codes, void *scales, int tiled, void *workspace,
                                   int64_t workspace_bytes, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                                   float scale, void *stream) {
    if (!codes || !scales) return qim::fail(QIM_ERR_ARG, "qim_attention_mxfp8: null pointer");
    return attention_run("qim_attention_mxfp8", q, ldq, k, ldk, v, ldv, nullptr, 0, codes, scales, tiled, workspace,
                         workspace_bytes, B, S, T, H, D, scale, stream);
}

extern "C" int64_t qim_attention_workspace_bytes(int64_t B, int64_t S, int64_t T, int64_t H, int64_t D) {
    if (B <= 0 || S <= 0 || T <= 0 || H <= 0 || D != ATT_D) return 0;
    return att_plan(B, S, T, H).total();
}
