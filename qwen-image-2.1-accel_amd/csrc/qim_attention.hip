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
constexpr int ATT_NSTAGE = 3;
constexpr int ATT_LDS = ATT_NSTAGE * ATT_STAGE;  // 96 KiB

struct AttnArgs {
    const uint16_t *q, *k;
    const uint16_t *vt;  // V^T tiles
    uint16_t *o;
    int64_t ldq, ldk, ldo;  // elements between consecutive tokens
    int S, T, H, nkb;       // queries, keys, heads, key blocks
    float scale_log2e;
};

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
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds_addr)
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

// The 8 DMA instructions of one wave for key block kb (4 of K, 4 of V^T); kb
// is clamped by the caller.  K instruction n covers keys 4n..4n+3: lane i
// lands at LDS row key 4n + i/16, physical chunk i % 16, whose source is the
// key's logical chunk (i % 16) ^ (key & 15).  V^T tiles are copied as they are.

__device__ __forceinline__ void att_issue(const AttnArgs &p, int b, int h, int wave, int lane, uint8_t *slot, int kb) {
    const uint32_t base = att_lds_addr(slot);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = wave * 4 + j;
        const int r = 4 * n + (lane >> 4);            // key row in the block
        int t = kb * ATT_KB + r;
        t = t < p.T ? t : p.T - 1;                     // rows past the end: masked in the softmax
        const int c = (lane & 15) ^ (r & 15);
        const uint32_t off = (uint32_t)((((int64_t)b * p.T + t) * p.ldk + (int64_t)h * ATT_D + c * 8) * 2);
        att_dma16(p.k, off, base + n * 1024);
    }
    const uint16_t *tile = p.vt + (((int64_t)b * p.H + h) * p.nkb + kb) * (ATT_KB * ATT_D);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = wave * 4 + j;
        att_dma16(tile, (uint32_t)(n * 1024 + lane * 16), base + ATT_TILE + n * 1024);
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_attn_fwd(AttnArgs p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qblk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lq = lane & 31, hf = lane >> 5;
    const int q0 = qblk * ATT_BQ + wave * 64;  // this wave's 64 queries: tiles t = 0, 1 of 32

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

    att_issue(p, b, h, wave, lane, lds, 0);
    att_issue(p, b, h, wave, lane, lds + ATT_STAGE, 1 < p.nkb ? 1 : p.nkb - 1);

    f32x16a_t o[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[t][dt] = f32x16a_t{};
    float m[2] = {-__builtin_inff(), -__builtin_inff()}, l[2] = {0.f, 0.f};

    for (int kb = 0; kb < p.nkb; ++kb) {
        // Block kb landed (block kb + 1 may still be in flight) for every wave,
        // and every wave is done with block kb - 1, whose slot is reloaded next.
        // A bare s_barrier: __syncthreads would also drain the loads in flight.
        att_wait_vmcnt<8>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        {
            const int nb = kb + 2 < p.nkb ? kb + 2 : p.nkb - 1;
            att_issue(p, b, h, wave, lane, lds + ((kb + 2) % ATT_NSTAGE) * ATT_STAGE, nb);
        }
        const uint8_t *kt_lds = lds + (kb % ATT_NSTAGE) * ATT_STAGE;
        const uint8_t *vt_lds = kt_lds + ATT_TILE;

        // S^T = K Q^T: two 32-key tiles x two 32-query tiles, 8 steps of 16 d.
        f32x16a_t s[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) s[t][kt] = f32x16a_t{};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const int r = 32 * kt + lq;
                const int pc = (2 * j + hf) ^ (r & 15);
                const uint4 kf = *reinterpret_cast<const uint4 *>(kt_lds + r * 256 + pc * 16);
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    s[t][kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf), as_bf16x8(qf[t][j]), s[t][kt],
                                                                       0, 0, 0);
            }
        }

        // Online softmax per query (lane-local over this lane's 32 keys, plus
        // the other half-wave's 32 keys of the same query).
        const int kbase = kb * ATT_KB;
        uint4 pf[2][2][2];  // bf16 P^T operands [query tile][key tile][16-key step]
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            float x[2][16];
            float mx = -__builtin_inff();
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = kbase + 32 * kt + 8 * (i >> 2) + 4 * hf + (i & 3);
                    x[kt][i] = key < p.T ? s[t][kt][i] * p.scale_log2e : -__builtin_inff();
                    mx = x[kt][i] > mx ? x[kt][i] : mx;
                }
            const float mo = __shfl_xor(mx, 32, 64);
            mx = mo > mx ? mo : mx;
            const float mnew = m[t] > mx ? m[t] : mx;
            const float alpha = mnew == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f(m[t] - mnew);
            float sum = 0.f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float e = mnew == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(x[kt][i] - mnew);
                    x[kt][i] = e;
                    sum += e;
                }
            l[t] = l[t] * alpha + sum;
            m[t] = mnew;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[t][dt] *= alpha;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    pf[t][kt][u] = make_uint4(pack_bf16x2(x[kt][8 * u + 0], x[kt][8 * u + 1]),
                                              pack_bf16x2(x[kt][8 * u + 2], x[kt][8 * u + 3]),
                                              pack_bf16x2(x[kt][8 * u + 4], x[kt][8 * u + 5]),
                                              pack_bf16x2(x[kt][8 * u + 6], x[kt][8 * u + 7]));
        }

        // O^T += V^T P^T: four 32-dim tiles, four 16-key steps.
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int d = 32 * dt + lq;
                const int pc = (2 * kk + hf) ^ ((d >> 1) & 7);
                const uint4 vf = *reinterpret_cast<const uint4 *>(vt_lds + d * (ATT_KB * 2) + pc * 16);
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    o[t][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(vf), as_bf16x8(pf[t][kk >> 1][kk & 1]),
                                                                       o[t][dt], 0, 0, 0);
            }
        }
    }
    att_wait_vmcnt<0>();  // the clamped tail loads land before the workgroup ends

    // O = O^T / l: lane (q, hf) holds dims 32dt + 8(i/4) + 4hf + i%4 of its query.
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const float lt = l[t] + __shfl_xor(l[t], 32, 64);
        const float inv = 1.0f / lt;
        const int qi = q0 + 32 * t + lq;
        if (qi >= p.S) continue;
        uint16_t *orow = p.o + ((int64_t)b * p.S + qi) * p.ldo + (int64_t)h * ATT_D;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * dt + 8 * g + 4 * hf;
                const uint2 w = make_uint2(pack_bf16x2(o[t][dt][4 * g + 0] * inv, o[t][dt][4 * g + 1] * inv),
                                           pack_bf16x2(o[t][dt][4 * g + 2] * inv, o[t][dt][4 * g + 3] * inv));
                *reinterpret_cast<uint2 *>(orow + d) = w;
            }
    }
}

}  // namespace qim

using namespace qim;

extern "C" int qim_attention(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                             void *o, int64_t ldo, void *vt_workspace, int64_t B, int64_t S, int64_t T, int64_t H,
                             int64_t D, float scale, void *stream) {
    QIM_REQUIRE(q && k && v && o && vt_workspace, QIM_ERR_ARG, "qim_attention: null pointer");
    QIM_REQUIRE(D == ATT_D, QIM_ERR_SHAPE, "qim_attention: head dim %lld (128 only)", (long long)D);
    QIM_REQUIRE(B > 0 && S > 0 && T > 0 && H > 0, QIM_ERR_SHAPE, "qim_attention: empty problem");
    QIM_REQUIRE(B < 65536 && H < 65536 && S < (1 << 30) && T < (1 << 30), QIM_ERR_SHAPE, "qim_attention: too large");
    QIM_REQUIRE(ldq >= H * D && ldk >= H * D && ldv >= H * D && ldo >= H * D && ldq % 8 == 0 && ldk % 8 == 0 &&
                    ldv % 8 == 0 && ldo % 4 == 0,
                QIM_ERR_LAYOUT, "qim_attention: token strides must cover H*D and be multiples of 8 (ldo: 4)");
    QIM_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(vt_workspace) &&
                    (reinterpret_cast<uintptr_t>(o) & 7u) == 0,
                QIM_ERR_LAYOUT, "qim_attention: q, k, v, workspace 16-byte aligned, o 8-byte aligned");
    const int64_t nkb = (T + ATT_KB - 1) / ATT_KB;
    QIM_REQUIRE(B * T * ldk < (1ll << 31), QIM_ERR_SHAPE, "qim_attention: K above 4 GiB of offsets");
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_fwd),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, ATT_LDS);
        if (e != hipSuccess)
            return fail(QIM_ERR_LAUNCH, "qim_attention: cannot reserve %d bytes of LDS: %s", ATT_LDS,
                        hipGetErrorString(e));
        configured = true;
    }
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(k_attn_vt, dim3((unsigned)nkb, (unsigned)H, (unsigned)B), dim3(256), 0, st,
                       (const uint16_t *)v, ldv, (uint16_t *)vt_workspace, (int)T, (int)H, (int)nkb);
    AttnArgs a{(const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)vt_workspace, (uint16_t *)o, ldq, ldk, ldo,
               (int)S, (int)T, (int)H, (int)nkb, scale * 1.4426950408889634f};
    hipLaunchKernelGGL(k_attn_fwd, dim3((unsigned)((S + ATT_BQ - 1) / ATT_BQ), (unsigned)H, (unsigned)B), dim3(256),
                       ATT_LDS, st, a);
    return check_launch("qim_attention");
}

extern "C" int64_t qim_attention_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D) {
    if (B <= 0 || T <= 0 || H <= 0 || D != ATT_D) return 0;
    return B * H * ((T + ATT_KB - 1) / ATT_KB) * ATT_KB * ATT_D * 2;
}
