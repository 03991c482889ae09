// Error state of the libqim C ABI and the test hooks of its device conversions.
#include <stdarg.h>
#include <stdio.h>

#include "qim_device.h"
#include "qim_runtime.h"

namespace qim {

static thread_local char g_error[512];

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

hipError_t &launch_error() {
    static thread_local hipError_t e = hipSuccess;
    return e;
}

int check_launch(const char *what) {
    const hipError_t e = launch_error();
    launch_error() = hipSuccess;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(QIM_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    }
    g_error[0] = '\0';
    return QIM_OK;
}

// Per-device caches are written by whichever thread calls first; the values
// written are the same from every thread, so relaxed atomics suffice.
int device_cus() {
    static std::atomic<int> cached[QIM_MAX_DEVICES] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < QIM_MAX_DEVICES) {
        const int c = cached[dev].load(std::memory_order_relaxed);
        if (c) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev < QIM_MAX_DEVICES) cached[dev].store(n, std::memory_order_relaxed);
    return n;
}

int reserve_lds(const void *fn, int bytes, std::atomic<bool> (&done)[QIM_MAX_DEVICES], const char *who) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return fail(QIM_ERR_LAUNCH, "%s: no current device", who);
    if (dev < QIM_MAX_DEVICES && done[dev].load(std::memory_order_relaxed)) return QIM_OK;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess)
        return fail(QIM_ERR_LAUNCH, "%s: cannot reserve %d bytes of LDS: %s", who, bytes, hipGetErrorString(e));
    if (dev < QIM_MAX_DEVICES) done[dev].store(true, std::memory_order_relaxed);
    return QIM_OK;
}

// ----------------------------------------------------------- test hooks ----

__global__ void k_debug_e4m3(const float *__restrict__ x, uint8_t *__restrict__ codes, int64_t n) {
    int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 4 <= n) {
        uint32_t w = cvt_e4m3x4(x[i], x[i + 1], x[i + 2], x[i + 3]);
        *reinterpret_cast<uint32_t *>(codes + i) = w;
    } else {
        for (int64_t j = i; j < n; ++j)
            codes[j] = (uint8_t)(cvt_e4m3x4(x[j], 0.0f, 0.0f, 0.0f) & 0xffu);
    }
}

// bf16 values (n % 4 == 0) -> E4M3 codes of x * 2^(127 - e) through the packed
// scaled conversion the quantizers use.
__global__ void k_debug_e4m3_scaled(const uint32_t *__restrict__ x, int e, uint32_t *__restrict__ codes, int64_t n4) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n4) codes[i] = cvt_e4m3x4_bf16(x[2 * i], x[2 * i + 1], mx_scale_operand(e));
}

__global__ void k_debug_bf16(const float *__restrict__ x, uint16_t *__restrict__ bits, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) bits[i] = (uint16_t)(pack_bf16x2(x[i], 0.0f) & 0xffffu);
}

// One v_mfma_scale_f32_32x32x64_f8f6f4 on a single tile.  Operand layout
// (CDNA4): lane l holds row (l % 32) of A and column (l % 32) of B; with
// h = l / 32 its bytes 0-15 are K [16h, +16) and bytes 16-31 are K [32 + 16h,
// +16); lane l supplies the exponent of (row l % 32, K block h).
// Result: lane l, register i holds D[8 * (i / 4) + 4 * (l / 32) + i % 4][l % 32].
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__global__ void k_debug_mfma(const uint8_t *__restrict__ a, const uint8_t *__restrict__ b,
                             const uint8_t *__restrict__ sa, const uint8_t *__restrict__ sb,
                             float *__restrict__ out) {
    const int l = threadIdx.x;
    const int r = l & 31, kh = l >> 5;
    i32x8_t av, bv;
    const int *ap = reinterpret_cast<const int *>(a + r * 64 + kh * 16);
    const int *bp = reinterpret_cast<const int *>(b + r * 64 + kh * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        av[i] = ap[i]; bv[i] = bp[i];            // K [16h, 16h + 16)
        av[i + 4] = ap[i + 8]; bv[i + 4] = bp[i + 8];  // K [32 + 16h, +16)
    }
    int sav = sa[r * 2 + kh], sbv = sb[r * 2 + kh];
    f32x16_t acc = {};
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, 0, 0, 0, sav, 0, sbv);
#pragma unroll
    for (int i = 0; i < 16; ++i) out[(8 * (i / 4) + 4 * kh + (i % 4)) * 32 + r] = acc[i];
}

// Scale-routing probe.  Experiment e = (operand, lane, byte): the probed
// operand is one-hot (code 0x38 = 1.0 at that lane and byte), the other is all
// ones; the probed operand's per-lane exponents are 100 + lane, the other's 127.
// The output then holds 2^(lane' - 27) exactly at the row (A) or column (B) fed
// by `lane`, where lane' is the lane whose exponent the hardware applied to
// that byte.  SHAPE 0: 32x32x64 (out 32x32), 1: 16x16x128 (out 16x16).
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int SHAPE>
__global__ void k_debug_mfma_probe(float *__restrict__ out) {
    const int e = blockIdx.x;               // 0 .. 4095
    const int operand = e >> 11, plane = (e >> 5) & 63, pbyte = e & 31;
    const int l = threadIdx.x;
    i32x8_t one_hot, ones;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ones[i] = 0x38383838;
        int w = 0;
        if (l == plane && (pbyte >> 2) == i) w = 0x38 << (8 * (pbyte & 3));
        one_hot[i] = w;
    }
    const int s_probe = 100 + l, s_one = 127;
    const i32x8_t a = operand == 0 ? one_hot : ones;
    const i32x8_t b = operand == 0 ? ones : one_hot;
    const int sa = operand == 0 ? s_probe : s_one;
    const int sb = operand == 0 ? s_one : s_probe;
    if constexpr (SHAPE == 0) {
        f32x16_t acc = {};
        acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, sa, 0, sb);
        float *o = out + (size_t)e * 1024;
#pragma unroll
        for (int i = 0; i < 16; ++i) o[(8 * (i / 4) + 4 * (l >> 5) + (i % 4)) * 32 + (l & 31)] = acc[i];
    } else {
        f32x4_t acc = {};
        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 0, 0, 0, sa, 0, sb);
        float *o = out + (size_t)e * 256;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[(4 * (l >> 4) + i) * 16 + (l & 15)] = acc[i];
    }
}

// bf16(silu(g)): odd threads through silu_bf16, even ones through the batched
// silu_bf16_n<8> on g[i .. i+7] (one element kept), so an exhaustive sweep
// covers both forms.
__global__ void k_debug_silu(const uint16_t *__restrict__ g, uint16_t *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float y;
    if (i & 1) {
        y = silu_bf16(bf16_to_f32(g[i]));
    } else {
        float x[8], r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = bf16_to_f32(g[i + j < n ? i + j : i]);
        silu_bf16_n<8>(x, r);
        y = r[0];
    }
    out[i] = (uint16_t)(__float_as_uint(y) >> 16);
}

// rstd_of(v, eps) against its definition fp32(1 / sqrt(double(v + eps)))
// for the fp32 values v with bit patterns [first, first + count): bad[0]
// counts disagreements, bad[1] keeps the smallest disagreeing pattern.
__global__ void k_debug_rstd_sweep(uint32_t first, uint32_t count, float eps, uint32_t *bad) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= count) return;
    const uint32_t bits = first + i;
    const float v = __uint_as_float(bits);
    const float fast = rstd_of(v, eps);
    const float ref = (float)(1.0 / sqrt((double)(v + eps)));
    if (__float_as_uint(fast) != __float_as_uint(ref)) {
        atomicAdd(bad, 1u);
        atomicMin(bad + 1, bits);
    }
}

// Streaming copy, one 16-byte vector per lane: the achievable-bandwidth
// reference and the calibration kernel of the HBM byte counters.
__global__ __launch_bounds__(256) void k_debug_copy(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                     int64_t nvec) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < nvec) st_nt(dst + i, ld_nt(src + i));
}

// Copy variants for the single-launch bandwidth ceiling: U 16-byte vectors
// per lane (all loads, then all stores); one-shot (each workgroup one chunk of
// 256 U vectors) or grid-stride over a persistent grid.
template <int U, bool PERSIST>
__global__ __launch_bounds__(256) void k_debug_copy_u(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                       int64_t nvec) {
    const int64_t stride = PERSIST ? (int64_t)gridDim.x * 256 * U : nvec;
    for (int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x; base < nvec; base += stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (base + u * 256 < nvec) v[u] = ld_nt(src + base + u * 256);
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (base + u * 256 < nvec) st_nt(dst + base + u * 256, v[u]);
    }
}

}  // namespace qim

using namespace qim;

extern "C" int qim_debug_copy_ex(const void *src, void *dst, int64_t nbytes, int vectors_per_lane, int blocks_per_cu,
                                 void *stream) {
    QIM_REQUIRE(src && dst && nbytes >= 0 && blocks_per_cu >= 0 && blocks_per_cu <= 64, QIM_ERR_ARG,
                "qim_debug_copy_ex: bad arguments");
    QIM_REQUIRE(vectors_per_lane == 1 || vectors_per_lane == 2 || vectors_per_lane == 4 || vectors_per_lane == 8,
                QIM_ERR_ARG, "qim_debug_copy_ex: vectors_per_lane must be 1, 2, 4 or 8");
    QIM_REQUIRE(nbytes % 16 == 0 && aligned16(src) && aligned16(dst), QIM_ERR_LAYOUT,
                "qim_debug_copy_ex: 16-byte aligned operands and size required");
    const int64_t nvec = nbytes / 16, per_block = 256ll * vectors_per_lane;
    QIM_REQUIRE(nvec / per_block < (1ll << 31), QIM_ERR_SHAPE, "qim_debug_copy_ex: too large");
    if (nvec == 0) return QIM_OK;
    const int cus = device_cus() > 0 ? device_cus() : 256;
    const int64_t grid = blocks_per_cu ? (int64_t)blocks_per_cu * cus : (nvec + per_block - 1) / per_block;
    const uint4 *s = (const uint4 *)src;
    uint4 *d = (uint4 *)dst;
    hipStream_t st = as_stream(stream);
    const dim3 g((unsigned)grid), b(256);
    switch (vectors_per_lane * 2 + (blocks_per_cu ? 1 : 0)) {
        case 2: launch(k_debug_copy_u<1, false>, g, b, 0, st, s, d, nvec); break;
        case 3: launch(k_debug_copy_u<1, true>, g, b, 0, st, s, d, nvec); break;
        case 4: launch(k_debug_copy_u<2, false>, g, b, 0, st, s, d, nvec); break;
        case 5: launch(k_debug_copy_u<2, true>, g, b, 0, st, s, d, nvec); break;
        case 8: launch(k_debug_copy_u<4, false>, g, b, 0, st, s, d, nvec); break;
        case 9: launch(k_debug_copy_u<4, true>, g, b, 0, st, s, d, nvec); break;
        case 16: launch(k_debug_copy_u<8, false>, g, b, 0, st, s, d, nvec); break;
        default: launch(k_debug_copy_u<8, true>, g, b, 0, st, s, d, nvec); break;
    }
    return check_launch("qim_debug_copy_ex");
}

extern "C" int qim_debug_silu(const void *g, void *out, int64_t n, void *stream) {
    QIM_REQUIRE(g && out && n >= 0, QIM_ERR_ARG, "qim_debug_silu: bad arguments");
    QIM_REQUIRE((n + 255) / 256 < (1ll << 31), QIM_ERR_SHAPE, "qim_debug_silu: too large");
    if (n == 0) return QIM_OK;
    launch(k_debug_silu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream),
                       (const uint16_t *)g, (uint16_t *)out, n);
    return check_launch("qim_debug_silu");
}

extern "C" int qim_debug_rstd_sweep(uint32_t first, uint32_t count, float eps, void *bad, void *stream) {
    QIM_REQUIRE(bad, QIM_ERR_ARG, "qim_debug_rstd_sweep: null pointer");
    QIM_REQUIRE((uint64_t)first + count <= 0x100000000ull, QIM_ERR_SHAPE,
                "qim_debug_rstd_sweep: patterns past 2^32");
    QIM_REQUIRE(((uintptr_t)bad & 3u) == 0, QIM_ERR_LAYOUT, "qim_debug_rstd_sweep: bad must be 4-byte aligned");
    if (count == 0) return QIM_OK;
    launch(k_debug_rstd_sweep, dim3((unsigned)(((uint64_t)count + 255) / 256)), dim3(256), 0, as_stream(stream),
           first, count, eps, (uint32_t *)bad);
    return check_launch("qim_debug_rstd_sweep");
}

extern "C" int qim_debug_copy(const void *src, void *dst, int64_t nbytes, void *stream) {
    QIM_REQUIRE(src && dst && nbytes >= 0, QIM_ERR_ARG, "qim_debug_copy: bad arguments");
    QIM_REQUIRE(nbytes % 16 == 0 && aligned16(src) && aligned16(dst), QIM_ERR_LAYOUT,
                "qim_debug_copy: 16-byte aligned operands and size required");
    const int64_t nvec = nbytes / 16;
    QIM_REQUIRE((nvec + 255) / 256 < (1ll << 31), QIM_ERR_SHAPE, "qim_debug_copy: too large");
    if (nvec == 0) return QIM_OK;
    launch(k_debug_copy, dim3((unsigned)((nvec + 255) / 256)), dim3(256), 0, as_stream(stream),
                       (const uint4 *)src, (uint4 *)dst, nvec);
    return check_launch("qim_debug_copy");
}

extern "C" int qim_debug_mfma_probe(int shape, float *out, void *stream) {
    QIM_REQUIRE(out && (shape == 0 || shape == 1), QIM_ERR_ARG, "qim_debug_mfma_probe: bad arguments");
    if (shape == 0)
        launch(k_debug_mfma_probe<0>, dim3(4096), dim3(64), 0, as_stream(stream), out);
    else
        launch(k_debug_mfma_probe<1>, dim3(4096), dim3(64), 0, as_stream(stream), out);
    return check_launch("qim_debug_mfma_probe");
}

extern "C" const char *qim_last_error(void) { return g_error; }

extern "C" int qim_abi_version(void) { return 3; }

extern "C" int qim_debug_e4m3_encode(const float *x, void *codes, int64_t n, void *stream) {
    QIM_REQUIRE(x && codes && n >= 0, QIM_ERR_ARG, "qim_debug_e4m3_encode: bad arguments");
    if (n == 0) return QIM_OK;
    int64_t threads = (n + 3) / 4;
    launch(k_debug_e4m3, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       as_stream(stream), x, (uint8_t *)codes, n);
    return check_launch("qim_debug_e4m3_encode");
}

extern "C" int qim_debug_e4m3_encode_scaled(const void *x, int e, void *codes, int64_t n, void *stream) {
    QIM_REQUIRE(x && codes && n >= 0 && n % 4 == 0 && e >= 0 && e <= 254 && aligned16(x) && aligned16(codes),
                QIM_ERR_ARG, "qim_debug_e4m3_encode_scaled: bad arguments");
    if (n == 0) return QIM_OK;
    const int64_t n4 = n / 4;
    launch(k_debug_e4m3_scaled, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, as_stream(stream),
           (const uint32_t *)x, e, (uint32_t *)codes, n4);
    return check_launch("qim_debug_e4m3_encode_scaled");
}

extern "C" int qim_debug_bf16_round(const float *x, void *bits, int64_t n, void *stream) {
    QIM_REQUIRE(x && bits && n >= 0, QIM_ERR_ARG, "qim_debug_bf16_round: bad arguments");
    if (n == 0) return QIM_OK;
    launch(k_debug_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       as_stream(stream), x, (uint16_t *)bits, n);
    return check_launch("qim_debug_bf16_round");
}

extern "C" int qim_debug_mfma_tile(const void *a, const void *b, const void *sa, const void *sb,
                                   float *out, void *stream) {
    QIM_REQUIRE(a && b && sa && sb && out, QIM_ERR_ARG, "qim_debug_mfma_tile: null pointer");
    QIM_REQUIRE(aligned16(a) && aligned16(b), QIM_ERR_LAYOUT, "qim_debug_mfma_tile: a, b must be 16-byte aligned");
    launch(k_debug_mfma, dim3(1), dim3(64), 0, as_stream(stream), (const uint8_t *)a,
                       (const uint8_t *)b, (const uint8_t *)sa, (const uint8_t *)sb, out);
    return check_launch("qim_debug_mfma_tile");
}
