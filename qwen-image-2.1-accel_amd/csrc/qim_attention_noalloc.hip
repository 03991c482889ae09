// qim_attention_noalloc: the attention core with its workspace in a buffer the
// library owns, for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops).  The workspace of qim_attention (the
// V^T tiles, and the partial rows of work items split over key ranges) lives
// in `scratch`, a file-scope device array of QIM_ATTENTION_NOALLOC_MAX_BYTES.
// Each device holds its own copy from the first call on it until the process
// ends; its address on each device is resolved once, with that device
// current, and kept in g_scratch.  Every call on a device reuses the array, so
// calls that overlap on one device race.  No call needs the array cleared:
// every byte a call reads was written earlier in the same call (k_attn_vt
// writes whole V^T tiles, zeros past the last key; each split chunk writes its
// partial rows before the merge pass reads them).
#include <mutex>

#include "qim_attention.h"
#include "qim_runtime.h"

namespace qim {

static __device__ __align__(256) uint8_t scratch[QIM_ATTENTION_NOALLOC_MAX_BYTES];

static std::mutex g_scratch_mu;
static void *g_scratch[QIM_MAX_DEVICES];

// Device address of `scratch` on the current device (hipGetSymbolAddress on
// the first call per device; the array's host-side name is not a device
// address and is never passed to a kernel).
static int scratch_on_current_device(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= QIM_MAX_DEVICES)
        return fail(QIM_ERR_LAUNCH, "qim_attention_noalloc: no usable current device");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(QIM_ERR_LAUNCH, "qim_attention_noalloc: cannot resolve the scratch buffer on device %d: %s",
                        dev, hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return QIM_OK;
}

}  // namespace qim

using namespace qim;

extern "C" int qim_attention_noalloc(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                                     int64_t ldv, void *o, int64_t ldo, int64_t B, int64_t S, int64_t T, int64_t H,
                                     int64_t D, float scale, void *stream) {
    const char *who = "qim_attention_noalloc";
    QIM_REQUIRE(q && k && v && o, QIM_ERR_ARG, "%s: null pointer (v is required: the scratch buffer holds no V^T)",
                who);
    QIM_REQUIRE(B > 0 && S > 0 && T > 0 && H > 0, QIM_ERR_SHAPE, "%s: empty problem", who);
    QIM_REQUIRE(B < 65536 && H < 65536 && S < (1 << 30) && T < (1 << 30), QIM_ERR_SHAPE, "%s: too large", who);
    const int64_t need = att_plan(B, S, T, H).total();
    QIM_REQUIRE(need <= QIM_ATTENTION_NOALLOC_MAX_BYTES, QIM_ERR_SHAPE,
                "%s: this problem needs %lld bytes of workspace, above the %lld-byte scratch buffer "
                "(use qim_attention with a workspace of qim_attention_workspace_bytes)",
                who, (long long)need, (long long)QIM_ATTENTION_NOALLOC_MAX_BYTES);
    void *ws = nullptr;
    if (const int rc = scratch_on_current_device(&ws)) return rc;
    return attention_run(who, q, ldq, k, ldk, v, ldv, o, ldo, nullptr, nullptr, 0, ws,
                         QIM_ATTENTION_NOALLOC_MAX_BYTES, B, S, T, H, D, scale, stream);
}
