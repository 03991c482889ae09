// Host-side helpers of the libqim C ABI: error reporting and argument checks.
#pragma once

#include <atomic>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>
#include <type_traits>
#include <utility>

#include "qim.h"

namespace qim {

// Records a message for qim_last_error() and returns `code`.
int fail(int code, const char *fmt, ...);

// First failed launch of the current entry point on this host thread
// (hipSuccess if none); launch() sets it, check_launch() reads and resets it.
hipError_t &launch_error();

// kernel<<<grid, block, shmem, stream>>>(args...) through hipLaunchKernel,
// whose return value is the status of this launch alone.  (hipGetLastError
// after a triple-chevron launch would also report an earlier failure of any
// runtime call on this thread, torch's included, as this launch's.)
template <typename... P, size_t... I>
hipError_t launch_packed(const void *fn, dim3 grid, dim3 block, size_t shmem, hipStream_t stream,
                         std::tuple<P...> &vals, std::index_sequence<I...>) {
    void *ptrs[sizeof...(P) > 0 ? sizeof...(P) : 1] = {static_cast<void *>(&std::get<I>(vals))...};
    return hipLaunchKernel(fn, grid, block, ptrs, shmem, stream);
}
template <typename... P, typename... A>
void launch(void (*kernel)(P...), dim3 grid, dim3 block, size_t shmem, hipStream_t stream, A &&...args) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    std::tuple<std::decay_t<P>...> vals(static_cast<std::decay_t<P>>(args)...);
    const hipError_t e = launch_packed(reinterpret_cast<const void *>(kernel), grid, block, shmem, stream, vals,
                                       std::index_sequence_for<P...>{});
    if (e != hipSuccess && launch_error() == hipSuccess) launch_error() = e;
}

// QIM_OK, or QIM_ERR_LAUNCH naming `what` and the first failed launch of this
// entry point (whose error is then cleared from HIP's per-thread state, so it
// is reported once, here).
int check_launch(const char *what);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device, cached per device (0 if unknown).
int device_cus();

// Lets kernel `fn` use `bytes` of dynamic LDS on the current device (HIP
// needs this above 64 KiB).  `done` is the caller's per-device record, so
// the attribute is set once per device and kernel.  QIM_OK, or
// QIM_ERR_LAUNCH with a message naming `who`.
constexpr int QIM_MAX_DEVICES = 64;
int reserve_lds(const void *fn, int bytes, std::atomic<bool> (&done)[QIM_MAX_DEVICES], const char *who);

}  // namespace qim

#define QIM_REQUIRE(cond, code, ...)                 \
    do {                                             \
        if (!(cond)) return ::qim::fail((code), __VA_ARGS__); \
    } while (0)
