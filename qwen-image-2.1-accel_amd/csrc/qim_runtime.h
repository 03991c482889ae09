// Host-side helpers of the libqim C ABI: error reporting and argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qim.h"

namespace qim {

// Records a message for qim_last_error() and returns `code`.
int fail(int code, const char *fmt, ...);

// Returns QIM_OK, or QIM_ERR_LAUNCH with the HIP error of the last launch.
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
int reserve_lds(const void *fn, int bytes, bool (&done)[QIM_MAX_DEVICES], const char *who);

}  // namespace qim

#define QIM_REQUIRE(cond, code, ...)                 \
    do {                                             \
        if (!(cond)) return ::qim::fail((code), __VA_ARGS__); \
    } while (0)
