// common.hpp — shared host-side plumbing of the mlx-hip library: status codes,
// per-thread error messages, HIP error mapping, device initialisation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mlxhip.h"

namespace mlxhip {

// Per-thread message of the last failure (mlxhip_last_error).
std::string& last_error();

// Records a failure and returns its status code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Records MlxError::ShapeMismatch{expected, got} (crates/mlx-core/src/lib.rs:40-41):
// the message "[context: ]Shape mismatch: expected [..], got [..]" and both
// shapes, which mlxhip_last_shape_mismatch returns. Returns
// MLXHIP_ERR_SHAPE_MISMATCH.
int fail_shape(std::vector<int64_t> expected, std::vector<int64_t> got, const char* context = nullptr);

// Maps a HIP runtime error onto MlxError::FfiFailed with the call site.
int hip_fail(hipError_t e, const char* what);

#define MLXHIP_HIP(call)                                              \
    do {                                                              \
        hipError_t e_ = (call);                                       \
        if (e_ != hipSuccess) return ::mlxhip::hip_fail(e_, #call);   \
    } while (0)

#define MLXHIP_TRY(expr)              \
    do {                              \
        int rc_ = (expr);             \
        if (rc_ != MLXHIP_OK) return rc_; \
    } while (0)

// Makes sure the calling thread has an initialised device (device 0 unless
// mlxhip_init chose another). Returns MLXHIP_ERR_BACKEND_UNAVAILABLE without
// a GPU.
int ensure_device();

// Checks the launch that was just issued.
inline int launch_check(const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, kernel);
    return MLXHIP_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Stream-ordered scratch: allocated on `s`, returned to the device's memory
// pool on `s` after every kernel enqueued before the destructor has run.
struct StreamBuf {
    void* p = nullptr;
    hipStream_t s;
    explicit StreamBuf(hipStream_t st) : s(st) {}
    int alloc(size_t bytes) {
        static std::once_flag keep[64];
        int dev = 0;
        if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
            std::call_once(keep[dev], [dev] {
                // Keep freed blocks in the pool instead of returning them to the
                // driver at every synchronisation.
                hipMemPool_t pool;
                if (hipDeviceGetDefaultMemPool(&pool, dev) == hipSuccess) {
                    uint64_t hi = UINT64_MAX;
                    (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &hi);
                }
            });
        }
        MLXHIP_HIP(hipMallocAsync(&p, bytes ? bytes : 16, s));
        return MLXHIP_OK;
    }
    ~StreamBuf() {
        if (p) (void)hipFreeAsync(p, s);
    }
};

}  // namespace mlxhip
