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

// Allocation-failure hook (mlxhip_debug_fail_allocations, or the
// environment variable MLXHIP_FAIL_ALLOC_AFTER=n read at the first device
// allocation): true when the device allocation about to be made must fail.
// Every device allocation of the library asks first.
bool forced_alloc_failure();

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

// Per-stream device workspace for kernels that need scratch (split-K
// partials, padded operand copies, reduction partials). Slot `slot` of
// stream `s` (and of the current device) is one cached block that grows on
// demand and is reused by every later call on that stream: work on one
// stream runs in order, so a block is never in use by two kernels at once,
// and no call allocates once the block is large enough. A block that is
// outgrown is retired, not freed (a HIP graph recorded earlier may still name
// it); retired and live blocks are released by release_stream_workspaces(s)
// after `s` has drained. Calls on different streams use different blocks.
enum WsSlot { WS_PACK = 0, WS_SPLITK = 1, WS_REDUCE = 2, WS_ATTN = 3 };
int stream_workspace(hipStream_t s, int slot, size_t bytes, void** out);
void release_stream_workspaces(hipStream_t s);

}  // namespace mlxhip
