// device_math.hpp — device helpers shared by the row, decode and attention
// kernels: wave64 reductions, the reference's sigmoid, and division of many
// values by one shared divisor.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mlxhip {
namespace dev {

constexpr int WAVE = 64;

// Butterfly reductions over the 64 lanes of a wavefront; every lane gets the
// result (fixed order, so deterministic).
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// sigmoid of crates/mlx-core/src/cpu_kernels.rs:104-106: 1 / (1 + exp(-x)).
__device__ inline float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// x / d for a divisor d shared by many values, given r = 1 / d (one IEEE
// division): q = x * r, then one Markstein correction with the exact
// remainder fma(-q, d, x). With r correctly rounded this returns the
// correctly rounded quotient -- the reference's x / d -- whenever the
// quotient and x are normal numbers (subnormal quotients may differ by one
// unit in the last place).
__device__ inline float div_by(float x, float d, float r) {
    const float q = x * r;
    return __builtin_fmaf(__builtin_fmaf(-q, d, x), r, q);
}

// r = 1 / d for div_by. A divisor that overflowed to +inf becomes (d = 1,
// r = 0), which gives x / inf = 0 for finite x and NaN for infinite x, as the
// division does.
__device__ inline void shared_divisor(float& d, float& r) {
    r = 1.0f / d;
    if (__builtin_isinf(d)) {
        d = 1.0f;
        r = 0.0f;
    }
}

}  // namespace dev
}  // namespace mlxhip
