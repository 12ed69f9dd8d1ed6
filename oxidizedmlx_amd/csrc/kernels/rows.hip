// rows.hip — row-wise reductions over the last axis of a row-major f32
// matrix: softmax, scaled-masked softmax, LayerNorm, RMSNorm and the VJPs of
// softmax / LayerNorm / RMSNorm.
//
// Reference semantics (crates/mlx-core/src/cpu_kernels.rs):
//   softmax               :276-315   m = max; e = exp(x - m); s = sum e; y = e / s
//   scaled_masked_softmax :671-712   x*scale, -1e9 where causal && col > row, softmax
//   layer_norm            :338-363   mean; var = mean((x-mean)^2); y = (x-mean)/sqrt(var+eps)
//   rms_norm              :647-669   y = x / sqrt(mean(x^2) + eps)
//   softmax_vjp           :515-553   dx = s * (dy - sum(dy*s))
//   layer_norm_vjp        :403-454
//   rms_norm_vjp          :462-510
// The arithmetic per element is the reference's (divide where it divides, no
// contraction into FMA); only the summation order differs (per-lane partial
// sums, then a butterfly across the wavefront and across waves). The
// per-element divisions by a row's sum / standard deviation / rms use the
// row's reciprocal plus one exact-remainder correction (div_by), which yields
// the same correctly rounded quotient as a division for normal values.
//
// Layout / launch (CDNA4, wave64): a row is owned by WPR wavefronts (64*WPR
// lanes). Each lane keeps NV vectors of VEC floats of the row in VGPRs, so
// the row is read from HBM once and written once. Lane t of the row reads
// vector j at element (j*64*WPR + t)*VEC: consecutive lanes touch consecutive
// 16-byte words (dwordx4, fully coalesced). A 256-thread workgroup holds
// 4/WPR rows. Rows longer than 64*WPR*NV*VEC fall back to a streaming
// kernel that re-reads the row (three passes).
#include "../common.hpp"
#include "../kernels.hpp"
#include "device_math.hpp"

#include <algorithm>

#pragma clang fp contract(off)

namespace mlxhip {
namespace {

constexpr int WAVE = 64;
constexpr int BLOCK = 256;

using dev::div_by;
using dev::wave_max;
using dev::wave_sum;

// The row divisors here are >= 1 (softmax) or square roots of a sum plus
// eps, so 1/d is normal unless d overflowed to +inf (handled by
// shared_divisor).
__device__ inline void row_divisor(float& d, float& r) { dev::shared_divisor(d, r); }

// Reductions across the WPR waves that share a row. Each reduction of a
// kernel has its own LDS slots (`slot`: WPR floats, or pairs), written once
// and read once, so one barrier per reduction suffices: nothing can
// overwrite a slot another wave has yet to read. Every lane of the row gets
// the same value.
template <int WPR, bool MAX>
__device__ inline float row_reduce(float v, float* slot, int wave_in_row, int lane) {
    v = MAX ? wave_max(v) : wave_sum(v);
    if constexpr (WPR > 1) {
        if (lane == 0) slot[wave_in_row] = v;
        __syncthreads();
        float r = slot[0];
#pragma unroll
        for (int w = 1; w < WPR; ++w) r = MAX ? fmaxf(r, slot[w]) : r + slot[w];
        v = r;
    }
    return v;
}

// Softmax statistics of a row in one exchange: each lane holds (m, s) with
// s = sum of exp(x - m) over its values; two pairs merge as
// m = max(m1, m2), s = s1 exp(m1 - m) + s2 exp(m2 - m). Butterfly inside
// the wave, then one LDS exchange across the row's waves (pairs in `slot`,
// 2 * WPR floats).
__device__ inline void merge_max_sum(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    // exp of the (non-positive) differences; an empty side (s = 0, m = -inf)
    // contributes nothing.
    const float a = m == -INFINITY ? 0.0f : s * __builtin_amdgcn_exp2f((m - mn) * 1.44269504088896340736f);
    const float b = m2 == -INFINITY ? 0.0f : s2 * __builtin_amdgcn_exp2f((m2 - mn) * 1.44269504088896340736f);
    m = mn;
    s = a + b;
}

template <int WPR>
__device__ inline void row_reduce_max_sum(float& m, float& s, float* slot, int wave_in_row, int lane) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) merge_max_sum(m, s, __shfl_xor(m, o, WAVE), __shfl_xor(s, o, WAVE));
    if constexpr (WPR > 1) {
        if (lane == 0) {
            slot[2 * wave_in_row] = m;
            slot[2 * wave_in_row + 1] = s;
        }
        __syncthreads();
        m = slot[0];
        s = slot[1];
#pragma unroll
        for (int w = 1; w < WPR; ++w) merge_max_sum(m, s, slot[2 * w], slot[2 * w + 1]);
    }
}

// LayerNorm statistics in one exchange (Chan, Golub and LeVeque's pairwise
// update): each lane holds (n, mean, M2) of its values, M2 the sum of
// squared deviations from that mean; two groups merge as
// mean = mean1 + (mean2 - mean1) n2 / n, M2 = M2a + M2b + (mean2 - mean1)^2 n1 n2 / n.
__device__ inline void merge_moments(float& n, float& mean, float& m2, float n2, float mean2, float m22) {
    const float nn = n + n2;
    if (nn == 0.0f) return;
    const float delta = mean2 - mean;
    const float f = n2 / nn;
    mean = mean + delta * f;
    m2 = m2 + m22 + delta * delta * (n * f);
    n = nn;
}

// merge_moments for two groups of the same count n: n2 / (n + n2) is then
// exactly 0.5, so this gives the same values without the division.
__device__ inline void merge_moments_equal(float& n, float& mean, float& m2, float mean2, float m22) {
    const float delta = mean2 - mean;
    mean = mean + delta * 0.5f;
    m2 = m2 + m22 + delta * delta * (n * 0.5f);
    n = n + n;
}

// EQUAL: every lane of the row holds the same number of values (whole rows),
// so each butterfly step merges equal counts.
template <int WPR, bool EQUAL = false>
__device__ inline void row_reduce_moments(float& n, float& mean, float& m2, float* slot, int wave_in_row, int lane) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        if constexpr (EQUAL)
            merge_moments_equal(n, mean, m2, __shfl_xor(mean, o, WAVE), __shfl_xor(m2, o, WAVE));
        else
            merge_moments(n, mean, m2, __shfl_xor(n, o, WAVE), __shfl_xor(mean, o, WAVE), __shfl_xor(m2, o, WAVE));
    }
    if constexpr (WPR > 1) {
        if (lane == 0) {
            slot[3 * wave_in_row] = n;
            slot[3 * wave_in_row + 1] = mean;
            slot[3 * wave_in_row + 2] = m2;
        }
        __syncthreads();
        if constexpr (EQUAL && (WPR & (WPR - 1)) == 0) {
            // Equal counts in every wave: a pairwise tree (waves 2i and 2i+1,
            // then the pairs) merges equal counts at every level, without
            // the division.
            float nn[WPR], mm[WPR], qq[WPR];
#pragma unroll
            for (int w = 0; w < WPR; ++w) nn[w] = slot[3 * w], mm[w] = slot[3 * w + 1], qq[w] = slot[3 * w + 2];
#pragma unroll
            for (int st = 1; st < WPR; st *= 2)
#pragma unroll
                for (int w = 0; w < WPR; w += 2 * st) merge_moments_equal(nn[w], mm[w], qq[w], mm[w + st], qq[w + st]);
            n = nn[0];
            mean = mm[0];
            m2 = qq[0];
        } else {
            n = slot[0];
            mean = slot[1];
            m2 = slot[2];
#pragma unroll
            for (int w = 1; w < WPR; ++w) merge_moments(n, mean, m2, slot[3 * w], slot[3 * w + 1], slot[3 * w + 2]);
        }
    }
}

// Rows whose vectors are not all present (EVEN false) read and write
// through a buffer descriptor over the row: a vector outside the row gets
// an offset past the descriptor's range, so it reads as zeros and its store
// is dropped, with no branch around the access (branches there made the
// compiler keep the whole row live across them and spill) and no memory
// traffic for it.
constexpr uint32_t ROW_OOB = 0xFFFFFF00u;   // past every row's range (rows are < 64 KiB here)
constexpr int ROW_BUF_FLAGS = 0x00020000;   // gfx9 buffer descriptor word 3 (32-bit data format)
constexpr int ROW_NT = 2;                   // cache policy: non-temporal

__device__ inline __amdgpu_buffer_rsrc_t row_rsrc(const float* row, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, bytes, ROW_BUF_FLAGS);
}

template <int VEC>
struct Vec;
template <>
struct Vec<4> {
    static __device__ inline void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, float* d) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 t = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, ROW_NT));
        d[0] = t[0]; d[1] = t[1]; d[2] = t[2]; d[3] = t[3];
    }
    static __device__ inline void store_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* d) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{d[0], d[1], d[2], d[3]}), r, off, 0,
                                               ROW_NT);
    }
    using T = float4;
    // Non-temporal loads: every input element is read exactly once (0.2-0.8
    // us less per [4096, 4096] row op from cold HBM than plain loads).
    static __device__ inline void load(const float* p, float* d) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
        d[0] = t[0]; d[1] = t[1]; d[2] = t[2]; d[3] = t[3];
    }
    // Non-temporal: the output is not read again by this kernel; streaming it
    // past the caches kept 1-read/1-write rows at ~80% of HBM bandwidth
    // instead of ~62%.
    static __device__ inline void store(float* p, const float* d) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(f32x4{d[0], d[1], d[2], d[3]}, reinterpret_cast<f32x4*>(p));
    }
};
template <>
struct Vec<1> {
    static __device__ inline void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, float* d) {
        d[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, ROW_NT));
    }
    static __device__ inline void store_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* d) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, d[0]), r, off, 0, ROW_NT);
    }
    static __device__ inline void load(const float* p, float* d) { d[0] = __builtin_nontemporal_load(p); }
    static __device__ inline void store(float* p, const float* d) { __builtin_nontemporal_store(d[0], p); }
};

// a: x (forward) or dy (VJP); b: second operand of a VJP (softmax output s,
// or the forward input x). p: eps or scale. EVEN: every row of the grid
// exists and holds exactly NV * VEC * 64 * WPR columns, so no element needs
// a bounds predicate.
// Single-input ops are held to 128 VGPRs so four 256-thread workgroups (16
// waves) are resident per CU: a [4096, 4096] problem is 1024 workgroups, i.e.
// exactly one round on 256 CUs.
template <int OP, int WPR, int NV, int VEC, bool EVEN>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(
    (OP == ROW_SOFTMAX_VJP || OP == ROW_LAYERNORM_VJP || OP == ROW_RMSNORM_VJP) ? 2 : 4))) void row_kernel(const float* __restrict__ a,
                                                    const float* __restrict__ b,
                                                    float* __restrict__ y, int64_t rows,
                                                    int cols, float p, int causal) {
    constexpr int ROWS_PER_BLOCK = BLOCK / (WAVE * WPR);
    constexpr int TPR = WAVE * WPR;  // threads per row
    constexpr int N = NV * VEC;
    constexpr bool TWO = (OP == ROW_SOFTMAX_VJP || OP == ROW_LAYERNORM_VJP || OP == ROW_RMSNORM_VJP);
    // Up to four reductions per kernel, each with its own slots (3 floats per
    // wave for the moment triples).
    __shared__ float red[4][ROWS_PER_BLOCK][WPR > 1 ? 3 * WPR : 1];

    const int tid = threadIdx.x;
    const int row_in_block = tid / TPR;
    const int t = tid % TPR;
    const int lane = tid % WAVE;
    const int wave_in_row = t / WAVE;
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + row_in_block;
    // Rows past the end still take part in the block barriers.
    const bool live = EVEN || row < rows;
    float* slot0 = red[0][row_in_block];
    float* slot1 = red[1][row_in_block];
    float* slot2 = red[2][row_in_block];
    float* slot3 = red[3][row_in_block];

    const float* ar = a + (live ? row : 0) * (int64_t)cols;
    const float* br = TWO ? b + (live ? row : 0) * (int64_t)cols : nullptr;

    float v[N];
    float w[TWO ? N : 1];
    bool ok[NV];
    // Without EVEN, vectors outside the row read as zeros (row_rsrc).
    const int row_bytes = live ? cols * 4 : 0;
    const __amdgpu_buffer_rsrc_t ra = row_rsrc(ar, row_bytes);
    const __amdgpu_buffer_rsrc_t rb = row_rsrc(TWO ? br : ar, row_bytes);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * TPR + t) * VEC;
        ok[j] = EVEN || (live && c < cols);
        if constexpr (EVEN) {
            Vec<VEC>::load(ar + c, &v[j * VEC]);
            if constexpr (TWO) Vec<VEC>::load(br + c, &w[j * VEC]);
        } else {
            const uint32_t off = ok[j] ? 4u * (uint32_t)c : ROW_OOB;
            Vec<VEC>::load_buf(ra, off, &v[j * VEC]);
            if constexpr (TWO) Vec<VEC>::load_buf(rb, off, &w[j * VEC]);
        }
    }
    const float d = (float)cols;

    if constexpr (OP == ROW_SOFTMAX || OP == ROW_SCALED_MASKED_SOFTMAX) {
        if constexpr (OP == ROW_SCALED_MASKED_SOFTMAX) {
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const int c = (j * TPR + t) * VEC + e;
                    float x = v[j * VEC + e] * p;
                    if (causal && (int64_t)c > row) x = -1e9f;
                    v[j * VEC + e] = x;
                }
        }
        // Lane statistics (m, s = sum exp(x - m)) merged across the row in
        // one exchange; then y = exp(x - m_row) / s_row, each lane's stored
        // exp(x - m_lane) rescaled by exp(m_lane - m_row). exp(d) is
        // 2^(d log2 e) on arguments d <= 0: relative error ~|d| * 2^-24 plus
        // one v_exp_f32 ulp per factor, far inside the 1e-5 tolerance, at a
        // quarter of expf's VALU cost.
        float ml = -INFINITY;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (ok[j])
#pragma unroll
                for (int e = 0; e < VEC; ++e) ml = fmaxf(ml, v[j * VEC + e]);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                // A lane whose values are all -inf adds nothing (its exps are
                // 0 against any finite row maximum); a row that is all -inf
                // still ends as NaN, as exp(-inf - -inf) makes it in the reference.
                float ex = (ok[j] && ml != -INFINITY)
                               ? __builtin_amdgcn_exp2f((v[j * VEC + e] - ml) * 1.44269504088896340736f)
                               : 0.0f;
                v[j * VEC + e] = ex;
                s += ex;
            }
        float m = ml;
        row_reduce_max_sum<WPR>(m, s, slot0, wave_in_row, lane);
        const float scale = ml == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml - m) * 1.44269504088896340736f);
        float r;
        row_divisor(s, r);
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = div_by(v[j] * scale, s, r);
    } else if constexpr (OP == ROW_LAYERNORM) {
        // Lane moments (count, mean, sum of squared deviations) by an exact
        // two-pass over the lane's values, merged across the row in one
        // exchange; var = M2 / d as the reference's biased variance.
        float cnt = 0.0f, ls = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (ok[j]) {
                cnt += (float)VEC;
#pragma unroll
                for (int e = 0; e < VEC; ++e) ls += v[j * VEC + e];
            }
        // Whole rows: cnt is N, a power of two, and ls * (1 / N) is ls / N exactly.
        float mean = (EVEN && (N & (N - 1)) == 0) ? ls * (1.0f / (float)N) : (cnt > 0.0f ? ls / cnt : 0.0f);
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (ok[j])
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    float dv = v[j * VEC + e] - mean;
                    q += dv * dv;
                }
        row_reduce_moments<WPR, EVEN>(cnt, mean, q, slot0, wave_in_row, lane);
        const float var = q / d;
        float sd = sqrtf(var + p), r;
        row_divisor(sd, r);
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = div_by(v[j] - mean, sd, r);
    } else if constexpr (OP == ROW_RMSNORM) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) s += v[j] * v[j];
        s = row_reduce<WPR, false>(s, slot0, wave_in_row, lane);
        float rms = sqrtf(s / d + p), r;
        row_divisor(rms, r);
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = div_by(v[j], rms, r);
    } else if constexpr (OP == ROW_SOFTMAX_VJP) {
        // v = dy, w = s
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) dot += v[j] * w[j];
        dot = row_reduce<WPR, false>(dot, slot0, wave_in_row, lane);
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = w[j] * (v[j] - dot);
    } else if constexpr (OP == ROW_LAYERNORM_VJP) {
        // v = dy, w = x
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) s += w[j];
        s = row_reduce<WPR, false>(s, slot0, wave_in_row, lane);
        const float mean = s / d;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (ok[j])
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    float dv = w[j * VEC + e] - mean;
                    q += dv * dv;
                }
        q = row_reduce<WPR, false>(q, slot1, wave_in_row, lane);
        const float var = q / d;
        const float inv_std = 1.0f / sqrtf(var + p);
        float sdy = 0.0f, sdx = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (ok[j])
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    float xh = (w[j * VEC + e] - mean) * inv_std;
                    w[j * VEC + e] = xh;
                    sdy += v[j * VEC + e];
                    sdx += v[j * VEC + e] * xh;
                }
        sdy = row_reduce<WPR, false>(sdy, slot2, wave_in_row, lane);
        sdx = row_reduce<WPR, false>(sdx, slot3, wave_in_row, lane);
        const float mdy = sdy / d, mdx = sdx / d;
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = inv_std * (v[j] - mdy - w[j] * mdx);
    } else if constexpr (OP == ROW_RMSNORM_VJP) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) s += w[j] * w[j];
        s = row_reduce<WPR, false>(s, slot0, wave_in_row, lane);
        const float inv_rms = 1.0f / sqrtf(s / d + p);
        float sdy = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            w[j] = w[j] * inv_rms;
            sdy += v[j] * w[j];
        }
        sdy = row_reduce<WPR, false>(sdy, slot1, wave_in_row, lane);
        const float m = sdy / d;
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = inv_rms * (v[j] - w[j] * m);
    }

    float* yr = y + (live ? row : 0) * (int64_t)cols;
    const __amdgpu_buffer_rsrc_t ry = row_rsrc(yr, row_bytes);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * TPR + t) * VEC;
        if constexpr (EVEN)
            Vec<VEC>::store(yr + c, &v[j * VEC]);
        else
            Vec<VEC>::store_buf(ry, ok[j] ? 4u * (uint32_t)c : ROW_OOB, &v[j * VEC]);
    }
}

// Streaming fallback for rows longer than the register-resident kernels hold:
// one 256-thread block per row, the row is read in three passes.
template <int OP>
__global__ __launch_bounds__(BLOCK) void row_stream_kernel(const float* __restrict__ a,
                                                           const float* __restrict__ b,
                                                           float* __restrict__ y, int64_t rows,
                                                           int64_t cols, float p, int causal) {
    __shared__ float red[BLOCK / WAVE];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid % WAVE, wv = tid / WAVE;
    const float* ar = a + row * cols;
    const float* br = b ? b + row * cols : nullptr;
    float* yr = y + row * cols;
    const float d = (float)cols;
    auto block_reduce = [&](float v, bool mx) -> float {
        v = mx ? wave_max(v) : wave_sum(v);
        __syncthreads();
        if (lane == 0) red[wv] = v;
        __syncthreads();
        float r = red[0];
        for (int w = 1; w < BLOCK / WAVE; ++w) r = mx ? fmaxf(r, red[w]) : r + red[w];
        return r;
    };
    auto xin = [&](int64_t c) -> float {
        float x = ar[c];
        if (OP == ROW_SCALED_MASKED_SOFTMAX) {
            x = x * p;
            if (causal && c > row) x = -1e9f;
        }
        return x;
    };
    if (OP == ROW_SOFTMAX || OP == ROW_SCALED_MASKED_SOFTMAX) {
        float m = -INFINITY;
        for (int64_t c = tid; c < cols; c += BLOCK) m = fmaxf(m, xin(c));
        m = block_reduce(m, true);
        float s = 0.0f;
        for (int64_t c = tid; c < cols; c += BLOCK) s += expf(xin(c) - m);
        s = block_reduce(s, false);
        for (int64_t c = tid; c < cols; c += BLOCK) yr[c] = expf(xin(c) - m) / s;
    } else if (OP == ROW_LAYERNORM || OP == ROW_LAYERNORM_VJP) {
        const float* xr = OP == ROW_LAYERNORM ? ar : br;
        float s = 0.0f;
        for (int64_t c = tid; c < cols; c += BLOCK) s += xr[c];
        const float mean = block_reduce(s, false) / d;
        float q = 0.0f;
        for (int64_t c = tid; c < cols; c += BLOCK) {
            float dv = xr[c] - mean;
            q += dv * dv;
        }
        const float var = block_reduce(q, false) / d;
        const float sd = sqrtf(var + p);
        if (OP == ROW_LAYERNORM) {
            for (int64_t c = tid; c < cols; c += BLOCK) yr[c] = (xr[c] - mean) / sd;
        } else {
            const float inv = 1.0f / sd;
            float sdy = 0.0f, sdx = 0.0f;
            for (int64_t c = tid; c < cols; c += BLOCK) {
                sdy += ar[c];
                sdx += ar[c] * ((xr[c] - mean) * inv);
            }
            const float mdy = block_reduce(sdy, false) / d;
            const float mdx = block_reduce(sdx, false) / d;
            for (int64_t c = tid; c < cols; c += BLOCK)
                yr[c] = inv * (ar[c] - mdy - ((xr[c] - mean) * inv) * mdx);
        }
    } else if (OP == ROW_RMSNORM || OP == ROW_RMSNORM_VJP) {
        const float* xr = OP == ROW_RMSNORM ? ar : br;
        float s = 0.0f;
        for (int64_t c = tid; c < cols; c += BLOCK) s += xr[c] * xr[c];
        s = block_reduce(s, false);
        if (OP == ROW_RMSNORM) {
            const float rms = sqrtf(s / d + p);
            for (int64_t c = tid; c < cols; c += BLOCK) yr[c] = xr[c] / rms;
        } else {
            const float inv = 1.0f / sqrtf(s / d + p);
            float sdy = 0.0f;
            for (int64_t c = tid; c < cols; c += BLOCK) sdy += ar[c] * (xr[c] * inv);
            const float m = block_reduce(sdy, false) / d;
            for (int64_t c = tid; c < cols; c += BLOCK) yr[c] = inv * (ar[c] - (xr[c] * inv) * m);
        }
    } else if (OP == ROW_SOFTMAX_VJP) {
        float dot = 0.0f;
        for (int64_t c = tid; c < cols; c += BLOCK) dot += ar[c] * br[c];
        dot = block_reduce(dot, false);
        for (int64_t c = tid; c < cols; c += BLOCK) yr[c] = br[c] * (ar[c] - dot);
    }
}

// Softmax / SoftmaxVjp along a non-last axis: one thread per (outer, inner)
// fibre walking `dim` with stride `inner` (adjacent threads read adjacent
// addresses). Same arithmetic as cpu_kernels.rs:293-313 / :538-550.
template <bool VJP>
__global__ __launch_bounds__(BLOCK) void fibre_softmax_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              float* __restrict__ y,
                                                              int64_t outer, int64_t dim,
                                                              int64_t inner) {
    for (int64_t f = (int64_t)blockIdx.x * BLOCK + threadIdx.x; f < outer * inner; f += (int64_t)gridDim.x * BLOCK) {
        const int64_t o = f / inner, i = f % inner;
        const int64_t base = o * dim * inner + i;
        if (!VJP) {
            float m = -INFINITY;
            for (int64_t d = 0; d < dim; ++d) m = fmaxf(m, a[base + d * inner]);
            float s = 0.0f;
            for (int64_t d = 0; d < dim; ++d) s += expf(a[base + d * inner] - m);
            for (int64_t d = 0; d < dim; ++d) y[base + d * inner] = expf(a[base + d * inner] - m) / s;
        } else {
            float dot = 0.0f;
            for (int64_t d = 0; d < dim; ++d) dot += a[base + d * inner] * b[base + d * inner];
            for (int64_t d = 0; d < dim; ++d)
                y[base + d * inner] = b[base + d * inner] * (a[base + d * inner] - dot);
        }
    }
}

template <int OP, int WPR, int NV, int VEC>
int launch_rows(const float* a, const float* b, float* y, int64_t rows, int64_t cols, float p,
                int causal, hipStream_t s) {
    constexpr int RPB = BLOCK / (WAVE * WPR);
    const int64_t grid = ceil_div(rows, RPB);
    if (cols == (int64_t)NV * VEC * WAVE * WPR && rows % RPB == 0)
        hipLaunchKernelGGL((row_kernel<OP, WPR, NV, VEC, true>), dim3((unsigned)grid), dim3(BLOCK), 0,
                           s, a, b, y, rows, (int)cols, p, causal);
    else
        hipLaunchKernelGGL((row_kernel<OP, WPR, NV, VEC, false>), dim3((unsigned)grid), dim3(BLOCK), 0,
                           s, a, b, y, rows, (int)cols, p, causal);
    return launch_check("row_kernel");
}

template <int OP>
int dispatch_rows(const float* a, const float* b, float* y, int64_t rows, int64_t cols, float p,
                  int causal, hipStream_t s, int force_wpr) {
    const bool two = (OP == ROW_SOFTMAX_VJP || OP == ROW_LAYERNORM_VJP || OP == ROW_RMSNORM_VJP);
    const bool vec4 = (cols % 4 == 0) && (reinterpret_cast<uintptr_t>(a) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                      (!two || reinterpret_cast<uintptr_t>(b) % 16 == 0);
    if (vec4) {
        // force_wpr: 0 = automatic, else waves per row (1, 2 or 4) for tuning.
        if (force_wpr <= 1) {
            if (cols <= 256) return launch_rows<OP, 1, 1, 4>(a, b, y, rows, cols, p, causal, s);
            if (cols <= 512) return launch_rows<OP, 1, 2, 4>(a, b, y, rows, cols, p, causal, s);
            if (cols <= 1024) return launch_rows<OP, 1, 4, 4>(a, b, y, rows, cols, p, causal, s);
            if (cols <= 2048) return launch_rows<OP, 1, 8, 4>(a, b, y, rows, cols, p, causal, s);
        }
        // 2049..4096 columns: four waves per row (16 values per lane). On
        // [4096, 4096] with cold HBM this measured 24.3 / 24.0 / 23.4 us for
        // softmax / LayerNorm / RMSNorm against 25.8 / 24.6 / 24.6 us with one
        // wave per row and 24.9 / 23.9 / 24.2 us with two: a shorter chain of
        // arithmetic per wave after its loads land.
        const int wpr = force_wpr ? force_wpr : 4;
        if (cols <= 4096) {
            if (wpr == 1) return launch_rows<OP, 1, 16, 4>(a, b, y, rows, cols, p, causal, s);
            if (wpr == 2) return launch_rows<OP, 2, 8, 4>(a, b, y, rows, cols, p, causal, s);
            return launch_rows<OP, 4, 4, 4>(a, b, y, rows, cols, p, causal, s);
        }
        if (cols <= 8192) return launch_rows<OP, 4, 8, 4>(a, b, y, rows, cols, p, causal, s);
        if (cols <= 16384) return launch_rows<OP, 4, 16, 4>(a, b, y, rows, cols, p, causal, s);
    } else {
        if (cols <= 256) return launch_rows<OP, 4, 1, 1>(a, b, y, rows, cols, p, causal, s);
        if (cols <= 1024) return launch_rows<OP, 4, 4, 1>(a, b, y, rows, cols, p, causal, s);
        if (cols <= 4096) return launch_rows<OP, 4, 16, 1>(a, b, y, rows, cols, p, causal, s);
    }
    hipLaunchKernelGGL((row_stream_kernel<OP>), dim3((unsigned)rows), dim3(BLOCK), 0, s, a, b, y,
                       rows, cols, p, causal);
    return launch_check("row_stream_kernel");
}

int row_force_wpr() {
    static int v = [] {
        const char* e = getenv("MLXHIP_ROW_WPR");
        return e ? atoi(e) : 0;
    }();
    return v;
}

}  // namespace

int row_op(int op, const float* a, const float* b, float* y, int64_t rows, int64_t cols, float p,
           int causal, hipStream_t s) {
    if (rows == 0 || cols == 0) return MLXHIP_OK;
    if (rows < 0 || cols < 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "row op: negative size");
    if (rows > (int64_t)INT32_MAX) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "row op: too many rows");
    if (cols > INT32_MAX) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "row op: row too long");
    // Rows are independent: a long non-causal batch runs as launches of at
    // most ROW_CHUNK rows, so no grid (up to 256 work-items per row) exceeds
    // the 32-bit work-item count of a dispatch. A causal mask is indexed by
    // the row, and causal score matrices are far below that size.
    constexpr int64_t ROW_CHUNK = int64_t(1) << 22;
    if (rows > ROW_CHUNK && !causal) {
        for (int64_t r0 = 0; r0 < rows; r0 += ROW_CHUNK) {
            const int64_t off = r0 * cols, n = std::min(ROW_CHUNK, rows - r0);
            MLXHIP_TRY(row_op(op, a + off, b ? b + off : nullptr, y + off, n, cols, p, 0, s));
        }
        return MLXHIP_OK;
    }
    // MLXHIP_ROW_WPR forces the waves per row (tuning); 0 / unset = automatic.
    const int fw = row_force_wpr();
    switch (op) {
        case ROW_SOFTMAX: return dispatch_rows<ROW_SOFTMAX>(a, b, y, rows, cols, p, causal, s, fw);
        case ROW_SCALED_MASKED_SOFTMAX:
            return dispatch_rows<ROW_SCALED_MASKED_SOFTMAX>(a, b, y, rows, cols, p, causal, s, fw);
        case ROW_LAYERNORM: return dispatch_rows<ROW_LAYERNORM>(a, b, y, rows, cols, p, causal, s, fw);
        case ROW_RMSNORM: return dispatch_rows<ROW_RMSNORM>(a, b, y, rows, cols, p, causal, s, fw);
        case ROW_SOFTMAX_VJP:
            return dispatch_rows<ROW_SOFTMAX_VJP>(a, b, y, rows, cols, p, causal, s, fw);
        case ROW_LAYERNORM_VJP:
            return dispatch_rows<ROW_LAYERNORM_VJP>(a, b, y, rows, cols, p, causal, s, fw);
        case ROW_RMSNORM_VJP:
            return dispatch_rows<ROW_RMSNORM_VJP>(a, b, y, rows, cols, p, causal, s, fw);
        default: return fail(MLXHIP_ERR_INVALID_ARGUMENT, "row op: unknown op %d", op);
    }
}

int fibre_softmax(bool vjp, const float* a, const float* b, float* y, int64_t outer, int64_t dim,
                  int64_t inner, hipStream_t s) {
    const int64_t n = outer * inner;
    if (n == 0 || dim == 0) return MLXHIP_OK;
    const int64_t grid = std::min<int64_t>(ceil_div(n, BLOCK), int64_t(1) << 18);  // grid-stride beyond
    if (vjp)
        hipLaunchKernelGGL((fibre_softmax_kernel<true>), dim3((unsigned)grid), dim3(BLOCK), 0, s, a,
                           b, y, outer, dim, inner);
    else
        hipLaunchKernelGGL((fibre_softmax_kernel<false>), dim3((unsigned)grid), dim3(BLOCK), 0, s,
                           a, b, y, outer, dim, inner);
    return launch_check("fibre_softmax_kernel");
}

}  // namespace mlxhip
