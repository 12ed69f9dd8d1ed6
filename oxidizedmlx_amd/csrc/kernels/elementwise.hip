// elementwise.hip — HBM-streaming kernels: the fused elementwise chain,
// transposes/permutations, broadcast, reductions, type casts and the gather /
// slice / rotary kernels the graph needs.
//
// Elementwise semantics follow crates/mlx-core/src/cpu_kernels.rs:
//   Add/Sub/Mul/Div :24-27,114-128   Neg/Exp/Log :28-39   Sqrt :85-88
//   Silu :51-54 with sigmoid :104-106   Gelu (tanh approx.) :55-67
//   SiluVjp :558-576   GeluVjp :582-606
// Contraction is off in this file, so x*w+b rounds twice exactly like the
// reference's two graph nodes; transcendental functions are the device
// libm's (ocml), not glibc's, so they can differ by an ulp or so.
//
// Streaming kernels move float4 (dwordx4) per lane, several per thread per
// grid-stride step so each wave keeps multiple 1 KiB loads in flight.
#include "../common.hpp"
#include "../kernels.hpp"
#include "device_math.hpp"

#include <algorithm>
#include <cstdlib>

#pragma clang fp contract(off)

namespace mlxhip {
namespace {

constexpr int BLOCK = 256;

// Per-element kernels walk [0, n) with a grid-stride loop and the host caps
// their grid at MAX_GRID workgroups (grid_for), so no launch exceeds the
// 32-bit work-item count of a dispatch, whatever the tensor size.
constexpr int64_t MAX_GRID = int64_t(1) << 18;
#define FOR_EACH_ELEMENT(i, n) \
    for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < (n); i += (int64_t)gridDim.x * BLOCK)

using dev::sigmoid_ref;

__device__ inline float gelu_ref(float x) {
    const float k = sqrtf(2.0f / 3.14159265358979323846f);
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

__device__ inline float silu_vjp_ref(float dy, float x) {
    const float sig = sigmoid_ref(x);
    return dy * sig * (1.0f + x * (1.0f - sig));
}

__device__ inline float gelu_vjp_ref(float dy, float x) {
    const float a = sqrtf(2.0f / 3.14159265358979323846f);
    const float b = 0.044715f;
    const float inner = a * (x + b * x * x * x);
    const float t = tanhf(inner);
    const float sech2 = 1.0f - t * t;
    const float dg = 0.5f * (1.0f + t) + 0.5f * x * sech2 * a * (1.0f + 3.0f * b * x * x);
    return dy * dg;
}

__device__ inline float apply(int op, float acc, float in) {
    switch (op) {
        case MLXHIP_EW_ADD: return acc + in;
        case MLXHIP_EW_SUB: return acc - in;
        case MLXHIP_EW_RSUB: return in - acc;
        case MLXHIP_EW_MUL: return acc * in;
        case MLXHIP_EW_DIV: return acc / in;
        case MLXHIP_EW_RDIV: return in / acc;
        case MLXHIP_EW_NEG: return -acc;
        case MLXHIP_EW_EXP: return expf(acc);
        case MLXHIP_EW_LOG: return logf(acc);
        case MLXHIP_EW_SQRT: return sqrtf(acc);
        case MLXHIP_EW_SILU: return acc * sigmoid_ref(acc);
        case MLXHIP_EW_GELU: return gelu_ref(acc);
        case MLXHIP_EW_SILU_VJP: return silu_vjp_ref(in, acc);
        case MLXHIP_EW_GELU_VJP: return gelu_vjp_ref(in, acc);
        default: return acc;
    }
}

__host__ __device__ inline bool ew_binary(int op) {
    return op == MLXHIP_EW_ADD || op == MLXHIP_EW_SUB || op == MLXHIP_EW_RSUB ||
           op == MLXHIP_EW_MUL || op == MLXHIP_EW_DIV || op == MLXHIP_EW_RDIV ||
           op == MLXHIP_EW_SILU_VJP || op == MLXHIP_EW_GELU_VJP;
}

// The whole program travels in kernel arguments, so every instruction field
// is wave-uniform (scalar registers) and the interpreter loop costs no VGPRs.
// period[i] > 0: input i holds `period` values repeated along the output
// (out index j reads in[j % period]; the tiling a right-aligned Broadcast
// makes), in float4 units in the vector kernel; 0: a full-size input.
struct EwProg {
    const float* in[MLXHIP_EW_MAX_INPUTS];
    int64_t period[MLXHIP_EW_MAX_INPUTS];
    int op[MLXHIP_EW_MAX_INSTR];
    int operand[MLXHIP_EW_MAX_INSTR];
    int n_instr;
    int scalar_mask;  // bit i: input i is one value for every element (vector kernel)
    // Optional (vector kernel): the output's three bf16 planes for the
    // split-f32 GEMM, in storage order (plane p at planes + p * plane), and
    // the flag word that receives gen when a value cannot be split.
    uint16_t* planes;
    int64_t plane;
    uint32_t* flag;
    uint32_t gen;
};

// The split-f32 GEMM's split of one f32 value (x6_split_kernel's
// arithmetic): hi = RN(x), mid = RN(x - hi), lo = RN(x - hi - mid), bf16
// round to nearest even; both differences are exact in f32. bad: hi is not
// finite (x is not, or rounds past the bf16 range).
__device__ inline void split3(float x, uint32_t& h, uint32_t& m, uint32_t& l, bool& bad) {
    const uint16_t hb = __builtin_bit_cast(uint16_t, (__bf16)x);
    const float r1 = x - __uint_as_float((uint32_t)hb << 16);
    const uint16_t mb = __builtin_bit_cast(uint16_t, (__bf16)r1);
    const float r2 = r1 - __uint_as_float((uint32_t)mb << 16);
    const uint16_t lb = __builtin_bit_cast(uint16_t, (__bf16)r2);
    bad |= !__builtin_isfinite(__uint_as_float((uint32_t)hb << 16));
    h = hb, m = mb, l = lb;
}

__device__ inline float4 apply4(int op, float4 a, float4 b) {
    return make_float4(apply(op, a.x, b.x), apply(op, a.y, b.y), apply(op, a.z, b.z), apply(op, a.w, b.w));
}

// NI inputs, U float4 per input per thread per grid-stride step. Every
// input's vectors are loaded before the program runs, so a thread has all
// NI * U loads in flight at once instead of one input's per instruction; the
// operand of each instruction is then picked by uniform (scalar) branches.
// PERIODIC: some inputs are periodic or scalar (prog.period / scalar_mask);
// their index is reduced modulo the period with 32-bit arithmetic (the host
// only sets PERIODIC when every vector index fits in 32 bits).
template <int NI, int U, bool NT, bool PERIODIC>
__global__ __launch_bounds__(BLOCK) void ew_chain_vec_kernel(EwProg prog, float* __restrict__ out,
                                                             int64_t n_vec) {
    const int64_t stride = (int64_t)gridDim.x * BLOCK * U;
    bool bad = false;  // a value the planes cannot hold (prog.planes)
    for (int64_t base = (int64_t)blockIdx.x * BLOCK * U + threadIdx.x; base < n_vec;
         base += stride) {
        float4 in[NI][U];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t idx = base + (int64_t)u * BLOCK;
                if (PERIODIC && (prog.scalar_mask >> i) & 1) {
                    const float v = prog.in[i][0];
                    in[i][u] = make_float4(v, v, v, v);
                } else if (PERIODIC && prog.period[i] > 0) {
                    const uint32_t j = (uint32_t)idx % (uint32_t)prog.period[i];
                    in[i][u] = idx < n_vec ? reinterpret_cast<const float4*>(prog.in[i])[j]
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
                } else if constexpr (NT) {
                    // Full-size inputs of a large chain are read exactly once.
                    typedef float f32x4 __attribute__((ext_vector_type(4)));
                    f32x4 v = {0.f, 0.f, 0.f, 0.f};
                    if (idx < n_vec) v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(prog.in[i]) + idx);
                    in[i][u] = make_float4(v[0], v[1], v[2], v[3]);
                } else {
                    in[i][u] = idx < n_vec ? reinterpret_cast<const float4*>(prog.in[i])[idx]
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        float4 acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = in[0][u];
        for (int k = 0; k < prog.n_instr; ++k) {
            const int op = prog.op[k];
            const int o = prog.operand[k];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                if (i == o) {
#pragma unroll
                    for (int u = 0; u < U; ++u) acc[u] = apply4(op, acc[u], in[i][u]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = base + (int64_t)u * BLOCK;
            if (idx < n_vec) {
                typedef float f32x4 __attribute__((ext_vector_type(4)));
                const f32x4 v = {acc[u].x, acc[u].y, acc[u].z, acc[u].w};
                if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out) + idx);
                else reinterpret_cast<f32x4*>(out)[idx] = v;
                if (prog.planes) {
                    uint32_t h[4], m[4], l[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) split3(v[e], h[e], m[e], l[e], bad);
                    uint2* hp = reinterpret_cast<uint2*>(prog.planes) + idx;
                    hp[0] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                    reinterpret_cast<uint2*>(prog.planes + prog.plane)[idx] =
                        make_uint2(m[0] | (m[1] << 16), m[2] | (m[3] << 16));
                    reinterpret_cast<uint2*>(prog.planes + 2 * prog.plane)[idx] =
                        make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
                }
            }
        }
    }
    // Every writer stores the same word, so the stores need no order.
    if (bad) *prog.flag = prog.gen;
}

// One float4 per input per thread: with more per thread, each instruction's
// uniform dispatch is repeated per component and the chain turns VALU-bound
// (SiLU(x*w+b) ran at 43% of HBM bandwidth with 4, 92% with 1).
template <int NI>
int launch_chain_vec(const EwProg& p, float* out, int64_t n_vec, bool periodic, hipStream_t s) {
    constexpr int U = 1;
    int64_t grid = ceil_div(n_vec, (int64_t)BLOCK * U);
    if (grid > 65536) grid = 65536;
    // A chain whose traffic is at least half the 256 MiB Infinity Cache
    // streams: non-temporal loads of its full-size inputs and non-temporal
    // stores.
    const bool stream = n_vec * 16 * (NI + 1) >= (int64_t(128) << 20);
    if (periodic)
        hipLaunchKernelGGL((ew_chain_vec_kernel<NI, U, false, true>), dim3((unsigned)grid), dim3(BLOCK), 0, s, p,
                           out, n_vec);
    else if (stream)
        hipLaunchKernelGGL((ew_chain_vec_kernel<NI, U, true, false>), dim3((unsigned)grid), dim3(BLOCK), 0, s, p,
                           out, n_vec);
    else
        hipLaunchKernelGGL((ew_chain_vec_kernel<NI, U, false, false>), dim3((unsigned)grid), dim3(BLOCK), 0, s, p,
                           out, n_vec);
    return launch_check("ew_chain_vec_kernel");
}

__global__ __launch_bounds__(BLOCK) void ew_chain_scalar_kernel(EwProg prog, float* __restrict__ out,
                                                                int64_t begin, int64_t n) {
    // Periods are in elements here.
    FOR_EACH_ELEMENT(j, n - begin) {
        const int64_t i = begin + j;
        auto at = [&](int in) {
            const int64_t p = prog.period[in];
            return prog.in[in][p > 0 ? i % p : i];
        };
        float acc = at(0);
        for (int k = 0; k < prog.n_instr; ++k) {
            const int op = prog.op[k];
            acc = apply(op, acc, ew_binary(op) ? at(prog.operand[k]) : 0.f);
        }
        out[i] = acc;
    }
}

// 2-D transpose through a padded 64x64 LDS tile (the +1 column breaks the
// bank conflicts of the column-wise read).
__global__ __launch_bounds__(BLOCK) void transpose2d_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t rows,
                                                            int64_t cols) {
    __shared__ float tile[64][65];
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
#pragma unroll
    for (int i = 0; i < 64; i += 4) {
        const int64_t r = r0 + ty + i, c = c0 + tx;
        if (r < rows && c < cols) tile[ty + i][tx] = x[r * cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 64; i += 4) {
        const int64_t c = c0 + ty + i, r = r0 + tx;
        if (r < rows && c < cols) y[c * rows + r] = tile[tx][ty + i];
    }
}

constexpr int MAXD = 8;
struct Dims {
    int64_t v[MAXD];
};

__global__ __launch_bounds__(BLOCK) void permute_kernel(const float* __restrict__ x,
                                                        float* __restrict__ y, Dims new_shape,
                                                        Dims old_stride_of_new, int ndim,
                                                        int64_t total) {
    FOR_EACH_ELEMENT(f, total) {
        int64_t rem = f, src = 0;
        for (int d = ndim - 1; d >= 0; --d) {
            const int64_t c = rem % new_shape.v[d];
            rem /= new_shape.v[d];
            src += c * old_stride_of_new.v[d];
        }
        y[f] = x[src];
    }
}

__global__ __launch_bounds__(BLOCK) void broadcast_kernel(const float* __restrict__ x,
                                                          float* __restrict__ y, Dims out_shape,
                                                          Dims in_stride, int out_ndim,
                                                          int64_t total) {
    FOR_EACH_ELEMENT(f, total) {
        int64_t rem = f, src = 0;
        for (int d = out_ndim - 1; d >= 0; --d) {
            const int64_t c = rem % out_shape.v[d];
            rem /= out_shape.v[d];
            src += c * in_stride.v[d];
        }
        y[f] = x[src];
    }
}

// ── gathers with 32-bit index arithmetic ────────────────────────────────
// out[u] = in[src(u)] over units of VEC floats: src is the sum over the
// output's axes of (coordinate of u on that axis) x (input stride of that
// axis, in units). The coordinates come from multiply-high division by
// invariant divisors (Granlund and Montgomery, PLDI 1994): for a divisor
// d >= 2 with l = ceil(log2 d), p = 31 + l and mul = ceil(2^p / d) < 2^32,
// floor(n / d) = umulhi(n, mul) >> (p - 32) for every 0 <= n < 2^31; d = 1 is
// taken as is. Used when every unit index and source offset fits 31 bits,
// in place of 64-bit divisions (tens of instructions each per axis).
struct Gather32 {
    int ndim;
    uint32_t dim[MAXD], mul[MAXD], shr[MAXD], stride[MAXD];
};

template <int VEC>
__global__ __launch_bounds__(BLOCK) void gather32_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                         Gather32 g, uint32_t total) {
    for (uint32_t u = blockIdx.x * BLOCK + threadIdx.x; u < total; u += gridDim.x * BLOCK) {
        uint32_t rem = u, src = 0;
        for (int d = g.ndim - 1; d >= 0; --d) {
            const uint32_t q = g.dim[d] == 1 ? rem : (__umulhi(rem, g.mul[d]) >> g.shr[d]);
            src += (rem - q * g.dim[d]) * g.stride[d];
            rem = q;
        }
        if constexpr (VEC == 4)
            reinterpret_cast<float4*>(y)[u] = reinterpret_cast<const float4*>(x)[src];
        else
            y[u] = x[src];
    }
}

// One thread per output element; sequential fold in the reference's order
// (reduce_along_axis, cpu_kernels.rs:166-195; Sum folds from -0.0), so the
// result is bit-identical to the CPU's. The fold is a chain of dependent
// adds, so each thread loads RED_U elements ahead and then folds them in
// order: the loads overlap instead of each waiting out a memory latency. One
// wave per workgroup spreads the (often few) outputs over more CUs; the
// grid is capped and strides over the outputs.
// KIND: 0 Sum, 1 Mean, 2 Max.
constexpr int RED_U = 64;
constexpr int RED_BLOCK = 64;

template <int KIND>
__device__ inline float fold(float v, float x) {
    return KIND == 2 ? fmaxf(v, x) : v + x;
}

template <int KIND>
__global__ __launch_bounds__(RED_BLOCK) void reduce_axis_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t outer, int64_t dim, int64_t inner) {
    for (int64_t f = (int64_t)blockIdx.x * RED_BLOCK + threadIdx.x; f < outer * inner;
         f += (int64_t)gridDim.x * RED_BLOCK) {
        const int64_t o = f / inner, i = f % inner;
        const float* p = x + o * dim * inner + i;
        float v = KIND == 2 ? -INFINITY : -0.0f;
        // Two register batches in turn: batch b is loaded while batch a is
        // folded and the other way round, so memory latency overlaps the chain
        // of dependent adds; neither batch is ever copied (a copy would wait for
        // its loads).
        const int64_t full = dim / (2 * RED_U) * (2 * RED_U);
        float a[RED_U], b[RED_U];
        if (full > 0) {
#pragma unroll
            for (int u = 0; u < RED_U; ++u) a[u] = p[(int64_t)u * inner];
        }
        for (int64_t d = 0; d < full; d += 2 * RED_U) {
#pragma unroll
            for (int u = 0; u < RED_U; ++u) b[u] = p[(d + RED_U + u) * inner];
#pragma unroll
            for (int u = 0; u < RED_U; ++u) v = fold<KIND>(v, a[u]);
            if (d + 2 * RED_U < full) {
#pragma unroll
                for (int u = 0; u < RED_U; ++u) a[u] = p[(d + 2 * RED_U + u) * inner];
            }
#pragma unroll
            for (int u = 0; u < RED_U; ++u) v = fold<KIND>(v, b[u]);
        }
        for (int64_t d = full; d < dim; ++d) v = fold<KIND>(v, p[d * inner]);
        if (KIND == 1) v = v / (float)dim;
        y[f] = v;
    }
}

// The same sequential fold for reductions over a long axis with few
// outputs (the bias gradients of a block: Sum over 2048 rows of [2048, N]).
// One thread per output leaves most CUs idle and each busy CU streaming its
// columns at the rate one CU can keep cache lines in flight. Here a
// workgroup owns COLS outputs of one outer index: its 256 threads copy
// chunks of RC_CH rows x COLS columns straight from memory into a ring of
// LDS slots (buffer loads with the LDS flag, 16 bytes per lane, RC_P chunks
// ahead), and COLS lanes of wave 0 fold each chunk in row order while the
// next ones arrive. Rows past the end read as zero (out of the buffer's
// range) and are never folded; columns past the end are never stored.
// Needs inner % 4 == 0, a 16-byte aligned x and a slab of under 2^32 bytes.
constexpr int RC_BLOCK = 256;

#define MLXHIP_LDS_AS __attribute__((address_space(3)))

// 16 bytes per lane from buffer offset `voff` into LDS at dst + 16 * lane.
// Inline assembly, so the compiler does not wait for these loads before
// every LDS read; the kernel waits for them itself (vmcnt, then a barrier).
__device__ inline void rc_lds_load16(__amdgpu_buffer_rsrc_t rsrc, MLXHIP_LDS_AS char* dst, uint32_t voff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(m0) : "memory");
}

template <int KIND, int COLS, int RC_CH, int RC_P, int FB>
__global__ __launch_bounds__(RC_BLOCK) void reduce_cols_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                               int64_t dim, int64_t inner, int64_t col_blocks) {
    constexpr int TPR = COLS / 4;                       // lanes per row
    constexpr int RPI = 64 / TPR;                       // rows per wave instruction (1 KiB)
    constexpr int RC_NB = RC_P + 1;
    constexpr int CHUNK_BYTES = RC_CH * COLS * 4;
    constexpr int L = CHUNK_BYTES / (RC_BLOCK * 16);    // loads per thread per chunk
    static_assert(L * RC_BLOCK * 16 == CHUNK_BYTES, "whole 1 KiB blocks per wave");
    // The ring; the vmcnt below assumes these loads are the only vector
    // memory operations in flight.
    __shared__ __align__(16) float ring[RC_NB][RC_CH * COLS];
    const int64_t o = blockIdx.x / col_blocks;
    const int64_t c0 = (blockIdx.x % col_blocks) * COLS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float* slab = x + o * dim * inner;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)slab, (short)0, (int)(uint32_t)(dim * inner * 4), 0x00020000);
    // Load l of a chunk: wave instruction q = l * 4 + wave covers rows
    // q * RPI .. q * RPI + RPI - 1 of the chunk; the lane's 16 bytes are
    // row lane / TPR, columns c0 + 4 * (lane % TPR) .. + 3.
    uint32_t voff[L];
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const int64_t row = (int64_t)(l * 4 + wave) * RPI + lane / TPR;
        voff[l] = (uint32_t)((row * inner + c0 + 4 * (lane % TPR)) * 4);
    }
    const uint32_t chunk_step = (uint32_t)(RC_CH * inner * 4);
    auto issue = [&](int ch) {
        MLXHIP_LDS_AS char* slot = (MLXHIP_LDS_AS char*)&ring[ch % RC_NB][0];
#pragma unroll
        for (int l = 0; l < L; ++l)
            rc_lds_load16(rsrc, slot + (l * 4 + wave) * 1024, voff[l] + (uint32_t)ch * chunk_step);
    };
    const int nch = (int)((dim + RC_CH - 1) / RC_CH);
    float v = KIND == 2 ? -INFINITY : -0.0f;
    for (int ch = 0; ch < RC_P; ++ch) issue(ch);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L * (RC_P - 1)) : "memory");
    __syncthreads();
    for (int c = 0; c < nch; ++c) {
        // Slot (c + P) % NB was folded in the previous pass, before the barrier.
        // Chunks past the end are issued too (every row out of range), so the
        // count of younger loads below is always L * (P - 1).
        issue(c + RC_P);
        if (tid < COLS) {
            const float* b = &ring[c % RC_NB][tid];
            const int rows = (int)std::min<int64_t>(RC_CH, dim - (int64_t)c * RC_CH);
            if (rows == RC_CH) {
                // Two register batches of FB rows in turn: batch B's LDS
                // reads are in flight while batch A is folded (the scheduling
                // barriers keep the compiler from sinking the reads to their
                // adds, which would expose the LDS latency on every pair).
                float a[FB], bb[FB];
#pragma unroll
                for (int i = 0; i < FB; ++i) a[i] = b[i * COLS];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int r = 0; r < RC_CH; r += 2 * FB) {
#pragma unroll
                    for (int i = 0; i < FB; ++i) bb[i] = b[(r + FB + i) * COLS];
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < FB; ++i) v = fold<KIND>(v, a[i]);
                    __builtin_amdgcn_sched_barrier(0);
                    if (r + 2 * FB < RC_CH) {
#pragma unroll
                        for (int i = 0; i < FB; ++i) a[i] = b[(r + 2 * FB + i) * COLS];
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < FB; ++i) v = fold<KIND>(v, bb[i]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                for (int i = 0; i < rows; ++i) v = fold<KIND>(v, b[i * COLS]);
            }
        }
        // This thread's loads of chunk c + 1 are done, then everyone's.
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L * (RC_P - 1)) : "memory");
        __syncthreads();
    }
    // Drain the loads past the end before the workgroup exits.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid < COLS && c0 + tid < inner) {
        if (KIND == 1) v = v / (float)dim;
        y[o * inner + c0 + tid] = v;
    }
}

// Sequential fold of all elements on one lane (bit-identical to the CPU fold).
__global__ void reduce_all_seq_kernel(int kind, const float* __restrict__ x, float* __restrict__ y,
                                      int64_t n) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float v = kind == 2 ? -INFINITY : -0.0f;
    for (int64_t i = 0; i < n; ++i) v = kind == 2 ? fmaxf(v, x[i]) : v + x[i];
    if (kind == 1) v = v / (float)n;
    y[0] = v;
}

// Tree reduction for large inputs (more than 65536 values): per-block
// partials, then one block folds them. The order of the additions differs
// from the sequential fold, so a sum or mean agrees with it to rounding.
__global__ __launch_bounds__(BLOCK) void reduce_partial_kernel(int kind, const float* __restrict__ x,
                                                               float* __restrict__ part, int64_t n) {
    __shared__ float sm[BLOCK];
    float v = kind == 2 ? -INFINITY : -0.0f;  // -0.0: a sum of -0.0s stays -0.0, as in the sequential fold
    for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n; i += (int64_t)gridDim.x * BLOCK)
        v = kind == 2 ? fmaxf(v, x[i]) : v + x[i];
    sm[threadIdx.x] = v;
    __syncthreads();
    for (int o = BLOCK / 2; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
            sm[threadIdx.x] = kind == 2 ? fmaxf(sm[threadIdx.x], sm[threadIdx.x + o])
                                        : sm[threadIdx.x] + sm[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = sm[0];
}

__global__ __launch_bounds__(BLOCK) void reduce_final_kernel(int kind, const float* __restrict__ part,
                                                             float* __restrict__ y, int np, int64_t n) {
    __shared__ float sm[BLOCK];
    float v = kind == 2 ? -INFINITY : -0.0f;
    for (int i = threadIdx.x; i < np; i += BLOCK) v = kind == 2 ? fmaxf(v, part[i]) : v + part[i];
    sm[threadIdx.x] = v;
    __syncthreads();
    for (int o = BLOCK / 2; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
            sm[threadIdx.x] = kind == 2 ? fmaxf(sm[threadIdx.x], sm[threadIdx.x + o])
                                        : sm[threadIdx.x] + sm[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) y[0] = kind == 1 ? sm[0] / (float)n : sm[0];
}

__device__ inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ __launch_bounds__(BLOCK) void cast_kernel(const void* __restrict__ x, int src,
                                                     void* __restrict__ y, int dst, int64_t n) {
    FOR_EACH_ELEMENT(i, n) {
        float v;
        if (src == MLXHIP_DTYPE_F32) v = static_cast<const float*>(x)[i];
        else if (src == MLXHIP_DTYPE_BF16) v = __uint_as_float((uint32_t)static_cast<const uint16_t*>(x)[i] << 16);
        else v = (float)static_cast<const _Float16*>(x)[i];
        if (dst == MLXHIP_DTYPE_F32) static_cast<float*>(y)[i] = v;
        else if (dst == MLXHIP_DTYPE_BF16) static_cast<uint16_t*>(y)[i] = f32_to_bf16_rne(v);
        else static_cast<_Float16*>(y)[i] = (_Float16)v;
    }
}

// Rust's `f as i32`: saturating, NaN -> 0.
__device__ inline int32_t f2i_sat(float f) {
    if (f != f) return 0;
    if (f >= 2147483647.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

__global__ __launch_bounds__(BLOCK) void embedding_kernel(const float* __restrict__ w,
                                                          const float* __restrict__ idx,
                                                          float* __restrict__ y, int64_t n_idx,
                                                          int64_t num_emb, int64_t dim) {
    FOR_EACH_ELEMENT(f, n_idx * dim) {
        const int64_t i = f / dim, d = f % dim;
        int64_t row = f2i_sat(idx[i]);
        row = row < 0 ? 0 : (row > num_emb - 1 ? num_emb - 1 : row);
        y[f] = w[row * dim + d];
    }
}

__global__ __launch_bounds__(BLOCK) void narrow_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t outer,
                                                       int64_t dim, int64_t inner, int64_t start,
                                                       int64_t length) {
    FOR_EACH_ELEMENT(f, outer * length * inner) {
        const int64_t o = f / (length * inner), r = f % (length * inner);
        y[f] = x[o * dim * inner + start * inner + r];
    }
}

__global__ __launch_bounds__(BLOCK) void concat_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t outer,
                                                       int64_t d, int64_t inner, int64_t total,
                                                       int64_t at) {
    FOR_EACH_ELEMENT(f, outer * d * inner) {
        const int64_t o = f / (d * inner), r = f % (d * inner);
        y[o * total * inner + at * inner + r] = x[f];
    }
}

// OpKind::Rope (cpu_rope, cpu_kernels.rs:608-645): interleaved pairs of the
// first rotary_dim columns; the rest is copied.
__global__ __launch_bounds__(BLOCK) void rope_interleaved_kernel(const float* __restrict__ x,
                                                                 float* __restrict__ y,
                                                                 int64_t tokens, int64_t hd,
                                                                 int64_t rd, int64_t pos_offset,
                                                                 float theta, int64_t len) {
    FOR_EACH_ELEMENT(f, len) {
        const int64_t t = f / hd, c = f % hd;
        if (t >= tokens || c >= rd) {
            y[f] = x[f];
            continue;
        }
        const int64_t i = c / 2;
        const float inv_freq = powf(theta, -2.0f * (float)i / (float)rd);
        const float angle = (float)(pos_offset + t) * inv_freq;
        const float sn = sinf(angle), cs = cosf(angle);
        const int64_t base = t * hd + i * 2;
        const float x0 = x[base], x1 = x[base + 1];
        y[f] = (c % 2 == 0) ? x0 * cs - x1 * sn : x0 * sn + x1 * cs;
    }
}

// OpKind::RoPE (rope, cpu_kernels.rs:896-956).
__global__ __launch_bounds__(BLOCK) void rope_mlx_kernel(const float* __restrict__ x,
                                                         float* __restrict__ y, int64_t n_rows,
                                                         int64_t hd, int64_t offset, float base,
                                                         int traditional) {
    const int64_t half = hd / 2;
    FOR_EACH_ELEMENT(f, n_rows * half) {
        const int64_t i = f / half, d = f % half;
        const float pos = (float)(offset + i);
        const float th = pos * powf(base, -(2.0f * (float)d / (float)hd));
        const float ct = cosf(th), st = sinf(th);
        int64_t i0, i1;
        if (traditional) {
            i0 = i * hd + 2 * d;
            i1 = i0 + 1;
        } else {
            i0 = i * hd + d;
            i1 = i * hd + d + half;
        }
        const float x0 = x[i0], x1 = x[i1];
        y[i0] = x0 * ct - x1 * st;
        y[i1] = x0 * st + x1 * ct;
    }
}

__global__ __launch_bounds__(BLOCK) void fill_kernel(float* __restrict__ y, float v, int64_t n) {
    FOR_EACH_ELEMENT(i, n) y[i] = v;
}

inline unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>(ceil_div(n, BLOCK), MAX_GRID); }

}  // namespace

int ew_chain(const mlxhip_ew_instr_t* prog, int n_instr, const float* const* inputs, int n_inputs,
             float* out, int64_t numel, hipStream_t s) {
    return ew_chain_periodic(prog, n_instr, inputs, nullptr, n_inputs, out, numel, s);
}

int ew_chain_periodic(const mlxhip_ew_instr_t* prog, int n_instr, const float* const* inputs,
                      const int64_t* periods, int n_inputs, float* out, int64_t numel, hipStream_t s) {
    return ew_chain_planes(prog, n_instr, inputs, periods, n_inputs, out, numel, nullptr, nullptr, 0, nullptr, s);
}

int ew_chain_planes(const mlxhip_ew_instr_t* prog, int n_instr, const float* const* inputs, const int64_t* periods,
                    int n_inputs, float* out, int64_t numel, uint16_t* planes, uint32_t* flag, uint32_t gen,
                    bool* written, hipStream_t s) {
    if (written) *written = false;
    if (n_instr < 0 || n_instr > MLXHIP_EW_MAX_INSTR)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ew_chain: %d instructions (max %d)", n_instr,
                    MLXHIP_EW_MAX_INSTR);
    if (n_inputs < 1 || n_inputs > MLXHIP_EW_MAX_INPUTS)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ew_chain: %d inputs (1..%d)", n_inputs,
                    MLXHIP_EW_MAX_INPUTS);
    if (numel < 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ew_chain: negative size");
    EwProg p{};
    bool aligned = reinterpret_cast<uintptr_t>(out) % 16 == 0;
    bool periodic = false;
    for (int i = 0; i < n_inputs; ++i) {
        if (!inputs[i] && numel) return fail(MLXHIP_ERR_NULL_PTR, "ew_chain: input %d is null", i);
        p.in[i] = inputs[i];
        const int64_t per = periods ? periods[i] : 0;
        if (per < 0 || (per > 0 && numel % per))
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ew_chain: period %lld does not divide %lld", (long long)per,
                        (long long)numel);
        p.period[i] = per == numel ? 0 : per;
        if (p.period[i] > 0) {
            periodic = true;
            // Vector loads need whole float4 periods (or one value for all).
            aligned = aligned && (p.period[i] == 1 || p.period[i] % 4 == 0);
        }
        aligned = aligned && reinterpret_cast<uintptr_t>(inputs[i]) % 16 == 0;
    }
    // 32-bit modulo in the vector kernel.
    if (periodic && numel / 4 > (int64_t)UINT32_MAX) aligned = false;
    for (int k = 0; k < n_instr; ++k) {
        if (prog[k].op < 0 || prog[k].op >= MLXHIP_EW_COUNT_)
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ew_chain: bad op %d", prog[k].op);
        if (ew_binary(prog[k].op) && (prog[k].operand < 0 || prog[k].operand >= n_inputs))
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ew_chain: operand %d out of range",
                        prog[k].operand);
        p.op[k] = prog[k].op;
        p.operand[k] = ew_binary(prog[k].op) ? prog[k].operand : 0;
    }
    p.n_instr = n_instr;
    if (numel == 0) return MLXHIP_OK;
    // Planes only from the vector kernel covering every element.
    const bool with_planes = planes && flag && aligned && numel % 4 == 0 &&
                             reinterpret_cast<uintptr_t>(planes) % 16 == 0;
    if (with_planes) {
        p.planes = planes;
        p.plane = numel;
        p.flag = flag;
        p.gen = gen;
    }
    int64_t done = 0;
    if (aligned) {
        const int64_t n_vec = numel / 4;
        EwProg pv = p;  // periods in float4 units; one-value inputs splat
        for (int i = 0; i < n_inputs; ++i) {
            if (p.period[i] == 1) {
                pv.scalar_mask |= 1 << i;
                pv.period[i] = 0;
            } else {
                pv.period[i] = p.period[i] / 4;
            }
        }
        if (n_vec > 0) {
            switch (n_inputs) {
                case 1: MLXHIP_TRY(launch_chain_vec<1>(pv, out, n_vec, periodic, s)); break;
                case 2: MLXHIP_TRY(launch_chain_vec<2>(pv, out, n_vec, periodic, s)); break;
                case 3: MLXHIP_TRY(launch_chain_vec<3>(pv, out, n_vec, periodic, s)); break;
                case 4: MLXHIP_TRY(launch_chain_vec<4>(pv, out, n_vec, periodic, s)); break;
                case 5: MLXHIP_TRY(launch_chain_vec<5>(pv, out, n_vec, periodic, s)); break;
                case 6: MLXHIP_TRY(launch_chain_vec<6>(pv, out, n_vec, periodic, s)); break;
                case 7: MLXHIP_TRY(launch_chain_vec<7>(pv, out, n_vec, periodic, s)); break;
                default: MLXHIP_TRY(launch_chain_vec<8>(pv, out, n_vec, periodic, s)); break;
            }
        }
        done = n_vec * 4;
    }
    if (done < numel) {
        hipLaunchKernelGGL(ew_chain_scalar_kernel, dim3(grid_for(numel - done)), dim3(BLOCK), 0, s,
                           p, out, done, numel);
        MLXHIP_TRY(launch_check("ew_chain_scalar_kernel"));
    }
    if (written) *written = with_planes;
    return MLXHIP_OK;
}

int transpose2d(const float* x, float* y, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows == 0 || cols == 0) return MLXHIP_OK;
    if (ceil_div(rows, 64) > 65535) {
        const int64_t shape[2] = {rows, cols}, perm[2] = {1, 0};
        return permute(x, y, shape, perm, 2, s);
    }
    dim3 grid((unsigned)ceil_div(cols, 64), (unsigned)ceil_div(rows, 64));
    hipLaunchKernelGGL(transpose2d_kernel, grid, dim3(BLOCK), 0, s, x, y, rows, cols);
    return launch_check("transpose2d_kernel");
}

// Host side of gather32_kernel: `dims` the output shape, `stride` each output
// axis's input stride (elements). Returns false (nothing launched) when the
// 32-bit form does not apply.
bool gather32(const float* x, float* y, const int64_t* dims, const int64_t* stride, int ndim, int64_t total,
              hipStream_t s, int* rc) {
    // float4 units when the innermost output axis is contiguous in the input
    // and holds a multiple of 4 elements, and both pointers are 16-byte aligned.
    const bool vec = ndim > 0 && stride[ndim - 1] == 1 && dims[ndim - 1] % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16 == 0;
    const int64_t unit = vec ? 4 : 1;
    const int64_t units = total / unit;
    if (units >= (int64_t(1) << 31)) return false;
    Gather32 g{};
    g.ndim = ndim;
    int64_t max_src = 0;
    for (int d = 0; d < ndim; ++d) {
        const int64_t n = d == ndim - 1 ? dims[d] / unit : dims[d];
        const int64_t st = d == ndim - 1 ? stride[d] : stride[d] / unit;
        if (d < ndim - 1 && stride[d] % unit) return false;
        max_src += (n - 1) * st;
        g.dim[d] = (uint32_t)n;
        g.stride[d] = (uint32_t)st;
        if (n >= 2) {
            int l = 0;
            while ((int64_t(1) << l) < n) ++l;
            const int p = 31 + l;
            g.mul[d] = (uint32_t)(((uint64_t(1) << p) + (uint64_t)n - 1) / (uint64_t)n);
            g.shr[d] = (uint32_t)(p - 32);
        }
    }
    if (max_src >= (int64_t(1) << 31)) return false;
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(units, BLOCK), MAX_GRID);
    if (vec) hipLaunchKernelGGL(gather32_kernel<4>, dim3(grid), dim3(BLOCK), 0, s, x, y, g, (uint32_t)units);
    else hipLaunchKernelGGL(gather32_kernel<1>, dim3(grid), dim3(BLOCK), 0, s, x, y, g, (uint32_t)units);
    *rc = launch_check("gather32_kernel");
    return true;
}

int permute(const float* x, float* y, const int64_t* shape, const int64_t* perm, int ndim,
            hipStream_t s) {
    if (ndim > MAXD) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "permute: rank %d > %d", ndim, MAXD);
    int64_t total = 1;
    for (int i = 0; i < ndim; ++i) total *= shape[i];
    if (total == 0) return MLXHIP_OK;
    if (ndim == 2 && perm[0] == 1 && perm[1] == 0 && ceil_div(shape[0], 64) <= 65535)
        return transpose2d(x, y, shape[0], shape[1], s);
    int64_t old_stride[MAXD];
    old_stride[ndim - 1] = 1;
    for (int i = ndim - 2; i >= 0; --i) old_stride[i] = old_stride[i + 1] * shape[i + 1];
    Dims ns{}, st{};
    bool seen[MAXD] = {};
    for (int i = 0; i < ndim; ++i) {
        // A repeated axis would index past the input: only true permutations run.
        if (perm[i] < 0 || perm[i] >= ndim || seen[perm[i]])
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose: axes must be a permutation of 0..%d", ndim - 1);
        seen[perm[i]] = true;
        ns.v[i] = shape[perm[i]];
        st.v[i] = old_stride[perm[i]];
    }
    int rc = MLXHIP_OK;
    if (gather32(x, y, ns.v, st.v, ndim, total, s, &rc)) return rc;
    hipLaunchKernelGGL(permute_kernel, dim3(grid_for(total)), dim3(BLOCK), 0, s, x, y, ns, st, ndim,
                       total);
    return launch_check("permute_kernel");
}

int broadcast(const float* x, float* y, const int64_t* in_shape, int in_ndim,
              const int64_t* out_shape, int out_ndim, hipStream_t s) {
    if (out_ndim > MAXD || in_ndim > out_ndim)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "broadcast: ranks %d -> %d", in_ndim, out_ndim);
    int64_t total = 1;
    for (int i = 0; i < out_ndim; ++i) total *= out_shape[i];
    if (total == 0) return MLXHIP_OK;
    Dims os{}, st{};
    const int pad = out_ndim - in_ndim;
    int64_t stride = 1;
    for (int d = out_ndim - 1; d >= 0; --d) {
        os.v[d] = out_shape[d];
        if (d >= pad) {
            const int64_t idim = in_shape[d - pad];
            if (idim != 1 && idim != out_shape[d])
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "broadcast: dim %lld vs %lld",
                            (long long)idim, (long long)out_shape[d]);
            st.v[d] = idim == 1 ? 0 : stride;
            stride *= idim;
        } else {
            st.v[d] = 0;
        }
    }
    int rc = MLXHIP_OK;
    if (gather32(x, y, os.v, st.v, out_ndim, total, s, &rc)) return rc;
    hipLaunchKernelGGL(broadcast_kernel, dim3(grid_for(total)), dim3(BLOCK), 0, s, x, y, os, st,
                       out_ndim, total);
    return launch_check("broadcast_kernel");
}

int reduce_axis(int kind, const float* x, float* y, int64_t outer, int64_t dim, int64_t inner,
                hipStream_t s) {
    const int64_t n = outer * inner;
    if (n == 0) return MLXHIP_OK;
    // Long axes over float4-aligned rows: the chunked LDS fold (same order).
    // Chunks of 256 rows, 4 in flight, folded from 32-row register batches:
    // the fastest of the chunk / prefetch / batch sizes measured on Sum over
    // 2048 rows of 1024 and 4096 columns (11.1 and 16.4 us, against 25.8 and
    // 26.3 us for one thread per output). Offsets up to P + 1 chunks past
    // the last row stay below 2^32.
    constexpr int CH = 256, PF = 4, FB = 32, COLS = 16;
    if (dim >= 2 * CH && inner % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        (dim + (PF + 1) * CH) * inner * 4 < (int64_t(1) << 32) && outer * ceil_div(inner, COLS) < (int64_t(1) << 31)) {
        const int64_t cb = ceil_div(inner, COLS);
        const dim3 g((unsigned)(outer * cb));
        if (kind == 0)
            hipLaunchKernelGGL((reduce_cols_kernel<0, COLS, CH, PF, FB>), g, dim3(RC_BLOCK), 0, s, x, y, dim, inner, cb);
        else if (kind == 1)
            hipLaunchKernelGGL((reduce_cols_kernel<1, COLS, CH, PF, FB>), g, dim3(RC_BLOCK), 0, s, x, y, dim, inner, cb);
        else
            hipLaunchKernelGGL((reduce_cols_kernel<2, COLS, CH, PF, FB>), g, dim3(RC_BLOCK), 0, s, x, y, dim, inner, cb);
        return launch_check("reduce_cols_kernel");
    }
    const dim3 grid((unsigned)std::min<int64_t>(ceil_div(n, RED_BLOCK), MAX_GRID));
    if (kind == 0) hipLaunchKernelGGL(reduce_axis_kernel<0>, grid, dim3(RED_BLOCK), 0, s, x, y, outer, dim, inner);
    else if (kind == 1) hipLaunchKernelGGL(reduce_axis_kernel<1>, grid, dim3(RED_BLOCK), 0, s, x, y, outer, dim, inner);
    else hipLaunchKernelGGL(reduce_axis_kernel<2>, grid, dim3(RED_BLOCK), 0, s, x, y, outer, dim, inner);
    return launch_check("reduce_axis_kernel");
}

int reduce_all(int kind, const float* x, float* y, int64_t n, hipStream_t s) {
    if (n <= 65536) {
        hipLaunchKernelGGL(reduce_all_seq_kernel, dim3(1), dim3(64), 0, s, kind, x, y, n);
        return launch_check("reduce_all_seq_kernel");
    }
    // Partials of the tree reduction: the stream's cached workspace, so calls
    // on different streams never share it and no call allocates.
    const int np = 1024;
    void* pb = nullptr;
    MLXHIP_TRY(stream_workspace(s, WS_REDUCE, sizeof(float) * np, &pb));
    float* part = static_cast<float*>(pb);
    hipLaunchKernelGGL(reduce_partial_kernel, dim3(np), dim3(BLOCK), 0, s, kind, x, part, n);
    MLXHIP_TRY(launch_check("reduce_partial_kernel"));
    hipLaunchKernelGGL(reduce_final_kernel, dim3(1), dim3(BLOCK), 0, s, kind, part, y, np, n);
    return launch_check("reduce_final_kernel");
}

int cast(const void* x, int src, void* y, int dst, int64_t n, hipStream_t s) {
    auto ok = [](int t) { return t == MLXHIP_DTYPE_F32 || t == MLXHIP_DTYPE_BF16 || t == MLXHIP_DTYPE_F16; };
    if (!ok(src) || !ok(dst)) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "cast: unsupported dtype");
    if (n == 0) return MLXHIP_OK;
    hipLaunchKernelGGL(cast_kernel, dim3(grid_for(n)), dim3(BLOCK), 0, s, x, src, y, dst, n);
    return launch_check("cast_kernel");
}

int embedding(const float* w, const float* idx, float* y, int64_t n_idx, int64_t num_emb,
              int64_t dim, hipStream_t s) {
    if (n_idx * dim == 0) return MLXHIP_OK;
    if (num_emb <= 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "embedding: empty table");
    hipLaunchKernelGGL(embedding_kernel, dim3(grid_for(n_idx * dim)), dim3(BLOCK), 0, s, w, idx, y,
                       n_idx, num_emb, dim);
    return launch_check("embedding_kernel");
}

int narrow(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, int64_t start,
           int64_t length, hipStream_t s) {
    const int64_t n = outer * length * inner;
    if (n == 0) return MLXHIP_OK;
    hipLaunchKernelGGL(narrow_kernel, dim3(grid_for(n)), dim3(BLOCK), 0, s, x, y, outer, dim, inner,
                       start, length);
    return launch_check("narrow_kernel");
}

int concat_part(const float* x, float* y, int64_t outer, int64_t d, int64_t inner, int64_t total,
                int64_t at, hipStream_t s) {
    const int64_t n = outer * d * inner;
    if (n == 0) return MLXHIP_OK;
    hipLaunchKernelGGL(concat_kernel, dim3(grid_for(n)), dim3(BLOCK), 0, s, x, y, outer, d, inner,
                       total, at);
    return launch_check("concat_kernel");
}

int rope_interleaved(const float* x, float* y, int64_t tokens, int64_t head_dim,
                     int64_t rotary_dim, int64_t pos_offset, float theta, int64_t len,
                     hipStream_t s) {
    if (len == 0) return MLXHIP_OK;
    hipLaunchKernelGGL(rope_interleaved_kernel, dim3(grid_for(len)), dim3(BLOCK), 0, s, x, y,
                       tokens, head_dim, rotary_dim, pos_offset, theta, len);
    return launch_check("rope_interleaved_kernel");
}

int rope_mlx(const float* x, float* y, int64_t n_rows, int64_t head_dim, int64_t offset, float base,
             int traditional, hipStream_t s) {
    const int64_t n = n_rows * (head_dim / 2);
    if (n == 0) return MLXHIP_OK;
    hipLaunchKernelGGL(rope_mlx_kernel, dim3(grid_for(n)), dim3(BLOCK), 0, s, x, y, n_rows, head_dim,
                       offset, base, traditional);
    return launch_check("rope_mlx_kernel");
}

int fill(float* y, float v, int64_t n, hipStream_t s) {
    if (n == 0) return MLXHIP_OK;
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(BLOCK), 0, s, y, v, n);
    return launch_check("fill_kernel");
}

}  // namespace mlxhip
