// gemm_small.hip — f32 GEMM for products too small to occupy the chip with
// 64 x 64 tiles (config 1: 512^3), in one launch with no workspace.
//
// C_b[M,N] = op(A_b) * op(B_b), f32 operands and output; replaces matmul
// (crates/mlx-core/src/cpu_kernels.rs:197-230) at these sizes.
//
// One workgroup per 32 x 32 tile of C. Its waves (4, or 8 when K > 256)
// split K into contiguous parts; each wave accumulates its quarter with
// v_mfma_f32_32x32x2_f32, where the two half-waves supply different k of
// each MFMA step: lane l (row / column r = l % 32, half h = l / 32) feeds k
// = base_w + h * KH + i at step i, so each lane's A values (and B values)
// are KH consecutive k. A K-contiguous operand is therefore read with
// 16-byte loads along K; an MN-contiguous one with 4-byte loads that are
// coalesced across the 32 lanes of a half-wave. Every load of a wave is
// issued before its first MFMA. The four partial tiles meet in LDS and are
// summed in wave order (deterministic), then stored. Each wave keeps four
// independent accumulator chains (summed in chain order at the end), so the
// matrix pipe is not held up by the latency of one chain of dependent MFMAs.
#include "../common.hpp"
#include "../kernels.hpp"

namespace mlxhip {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int K_MAX = 512;  // 8 waves x 2 half-waves x 32 k

// One half-wave's KH operand values of row / column r (k = kb .. kb+KH-1),
// zero outside the matrix (R >= 1, K >= 1). KC: the operand is stored
// [rows][K] (pitch ld); else [K][rows]. Branch-free: every address is
// clamped into the matrix and out-of-range values are zeroed by selects
// after the loads, so all loads are issued back to back (a guarded load per
// element compiles to masked branches that wait for each load in turn).
template <bool KC, int KH>
__device__ inline void load_run(const float* __restrict__ base, int64_t ld, int64_t r, int64_t R, int64_t kb,
                                int64_t K, bool vec, float* v) {
    const bool rok = r < R;
    const int64_t rr = rok ? r : R - 1;
    if constexpr (KC) {
        const float* p = base + rr * ld;
        if (vec && kb + KH <= K) {
#pragma unroll
            for (int i = 0; i < KH; i += 4) {
                const float4 t = *reinterpret_cast<const float4*>(p + kb + i);
                v[i] = t.x, v[i + 1] = t.y, v[i + 2] = t.z, v[i + 3] = t.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < KH; ++i) {
                const int64_t kk = kb + i < K ? kb + i : K - 1;
                const float t = p[kk];
                v[i] = kb + i < K ? t : 0.0f;
            }
        }
    } else {
        const float* p = base + rr;
#pragma unroll
        for (int i = 0; i < KH; ++i) {
            const int64_t kk = kb + i < K ? kb + i : K - 1;
            const float t = p[kk * ld];
            v[i] = kb + i < K ? t : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < KH; ++i) v[i] = rok ? v[i] : 0.0f;
}

template <int TA, int TB, int KH, int WAVES>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WAVES, 64 * WAVES), amdgpu_waves_per_eu(1, 2))) void gemm_small_kernel(const float* __restrict__ a, int64_t lda, int64_t sa,
                                                          const float* __restrict__ b, int64_t ldb, int64_t sb,
                                                          float* __restrict__ c, int64_t ldc, int64_t sc,
                                                          int64_t m, int64_t n, int64_t k, int vec_a, int vec_b) {
    __shared__ float part[WAVES][32][33];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Tile order: consecutive workgroup ids go to the 8 XCDs round-robin;
    // give each XCD a contiguous range of ids, and order ids in groups of 4
    // tile rows, so an XCD reads few A row panels and B column panels into
    // its own L2 (every launch starts with cold L2s).
    const int tiles_n = (int)((n + 31) / 32), tiles_m = (int)((m + 31) / 32);
    const int per_batch = tiles_m * tiles_n;
    const int total = per_batch * (int)gridDim.y;
    int lin = (int)blockIdx.x + (int)blockIdx.y * (int)gridDim.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int64_t bt = lin / per_batch;
    const int id = lin - (int)bt * per_batch;
    constexpr int GROUP_M = 4;
    const int in_group = GROUP_M * tiles_n;
    const int first_m = (id / in_group) * GROUP_M;
    const int gsz = min(tiles_m - first_m, GROUP_M);
    const int64_t m0 = (int64_t)(first_m + (id % in_group) % gsz) * 32;
    const int64_t n0 = (int64_t)((id % in_group) / gsz) * 32;
    const int r = lane & 31, h = lane >> 5;
    const int64_t kb = (int64_t)(2 * wave + h) * KH;  // this half-wave's first k
    float av[KH], bv[KH];
    load_run<TA == 0, KH>(a + bt * sa, lda, m0 + r, m, kb, k, vec_a, av);
    load_run<TB == 1, KH>(b + bt * sb, ldb, n0 + r, n, kb, k, vec_b, bv);
    // Keep every load ahead of the MFMAs (one memory latency per wave);
    // left alone, the scheduler moves each load next to its MFMA to save
    // registers and the wave waits once per step.
    __builtin_amdgcn_sched_barrier(0);
    // Four independent accumulator chains (step i feeds chain i % 4): one
    // chain of dependent MFMAs waits for each result before the next step.
    constexpr int CHAINS = KH >= 16 ? 4 : 1;
    f32x16 acc[CHAINS];
#pragma unroll
    for (int q = 0; q < CHAINS; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.0f;
#pragma unroll
    for (int i = 0; i < KH; ++i)
        acc[i % CHAINS] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc[i % CHAINS], 0, 0, 0);
#pragma unroll
    for (int q = 1; q < CHAINS; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[0][v] += acc[q][v];
    // Accumulator element v of lane l is C[8*(v/4) + 4*(l/32) + v%4][l%32].
#pragma unroll
    for (int v = 0; v < 16; ++v) part[wave][8 * (v >> 2) + 4 * h + (v & 3)][r] = acc[0][v];
    __syncthreads();
#pragma unroll
    for (int e = tid; e < 32 * 32; e += 64 * WAVES) {
        const int i = e >> 5, j = e & 31;
        float s = part[0][i][j];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) s += part[w][i][j];
        const int64_t row = m0 + i, col = n0 + j;
        if (row < m && col < n) c[bt * sc + row * ldc + col] = s;
    }
}

template <int TA, int TB>
int launch_small(const float* a, int64_t lda, int64_t sa, const float* b, int64_t ldb, int64_t sb, float* c,
                 int64_t ldc, int64_t sc, int64_t m, int64_t n, int64_t k, int64_t batch, hipStream_t s) {
    const dim3 grid((unsigned)(ceil_div(n, 32) * ceil_div(m, 32)), (unsigned)batch);
    const int va = TA == 0 && lda % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 && (batch == 1 || sa % 4 == 0);
    const int vb = TB == 1 && ldb % 4 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 && (batch == 1 || sb % 4 == 0);
    // k per half-wave (a multiple of 4 so 16-byte runs stay aligned): four
    // waves up to K = 256, eight beyond, so no lane holds more than 32 k of
    // each operand (a run of 64 scalar loads plus the 16-byte ones would pass
    // the 63 loads a wave can have in flight and wait in the middle).
#define MLXHIP_SMALL(KHV, W)                                                                                  \
    hipLaunchKernelGGL((gemm_small_kernel<TA, TB, KHV, W>), grid, dim3(64 * W), 0, s, a, lda, sa, b, ldb, sb, c, \
                       ldc, sc, m, n, k, va, vb)
    if (k <= 64) MLXHIP_SMALL(8, 4);
    else if (k <= 128) MLXHIP_SMALL(16, 4);
    else if (k <= 256) MLXHIP_SMALL(32, 4);
    else MLXHIP_SMALL(32, 8);
#undef MLXHIP_SMALL
    return launch_check("gemm_small_kernel");
}

}  // namespace

bool gemm_small_f32_fits(int64_t m, int64_t n, int64_t k, int64_t batch) {
    // At most two rounds of 32 x 32 tiles on 256 CUs: beyond that the 64 x 64
    // and larger tiles of the general kernel reuse operands better.
    return k >= 1 && k <= K_MAX && ceil_div(m, 32) * ceil_div(n, 32) * batch <= 512 && batch <= 65535 &&
           ceil_div(m, 32) <= 65535;
}

int gemm_small_f32(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const float* a, int64_t lda,
                   int64_t sa, const float* b, int64_t ldb, int64_t sb, float* c, int64_t ldc, int64_t sc,
                   hipStream_t s) {
    if (!ta && !tb) return launch_small<0, 0>(a, lda, sa, b, ldb, sb, c, ldc, sc, m, n, k, batch, s);
    if (!ta && tb) return launch_small<0, 1>(a, lda, sa, b, ldb, sb, c, ldc, sc, m, n, k, batch, s);
    if (ta && !tb) return launch_small<1, 0>(a, lda, sa, b, ldb, sb, c, ldc, sc, m, n, k, batch, s);
    return launch_small<1, 1>(a, lda, sa, b, ldb, sb, c, ldc, sc, m, n, k, batch, s);
}

}  // namespace mlxhip
