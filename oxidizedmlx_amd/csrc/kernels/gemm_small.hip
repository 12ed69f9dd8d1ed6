// gemm_small.hip — f32 GEMM for products too small to occupy the chip with
// 64 x 64 tiles (config 1: 512^3), in one launch with no workspace.
//
// C_b[M,N] = op(A_b) * op(B_b), f32 operands and output; replaces matmul
// (crates/mlx-core/src/cpu_kernels.rs:197-230) at these sizes.
//
// One workgroup of 4 waves (one per SIMD) per 32 x 32 tile of C. The K axis
// is cut into 8 contiguous runs of KH (KH = 8, 16, 32 or 64, the smallest
// with 8 * KH >= K), one per half-wave: wave w's half h takes k = (2w + h) *
// KH + i at MFMA step i of v_mfma_f32_32x32x2_f32, whose two half-waves
// supply the two k of each step. Each lane thus holds KH consecutive k of
// its row of A and of its column of B: a K-contiguous operand is read with
// 16-byte loads along K, an MN-contiguous one with 4-byte loads that are
// coalesced across the 32 lanes of a half-wave. Loads are buffer loads with
// 32-bit offsets from each operand slice's base (no 64-bit address
// arithmetic per load), issued A then B four k at a time so the first
// MFMAs start while later loads are in flight; every load of a wave is
// issued before its first MFMA. Elements outside the matrix are read
// through an offset past the descriptor's range, which returns zeros. The
// four waves' partial tiles meet in LDS and are summed in wave order
// (deterministic), then stored. Each wave keeps four independent
// accumulator chains (summed in chain order at the end), so the matrix pipe
// is not held up by the latency of one chain of dependent MFMAs.
//
// Whole-tile products (M, N multiples of 32, K = 8 * KH, every operand run
// 16-byte aligned) run an 8-wave kernel instead (gemm_small_staged_kernel)
// that brings MN-contiguous operands in through LDS with 16-byte loads.
// Measured on MI355X for 512^3 (NN): the 4-wave kernel without range
// selects took 6.0 us per launch back to back on warm operands (2.5 us of it
// the cost of launching an empty grid of the same shape) and 7.10-7.45 us on
// eight operand sets in rotation; the staged kernel takes 6.46-6.61 us on
// the rotating sets.
#include "../common.hpp"
#include "../kernels.hpp"

namespace mlxhip {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int K_MAX = 512;                   // 8 half-waves x 64 k
constexpr uint32_t OOB_OFF = 0xFFFFFF00u;    // beyond every descriptor range (slices are < 2 GiB)
constexpr int BUF_FLAGS = 0x00020000;        // gfx9 buffer descriptor word 3 (32-bit data format)
constexpr int64_t SLICE_MAX_BYTES = int64_t(1) << 31;

struct SmallArgs {
    const float* a;
    const float* b;
    float* c;
    int64_t sa, sb, sc, ldc;
    int64_t m, n, k;
    uint32_t lda4, ldb4;     // leading dimensions in bytes
    uint32_t nrec_a, nrec_b; // descriptor ranges: one operand slice's bytes
    int tiles_n, tiles_m;
};

// Byte offset of the lane's first element (k = kb) and the byte step per
// unit of k, for a K-contiguous operand (element (row, k) at row * ld + k)
// or an MN-contiguous one (element (k, row) at k * ld + row).
template <bool KC>
__device__ inline uint32_t first_offset(int64_t row, int64_t kb, uint32_t ld4) {
    if constexpr (KC) return (uint32_t)row * ld4 + (uint32_t)kb * 4u;
    else return (uint32_t)kb * ld4 + (uint32_t)row * 4u;
}

// Four operand values, k = kb + i .. kb + i + 3, of the lane's row (or
// column). EVEN: every element is inside the matrix and a K-contiguous run
// is 16-byte aligned (one 16-byte load); otherwise one 4-byte load per
// element, through an out-of-range offset (zeros) when the element is
// outside the matrix.
template <bool KC, bool EVEN>
__device__ inline void load4(__amdgpu_buffer_rsrc_t rs, uint32_t off0, uint32_t ld4, int i, bool row_ok, int64_t kb,
                             int64_t K, float* v) {
    if constexpr (KC && EVEN) {
        const f32x4v t = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(rs, off0 + 4u * i, 0, 0));
        v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t step = KC ? 4u * (uint32_t)(i + j) : (uint32_t)(i + j) * ld4;
            uint32_t off = off0 + step;
            if constexpr (!EVEN) off = row_ok && kb + i + j < K ? off : OOB_OFF;
            v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
        }
    }
}

template <int TA, int TB, int KH>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256))) void gemm_small_kernel(SmallArgs g) {
    __shared__ float part[4][32][33];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Tile order: consecutive workgroup ids go to the 8 XCDs round-robin;
    // give each XCD a contiguous range of ids, and order ids in groups of 4
    // tile rows, so an XCD reads few A row panels and B column panels into
    // its own L2 (every launch starts with cold L2s).
    const int per_batch = g.tiles_m * g.tiles_n;
    const int total = per_batch * (int)gridDim.y;
    int lin = (int)blockIdx.x + (int)blockIdx.y * (int)gridDim.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int bt = lin / per_batch;
    const int id = lin - bt * per_batch;
    constexpr int GROUP_M = 4;
    const int in_group = GROUP_M * g.tiles_n;
    const int first_m = (id / in_group) * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int64_t m0 = (int64_t)(first_m + (id % in_group) % gsz) * 32;
    const int64_t n0 = (int64_t)((id % in_group) / gsz) * 32;
    const int r = lane & 31, h = lane >> 5;
    const int64_t kb = (int64_t)(2 * wave + h) * KH;  // this half-wave's first k

    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.a + bt * g.sa), (short)0, (int)g.nrec_a, BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.b + bt * g.sb), (short)0, (int)g.nrec_b, BUF_FLAGS);
    const bool a_ok = m0 + r < g.m, b_ok = n0 + r < g.n;
    // Rows past the matrix edge take row 0's offsets (their loads are
    // redirected out of range), so no offset is computed from them.
    const uint32_t oa = first_offset<TA == 0>(a_ok ? m0 + r : 0, kb < g.k ? kb : 0, g.lda4);
    const uint32_t ob = first_offset<TB == 1>(b_ok ? n0 + r : 0, kb < g.k ? kb : 0, g.ldb4);
    float av[KH], bv[KH];
#pragma unroll
    for (int i = 0; i < KH; i += 4) {
        load4<TA == 0, false>(ra, oa, g.lda4, i, a_ok, kb, g.k, av + i);
        load4<TB == 1, false>(rb, ob, g.ldb4, i, b_ok, kb, g.k, bv + i);
    }
    // Keep every load ahead of the MFMAs (one memory latency per wave);
    // left alone, the scheduler moves each load next to its MFMA to save
    // registers and the wave waits once per step.
    __builtin_amdgcn_sched_barrier(0);
    // Four independent accumulator chains (step i feeds chain i % 4).
    f32x16 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.0f;
#pragma unroll
    for (int i = 0; i < KH; ++i)
        acc[i % 4] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc[i % 4], 0, 0, 0);
#pragma unroll
    for (int q = 1; q < 4; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[0][v] += acc[q][v];
    // Accumulator element v of lane l is C[8*(v/4) + 4*(l/32) + v%4][l%32].
#pragma unroll
    for (int v = 0; v < 16; ++v) part[wave][8 * (v >> 2) + 4 * h + (v & 3)][r] = acc[0][v];
    __syncthreads();
    float* cb = g.c + bt * g.sc;
#pragma unroll
    for (int e = tid; e < 32 * 32; e += 256) {
        const int i = e >> 5, j = e & 31;
        const float s = ((part[0][i][j] + part[1][i][j]) + part[2][i][j]) + part[3][i][j];
        const int64_t row = m0 + i, col = n0 + j;
        if (row < g.m && col < g.n) cb[row * g.ldc + col] = s;
    }
}

// Whole-tile products (EVEN), 8 waves: K is cut into 16 runs of KH (one per
// half-wave, KH = 4 .. 32), and an MN-contiguous operand (A stored [K][M],
// B stored [K][N]) is staged through LDS: its 32-wide panel over all of K
// comes in with 16-byte loads along M / N (8 per k row) instead of one 4-byte
// load per lane and k, and each lane then reads its own row's or column's KH
// values from LDS. A K-contiguous operand is read straight into registers
// with 16-byte loads along K, as in the kernel above. The eight waves'
// partial tiles are summed in wave order through LDS (reusing the staging
// area). 512^3 NN on MI355X, HIP events, eight operand sets in rotation:
// 6.46-6.61 us per launch against 7.10-7.45 us for the 4-wave kernel.
template <int TA, int TB, int KH>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512))) void gemm_small_staged_kernel(SmallArgs g) {
    constexpr int W = 8, NT = 64 * W, K = 2 * W * KH;
    constexpr bool SA = TA == 1, SB = TB == 0;  // operands staged through LDS
    constexpr int PITCH = 33;                   // floats per staged k row (32 + 1)
    constexpr int A_OFF = 0, B_OFF = SA ? K * PITCH : 0;
    constexpr int STAGE = (SA ? K * PITCH : 0) + (SB ? K * PITCH : 0);
    constexpr int PART = W * 32 * 33;
    __shared__ __attribute__((aligned(16))) float lds[STAGE > PART ? STAGE : PART];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Tile order as in gemm_small_kernel.
    const int per_batch = g.tiles_m * g.tiles_n;
    const int total = per_batch * (int)gridDim.y;
    int lin = (int)blockIdx.x + (int)blockIdx.y * (int)gridDim.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int bt = lin / per_batch;
    const int id = lin - bt * per_batch;
    constexpr int GROUP_M = 4;
    const int in_group = GROUP_M * g.tiles_n;
    const int first_m = (id / in_group) * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int64_t m0 = (int64_t)(first_m + (id % in_group) % gsz) * 32;
    const int64_t n0 = (int64_t)((id % in_group) / gsz) * 32;
    const int r = lane & 31, h = lane >> 5;
    const int kb = (2 * wave + h) * KH;  // this half-wave's first k

    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.a + bt * g.sa), (short)0, (int)g.nrec_a, BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.b + bt * g.sb), (short)0, (int)g.nrec_b, BUF_FLAGS);
    // Staged panels: thread t loads 16-byte chunk t % 8 of k rows t / 8 + 64 j.
    constexpr int PJ = K * 8 / NT;
    const int prow = tid / 8, pq = tid % 8;
    f32x4v pa[SA ? PJ : 1], pb[SB ? PJ : 1];
    if constexpr (SA) {
#pragma unroll
        for (int j = 0; j < PJ; ++j)
            pa[j] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                   ra, (uint32_t)(prow + (NT / 8) * j) * g.lda4 + (uint32_t)(m0 + 4 * pq) * 4u, 0, 0));
    }
    if constexpr (SB) {
#pragma unroll
        for (int j = 0; j < PJ; ++j)
            pb[j] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rb, (uint32_t)(prow + (NT / 8) * j) * g.ldb4 + (uint32_t)(n0 + 4 * pq) * 4u, 0, 0));
    }
    // K-contiguous operands: the lane's KH values straight into registers.
    float av[KH], bv[KH];
    if constexpr (!SA) {
        const uint32_t oa = first_offset<true>(m0 + r, kb, g.lda4);
#pragma unroll
        for (int i = 0; i < KH; i += 4) load4<true, true>(ra, oa, g.lda4, i, true, kb, g.k, av + i);
    }
    if constexpr (!SB) {
        const uint32_t ob = first_offset<true>(n0 + r, kb, g.ldb4);
#pragma unroll
        for (int i = 0; i < KH; i += 4) load4<true, true>(rb, ob, g.ldb4, i, true, kb, g.k, bv + i);
    }
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
        float* ra_row = lds + A_OFF + (prow + (NT / 8) * j) * PITCH + 4 * pq;
        float* rb_row = lds + B_OFF + (prow + (NT / 8) * j) * PITCH + 4 * pq;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (SA) ra_row[e] = pa[j][e];
            if constexpr (SB) rb_row[e] = pb[j][e];
        }
    }
    __syncthreads();
    if constexpr (SA) {
#pragma unroll
        for (int i = 0; i < KH; ++i) av[i] = lds[A_OFF + (kb + i) * PITCH + r];
    }
    if constexpr (SB) {
#pragma unroll
        for (int i = 0; i < KH; ++i) bv[i] = lds[B_OFF + (kb + i) * PITCH + r];
    }
    f32x16 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.0f;
#pragma unroll
    for (int i = 0; i < KH; ++i)
        acc[i % 4] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc[i % 4], 0, 0, 0);
#pragma unroll
    for (int q = 1; q < 4; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[0][v] += acc[q][v];
    __syncthreads();  // every wave is done with the staged panels
    float* part = lds;  // [W][32][33]
#pragma unroll
    for (int v = 0; v < 16; ++v) part[(wave * 32 + 8 * (v >> 2) + 4 * h + (v & 3)) * 33 + r] = acc[0][v];
    __syncthreads();
    float* cb = g.c + bt * g.sc;
    for (int e = tid; e < 32 * 32; e += NT) {
        const int i = e >> 5, j = e & 31;
        float s = part[i * 33 + j];
#pragma unroll
        for (int w = 1; w < W; ++w) s += part[(w * 32 + i) * 33 + j];
        cb[(m0 + i) * g.ldc + n0 + j] = s;
    }
}

// Bytes of one operand slice: `rows` runs of `cols` elements, `ld` apart.
int64_t slice_bytes(int64_t rows, int64_t cols, int64_t ld) { return ((rows - 1) * ld + cols) * 4; }

template <int TA, int TB, int KH>
int launch_kh(const SmallArgs& g, bool even, int64_t batch, hipStream_t s) {
    const dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)batch);
    if (even) hipLaunchKernelGGL((gemm_small_staged_kernel<TA, TB, KH / 2>), grid, dim3(512), 0, s, g);
    else hipLaunchKernelGGL((gemm_small_kernel<TA, TB, KH>), grid, dim3(256), 0, s, g);
    return launch_check("gemm_small_kernel");
}

template <int TA, int TB>
int launch_small(SmallArgs& g, const float* a, int64_t lda, int64_t sa, const float* b, int64_t ldb, int64_t sb,
                 int64_t batch, hipStream_t s) {
    const int64_t m = g.m, n = g.n, k = g.k;
    // k per half-wave: the smallest of 8, 16, 32, 64 covering K in 8 runs.
    const int kh = k <= 64 ? 8 : k <= 128 ? 16 : k <= 256 ? 32 : 64;
    // 16-byte loads need every K-contiguous run 16-byte aligned.
    auto kc_aligned = [&](const float* p, int64_t ld, int64_t st) {
        return reinterpret_cast<uintptr_t>(p) % 16 == 0 && ld % 4 == 0 && (batch == 1 || st % 4 == 0);
    };
    // Whole tiles: 16-byte loads along K (K-contiguous operands) or along
    // M / N (the staged, MN-contiguous ones) need every run 16-byte aligned.
    const bool even = m % 32 == 0 && n % 32 == 0 && k == 8 * kh && kc_aligned(a, lda, sa) && kc_aligned(b, ldb, sb);
    switch (kh) {
        case 8: return launch_kh<TA, TB, 8>(g, even, batch, s);
        case 16: return launch_kh<TA, TB, 16>(g, even, batch, s);
        case 32: return launch_kh<TA, TB, 32>(g, even, batch, s);
        default: return launch_kh<TA, TB, 64>(g, even, batch, s);
    }
}

}  // namespace

bool gemm_small_f32_fits(int64_t m, int64_t n, int64_t k, int64_t batch, int64_t lda, int64_t ldb, int ta, int tb) {
    // At most two rounds of 32 x 32 tiles on 256 CUs: beyond that the 64 x 64
    // and larger tiles of the general kernel reuse operands better. Every
    // operand slice must be addressable with 32-bit offsets.
    if (!(m >= 1 && n >= 1 && k >= 1 && k <= K_MAX && ceil_div(m, 32) * ceil_div(n, 32) * batch <= 512 &&
          batch <= 65535))
        return false;
    const int64_t a_bytes = ta ? slice_bytes(k, m, lda) : slice_bytes(m, k, lda);
    const int64_t b_bytes = tb ? slice_bytes(n, k, ldb) : slice_bytes(k, n, ldb);
    return a_bytes < SLICE_MAX_BYTES && b_bytes < SLICE_MAX_BYTES && lda < SLICE_MAX_BYTES / 4 &&
           ldb < SLICE_MAX_BYTES / 4;
}

int gemm_small_f32(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const float* a, int64_t lda,
                   int64_t sa, const float* b, int64_t ldb, int64_t sb, float* c, int64_t ldc, int64_t sc,
                   hipStream_t s) {
    if (!gemm_small_f32_fits(m, n, k, batch, lda, ldb, ta, tb))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm_small_f32: shape outside the small kernel's range");
    SmallArgs g;
    g.a = a, g.b = b, g.c = c;
    g.sa = sa, g.sb = sb, g.sc = sc, g.ldc = ldc;
    g.m = m, g.n = n, g.k = k;
    g.lda4 = (uint32_t)(lda * 4), g.ldb4 = (uint32_t)(ldb * 4);
    g.nrec_a = (uint32_t)(ta ? slice_bytes(k, m, lda) : slice_bytes(m, k, lda));
    g.nrec_b = (uint32_t)(tb ? slice_bytes(n, k, ldb) : slice_bytes(k, n, ldb));
    g.tiles_n = (int)ceil_div(n, 32), g.tiles_m = (int)ceil_div(m, 32);
    if (!ta && !tb) return launch_small<0, 0>(g, a, lda, sa, b, ldb, sb, batch, s);
    if (!ta && tb) return launch_small<0, 1>(g, a, lda, sa, b, ldb, sb, batch, s);
    if (ta && !tb) return launch_small<1, 0>(g, a, lda, sa, b, ldb, sb, batch, s);
    return launch_small<1, 1>(g, a, lda, sa, b, ldb, sb, batch, s);
}

}  // namespace mlxhip
