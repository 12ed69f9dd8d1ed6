// gemm_thin.hip — batched f32 products of attention over many heads, where
// one extent is the head dimension: the scores C_b[M,N] = A_b[M,K]
// B_b[N,K]^T with K <= 64 (S = Q K^T, dP = dO V^T; gemm_thin_nt_kernel) and
// the outputs C_b[M,64] = op(A_b) B_b (P V, dS K, P^T dO, dS^T Q;
// gemm_thin_n64_kernel, further below), as config 4's composed block
// computes them for 64 heads of [512, 64]. They replace matmul
// (crates/mlx-core/src/cpu_kernels.rs:197-230) at these shapes.
//
// Such a product writes far more than it reads (C is M x N, the operands
// M x K and N x K), so it runs at the rate C can be written, as long as the
// stores of some tiles overlap the loads and MFMAs of others. A block-tiled
// GEMM with one large tile per CU does the opposite: every CU loads, then
// computes, then stores its whole tile at the same moment as every other
// CU.
//
// Here a workgroup of 4 waves owns a 64 x 128 block of C, and three
// workgroups share a CU, each in its own phase. The block's rows of A and B
// (K padded with zeros to KP = 2 KH, KH = 8, 16 or 32) come in with
// coalesced 16-byte loads (KP / 4 lanes per row) and go to LDS rows of
// KP + 4 floats; after one barrier each wave computes a 32 x 64 tile from
// LDS. The K axis is cut into two runs of KH, one per half-wave: at step i
// of v_mfma_f32_32x32x2_f32 lane (r, h) supplies A[m + r][KH h + i] and
// B[n + 32 t + r][KH h + i] for the tile's column half t, read from LDS
// with 16-byte reads. (Reading those runs straight from memory, a lane per
// row, touches 64 cache lines per load instruction and ran at two thirds of
// the block-tiled kernel's speed.) Products are exact f32 MFMA products
// with f32 sums, as in the general kernel, one accumulator chain per column
// half (the two chains alternate, so neither waits on its own previous
// MFMA). Accumulator element v of lane (r, h) is C[8 (v / 4) + 4 h +
// v % 4][r], so each store instruction writes two 128-byte row segments.
//
// Workgroups are ordered so that each XCD takes a contiguous range of
// batch slices: a slice's operands are fetched into one L2.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "../common.hpp"
#include "../kernels.hpp"

namespace mlxhip {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr uint32_t OOB_OFF = 0xFFFFFF00u;  // beyond every descriptor range (slices are < 2 GiB)
constexpr int BUF_FLAGS = 0x00020000;      // gfx9 buffer descriptor word 3 (32-bit data format)
constexpr int64_t SLICE_MAX_BYTES = (int64_t(1) << 31) - 256;
constexpr int BM = 64, BN = 128;            // workgroup block
constexpr int THREADS = 256;
constexpr int C_POLICY = 2;                 // C stores: non-temporal (written once, read by a later kernel)

struct ThinArgs {
    const float* a;
    const float* b;
    float* c;
    int64_t sa, sb, sc, ldc;
    uint32_t lda4, ldb4, ldc4;        // leading dimensions in bytes
    uint32_t nrec_a, nrec_b, nrec_c;  // descriptor ranges: one slice's bytes
    int k;
    int blocks_m, blocks_n;   // workgroup blocks per slice
    int blocks;               // in all
    // Slice bt starts (bt / inner) * s + (bt % inner) * s2 elements into its
    // operand (s = sa, sb or sc; s2 = sa2, sb2 or sc2): heads of a
    // [batch, seq, heads * dh] row-major tensor are slices with inner =
    // heads, s = seq * heads * dh and s2 = dh. inner = 1: plain strides.
    int inner;
    int64_t sa2, sb2, sc2;
};

__device__ inline int64_t slice_at(int bt, int inner, int64_t s, int64_t s2) {
    const int o = bt / inner;
    return o * s + (int64_t)(bt - o * inner) * s2;
}

template <int KH>
__global__ __launch_bounds__(THREADS) void gemm_thin_nt_kernel(ThinArgs g) {
    constexpr int KP = 2 * KH, PITCH = KP + 4, CPR = KP / 4;  // 16-byte chunks per row
    __shared__ __attribute__((aligned(16))) float lds[(BM + BN) * PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per_slice = g.blocks_m * g.blocks_n;
    // Block j of this workgroup (g.blocks past the last one): XCD x
    // (workgroup i runs on XCD i % 8) walks its own contiguous eighth of the
    // blocks when they divide evenly.
    const int nwg = (int)gridDim.x, w = (int)blockIdx.x;
    const bool remap = (g.blocks & 7) == 0 && (nwg & 7) == 0;
    auto block_of = [&](int j) {
        if (!remap) return w + j * nwg;
        const int l = (w >> 3) + j * (nwg >> 3);
        return l < (g.blocks >> 3) ? (w & 7) * (g.blocks >> 3) + l : g.blocks;
    };
    // Chunk c of a block: row c / CPR, k = 4 (c % CPR). K is a multiple of
    // 4, so a chunk is wholly inside K or wholly past it (zeros).
    constexpr int CA = BM * CPR / THREADS, CB = BN * CPR / THREADS;
    static_assert(CA * THREADS == BM * CPR && CB * THREADS == BN * CPR, "whole chunks per thread");
    f32x4v xa[CA], xb[CB];
    auto issue = [&](int blk) {
        const int bt = blk / per_slice, id = blk - bt * per_slice;
        const int64_t m0 = (int64_t)(id / g.blocks_n) * BM, n0 = (int64_t)(id % g.blocks_n) * BN;
        const __amdgpu_buffer_rsrc_t ra =
            __builtin_amdgcn_make_buffer_rsrc((void*)(g.a + slice_at(bt, g.inner, g.sa, g.sa2)), (short)0, (int)g.nrec_a, BUF_FLAGS);
        const __amdgpu_buffer_rsrc_t rb =
            __builtin_amdgcn_make_buffer_rsrc((void*)(g.b + slice_at(bt, g.inner, g.sb, g.sb2)), (short)0, (int)g.nrec_b, BUF_FLAGS);
#pragma unroll
        for (int j = 0; j < CA; ++j) {
            const int c = tid + THREADS * j, row = c / CPR, k = 4 * (c % CPR);
            const uint32_t off = k < g.k ? (uint32_t)(m0 + row) * g.lda4 + 4u * k : OOB_OFF;
            xa[j] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int c = tid + THREADS * j, row = c / CPR, k = 4 * (c % CPR);
            const uint32_t off = k < g.k ? (uint32_t)(n0 + row) * g.ldb4 + 4u * k : OOB_OFF;
            xb[j] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int j = 0; j < CA; ++j) {
            const int c = tid + THREADS * j;
            *reinterpret_cast<f32x4v*>(&lds[(c / CPR) * PITCH + 4 * (c % CPR)]) = xa[j];
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int c = tid + THREADS * j;
            *reinterpret_cast<f32x4v*>(&lds[(BM + c / CPR) * PITCH + 4 * (c % CPR)]) = xb[j];
        }
    };
    const int r = lane & 31, h = lane >> 5, wm = wave >> 1, wn = wave & 1;
    const float* pa = &lds[(32 * wm + r) * PITCH + KH * h];
    const float* pb = &lds[(BM + 64 * wn + r) * PITCH + KH * h];
    // Block blk's C through a buffer descriptor over its slice: the lane's
    // byte offset (row 4 h, column r of the wave's 32 x 64 tile) in a VGPR,
    // the per-element part (row 8 (v / 4) + v % 4, column 32 t) uniform.
    struct COut {
        __amdgpu_buffer_rsrc_t rs;
        uint32_t off;
    };
    auto c_out = [&](int blk) {
        const int bt = blk / per_slice, id = blk - bt * per_slice;
        const int64_t m0 = (int64_t)(id / g.blocks_n) * BM, n0 = (int64_t)(id % g.blocks_n) * BN;
        COut o;
        o.rs = __builtin_amdgcn_make_buffer_rsrc((void*)(g.c + slice_at(bt, g.inner, g.sc, g.sc2)), (short)0, (int)g.nrec_c, BUF_FLAGS);
        o.off = (uint32_t)(((m0 + 32 * wm + 4 * h) * g.ldc + n0 + 64 * wn + r) * 4);
        return o;
    };
    auto store_one = [&](const f32x16 (&acc)[2], const COut& o, int e) {
        const int t = e >> 4, v = e & 15;
        const uint32_t so = (uint32_t)(8 * (v >> 2) + (v & 3)) * g.ldc4 + 128u * t;
        // The element as a scalar first: a bit cast of the vector element
        // itself read element 0 of the vector.
        const float x = acc[t][v];
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), o.rs, o.off, so, C_POLICY);
    };
    // The MFMAs of the block whose operands are in LDS into `cur`; with
    // WITH_PREV, the 32 stores of the previous block's `prev` go out between
    // them (32 / KH per step), so a wave whose store has to wait for the
    // memory system holds up at most one step's MFMAs instead of a whole
    // block's.
    auto compute = [&](f32x16 (&cur)[2], const f32x16 (&prev)[2], const COut& po, auto with_prev) {
        float av[KH], bv[2][KH];
#pragma unroll
        for (int i = 0; i < KH; i += 4) {
            const f32x4v x = *reinterpret_cast<const f32x4v*>(pa + i);
            const f32x4v y0 = *reinterpret_cast<const f32x4v*>(pb + i);
            const f32x4v y1 = *reinterpret_cast<const f32x4v*>(pb + 32 * PITCH + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) av[i + e] = x[e], bv[0][i + e] = y0[e], bv[1][i + e] = y1[e];
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) cur[t][v] = 0.0f;
        constexpr int SPS = 32 / KH;  // stores per step
#pragma unroll
        for (int i = 0; i < KH; ++i) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
                cur[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[t][i], cur[t], 0, 0, 0);
            if constexpr (decltype(with_prev)::value) {
#pragma unroll
                for (int q = 0; q < SPS; ++q) store_one(prev, po, i * SPS + q);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto store_all = [&](const f32x16 (&acc)[2], const COut& o) {
#pragma unroll
        for (int e = 0; e < 32; ++e) store_one(acc, o, e);
    };
    // Requests block nxt's operands (before any store of the current step:
    // memory operations complete in order, so the wait for them in stage()
    // leaves the stores in flight).
    auto next = [&](int j, int& nxt) {
        nxt = block_of(j);
        const bool more = nxt < g.blocks;
        if (more) issue(nxt);
        return more;
    };
    auto advance = [&]() {
        __syncthreads();  // every wave has read this block's operands from LDS
        stage();
        __syncthreads();
    };

    f32x16 acc0[2], acc1[2];
    int blk = block_of(0), nxt = 0;
    issue(blk);
    stage();
    __syncthreads();
    bool more = next(1, nxt);
    COut po = c_out(blk);
    compute(acc0, acc1, po, std::false_type{});
    if (!more) {
        store_all(acc0, po);
        return;
    }
    advance();
    blk = nxt;
    for (int j = 2;; j += 2) {
        more = next(j, nxt);
        compute(acc1, acc0, po, std::true_type{});
        po = c_out(blk);
        if (!more) {
            store_all(acc1, po);
            return;
        }
        advance();
        blk = nxt;
        more = next(j + 1, nxt);
        compute(acc0, acc1, po, std::true_type{});
        po = c_out(blk);
        if (!more) {
            store_all(acc0, po);
            return;
        }
        advance();
        blk = nxt;
    }
}

// C_b[M, 64] = op(A_b) B_b with B [K][64] (N-contiguous) and op(A) = A
// [M][K] (TA = 0) or A^T with A [K][M] (TA = 1): the products of attention
// with the head dimension as N (P V, dS K, P^T dO, dS^T Q), which read a
// large A once and write a small C. A workgroup owns 64 rows of C (all 64
// columns); K streams through two LDS stages of 64 k each (coalesced
// 16-byte loads of the next chunk in flight while the current one is
// multiplied, one barrier per chunk; A's loads non-temporal with APOL = 2,
// as A is read once). KS groups of 4 waves split each chunk's k; each wave
// computes a 32 x 32 tile, lane (r, h) taking k = KW g + (KW / 2) h + i of
// the chunk at step i (KW = 64 / KS, g its group), so a K-contiguous A
// gives it 16-byte LDS reads along its row (rows of 68 floats), while an
// N- or M-contiguous operand is read one float per step across the lanes'
// consecutive columns (rows of 65 floats: the two half-waves' rows fall in
// different banks). Two accumulator chains (even and odd steps) are added
// at the end, then the groups' tiles in group order through LDS; C goes out
// with non-temporal stores. On 64 heads of [512, 512] x [512, 64]: KS = 2
// 25.3-25.7 us (P V) and 27.3 us (P^T dO) against 27.3 and 28.8-29.0 with
// KS = 1 and A loads cached.
template <int TA, int KS, int APOL>
__global__ __launch_bounds__(THREADS * KS) void gemm_thin_n64_kernel(ThinArgs g) {
    constexpr int NT = THREADS * KS;                // KS wave groups split each chunk's k
    constexpr int KC = 64;                          // k per chunk
    constexpr int KW = KC / KS;                     // k per wave group and chunk
    constexpr int PA = TA ? 65 : KC + 4, PB = 65;   // LDS row pitches (floats)
    constexpr int SA = 64 * PA, SB = KC * PB;       // one stage of A ([m][k] or [k][m]) and of B ([k][n])
    __shared__ __attribute__((aligned(16))) float lds[2 * (SA + SB)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwg = (int)gridDim.x;
    int w = (int)blockIdx.x;
    if ((nwg & 7) == 0) w = (w & 7) * (nwg >> 3) + (w >> 3);
    const int bt = w / g.blocks_m;
    const int64_t m0 = (int64_t)(w - bt * g.blocks_m) * 64;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.a + slice_at(bt, g.inner, g.sa, g.sa2)), (short)0, (int)g.nrec_a, BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.b + slice_at(bt, g.inner, g.sb, g.sb2)), (short)0, (int)g.nrec_b, BUF_FLAGS);
    // Chunk loads: 64 rows of 64 floats for each operand, 16 lanes per row.
    // A's rows are m (TA = 0, k along the row) or k (TA = 1, m along the
    // row); B's rows are k.
    constexpr int LPT = 1024 / NT;  // 16-byte loads per thread and operand
    f32x4v xa[LPT], xb[LPT];
    auto issue = [&](int k0) {
#pragma unroll
        for (int j = 0; j < LPT; ++j) {
            const int c = tid + NT * j, row = c >> 4, q = c & 15;
            const uint32_t oa = TA ? (uint32_t)(k0 + row) * g.lda4 + (uint32_t)(m0 + 4 * q) * 4u
                                   : (uint32_t)(m0 + row) * g.lda4 + (uint32_t)(k0 + 4 * q) * 4u;
            xa[j] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(ra, oa, 0, APOL));
            xb[j] = __builtin_bit_cast(
                f32x4v, __builtin_amdgcn_raw_buffer_load_b128(rb, (uint32_t)(k0 + row) * g.ldb4 + 16u * q, 0, 0));
        }
    };
    auto stage = [&](int st) {
        float* la = lds + st * (SA + SB);
        float* lb = la + SA;
#pragma unroll
        for (int j = 0; j < LPT; ++j) {
            const int c = tid + NT * j, row = c >> 4, q = c & 15;
            if constexpr (TA) {
#pragma unroll
                for (int e = 0; e < 4; ++e) la[row * PA + 4 * q + e] = xa[j][e];
            } else {
                *reinterpret_cast<f32x4v*>(&la[row * PA + 4 * q]) = xa[j];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) lb[row * PB + 4 * q + e] = xb[j][e];
        }
    };
    const int r = lane & 31, h = lane >> 5, wq = wave & 3, wk = wave >> 2, wm = wq >> 1, wn = wq & 1;
    const int kw = KW * wk + (KW / 2) * h;  // this lane's first k of each chunk
    f32x16 acc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.0f;
    const int nch = g.k / KC;
    issue(0);
    stage(0);
    __syncthreads();
    for (int ch = 0; ch < nch; ++ch) {
        const bool more = ch + 1 < nch;
        if (more) issue((ch + 1) * KC);
        const float* la = lds + (ch & 1) * (SA + SB);
        const float* lb = la + SA;
#pragma unroll
        for (int i0 = 0; i0 < KW / 2; i0 += 4) {
            float av[4], bv[4];
            if constexpr (TA) {
#pragma unroll
                for (int e = 0; e < 4; ++e) av[e] = la[(kw + i0 + e) * PA + 32 * wm + r];
            } else {
                const f32x4v x = *reinterpret_cast<const f32x4v*>(&la[(32 * wm + r) * PA + kw + i0]);
#pragma unroll
                for (int e = 0; e < 4; ++e) av[e] = x[e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = lb[(kw + i0 + e) * PB + 32 * wn + r];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc[e & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], bv[e], acc[e & 1], 0, 0, 0);
        }
        if (more) stage((ch + 1) & 1);  // its previous contents were read before the last barrier
        __syncthreads();
    }
    f32x16 sum;
#pragma unroll
    for (int v = 0; v < 16; ++v) sum[v] = acc[0][v] + acc[1][v];
    if constexpr (KS > 1) {
        // The second wave group's partial tiles through LDS, added after the
        // first group's (fixed order).
        float* part = lds;  // [4 waves][16][64 lanes]; the stages are free after the last barrier
        if (wk == 1) {
#pragma unroll
            for (int v = 0; v < 16; ++v) part[(wq * 16 + v) * 64 + lane] = sum[v];
        }
        __syncthreads();
        if (wk == 1) return;
#pragma unroll
        for (int v = 0; v < 16; ++v) sum[v] += part[(wq * 16 + v) * 64 + lane];
    }
    const __amdgpu_buffer_rsrc_t rc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(g.c + slice_at(bt, g.inner, g.sc, g.sc2)), (short)0, (int)g.nrec_c, BUF_FLAGS);
    const uint32_t off = (uint32_t)(((m0 + 32 * wm + 4 * h) * g.ldc + 32 * wn + r) * 4);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const float x = sum[v];
        const uint32_t so = (uint32_t)(8 * (v >> 2) + (v & 3)) * g.ldc4;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), rc, off, so, C_POLICY);
    }
}

int64_t slice_bytes(int64_t rows, int64_t cols, int64_t ld) { return ((rows - 1) * ld + cols) * 4; }

// Compute units of the current device (256 on MI355X), read once per device.
int cu_count() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
    return n;
}


bool gemm_thin_f32_fits(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const void* a,
                        int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, const void* c,
                        int64_t ldc, int64_t sc) {
    // A [M][K] and B [N][K] (C = A B^T), whole blocks, 16-byte runs along K,
    // 32-bit offsets inside each slice, and enough blocks for several per CU
    // (fewer go to the block-tiled kernels).
    if (ta != 0 || tb != 1 || k < 1 || k > 64 || k % 4 || m % BM || n % BN || batch < 1) return false;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (!al(a) || !al(b) || !c || lda % 4 || ldb % 4 || (batch > 1 && (sa % 4 || sb % 4))) return false;
    if (ldc < n || slice_bytes(m, k, lda) >= SLICE_MAX_BYTES || slice_bytes(n, k, ldb) >= SLICE_MAX_BYTES ||
        slice_bytes(m, n, ldc) >= SLICE_MAX_BYTES)
        return false;
    (void)sc;
    const int64_t blocks = (m / BM) * (n / BN) * batch;
    return blocks >= 1024 && blocks <= INT32_MAX;
}

// Both thin kernels' shared checks on one operand or C: a 16-byte-aligned
// base, leading dimension and slice strides (so every slice starts on a
// 16-byte boundary), and a slice (rows runs of cols, ld apart) addressable
// with 32-bit offsets.
bool view_ok(const ThinView& v, int64_t rows, int64_t cols, int64_t batch, int inner) {
    if (!v.p || reinterpret_cast<uintptr_t>(v.p) % 16 || v.ld < cols || v.ld % 4) return false;
    if (batch > inner && v.s % 4) return false;
    if (inner > 1 && v.s2 % 4) return false;
    return slice_bytes(rows, cols, v.ld) < SLICE_MAX_BYTES;
}

int thin_kind(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, int inner, const ThinView& a,
              const ThinView& b, const ThinView& c) {
    if (m < 1 || n < 1 || k < 1 || batch < 1 || inner < 1 || batch % inner) return 0;
    if (!view_ok(c, m, n, batch, inner)) return 0;
    // Scores: C = A B^T, A [M][K], B [N][K], K <= 64; whole 64 x 128 blocks
    // and enough of them for several per CU (fewer go to the block-tiled
    // kernels).
    if (ta == 0 && tb == 1 && k <= 64 && k % 4 == 0 && m % BM == 0 && n % BN == 0 && view_ok(a, m, k, batch, inner) &&
        view_ok(b, n, k, batch, inner)) {
        const int64_t blocks = (m / BM) * (n / BN) * batch;
        if (blocks >= 1024 && blocks <= INT32_MAX) return 1;
    }
    // Head-dimension outputs: op(A) [M][K] times B [K][64], whole 64-row
    // blocks, whole chunks of 64 k, at least two blocks per CU.
    if (tb == 0 && n == 64 && k % 64 == 0 && m % 64 == 0 && (ta ? view_ok(a, k, m, batch, inner) : view_ok(a, m, k, batch, inner)) &&
        view_ok(b, k, n, batch, inner)) {
        const int64_t blocks = (m / 64) * batch;
        if (blocks >= 512 && blocks <= INT32_MAX) return 2;
    }
    return 0;
}

}  // namespace

bool gemm_thin_view_fits(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, int inner,
                         const ThinView& a, const ThinView& b, const ThinView& c) {
    return thin_kind(ta, tb, m, n, k, batch, inner, a, b, c) != 0;
}

int gemm_thin_view(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, int inner, const ThinView& a,
                   const ThinView& b, const ThinView& c, hipStream_t s) {
    const int kind = thin_kind(ta, tb, m, n, k, batch, inner, a, b, c);
    if (!kind) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm_thin: shape or layout outside the thin kernels' range");
    ThinArgs g{};
    g.a = a.p, g.b = b.p, g.c = const_cast<float*>(c.p);
    g.sa = a.s, g.sb = b.s, g.sc = c.s, g.sa2 = a.s2, g.sb2 = b.s2, g.sc2 = c.s2, g.inner = inner;
    g.ldc = c.ld;
    g.lda4 = (uint32_t)(a.ld * 4), g.ldb4 = (uint32_t)(b.ld * 4), g.ldc4 = (uint32_t)(c.ld * 4);
    g.nrec_c = (uint32_t)slice_bytes(m, n, c.ld);
    g.k = (int)k;
    if (kind == 2) {
        g.nrec_a = (uint32_t)(ta ? slice_bytes(k, m, a.ld) : slice_bytes(m, k, a.ld));
        g.nrec_b = (uint32_t)slice_bytes(k, n, b.ld);
        g.blocks_m = (int)(m / 64), g.blocks_n = 1;
        g.blocks = (int)(g.blocks_m * batch);
        const dim3 grid((unsigned)g.blocks);
        constexpr int KS = 2, APOL = 2;  // two wave groups per chunk; A read once, non-temporally
        if (ta) hipLaunchKernelGGL((gemm_thin_n64_kernel<1, KS, APOL>), grid, dim3(THREADS * KS), 0, s, g);
        else hipLaunchKernelGGL((gemm_thin_n64_kernel<0, KS, APOL>), grid, dim3(THREADS * KS), 0, s, g);
        return launch_check("gemm_thin_n64_kernel");
    }
    g.nrec_a = (uint32_t)slice_bytes(m, k, a.ld);
    g.nrec_b = (uint32_t)slice_bytes(n, k, b.ld);
    g.blocks_m = (int)(m / BM), g.blocks_n = (int)(n / BN);
    g.blocks = (int)(g.blocks_m * g.blocks_n * batch);
    // Persistent workgroups, two per CU (each block of every workgroup
    // overlaps its C stores with the next block's loads and MFMAs).
    const int per_cu = 2;
    const dim3 grid((unsigned)std::min(g.blocks, per_cu * cu_count())), block(THREADS);
    if (k <= 16) hipLaunchKernelGGL(gemm_thin_nt_kernel<8>, grid, block, 0, s, g);
    else if (k <= 32) hipLaunchKernelGGL(gemm_thin_nt_kernel<16>, grid, block, 0, s, g);
    else hipLaunchKernelGGL(gemm_thin_nt_kernel<32>, grid, block, 0, s, g);
    return launch_check("gemm_thin_nt_kernel");
}

bool gemm_thin_f32_fits(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const void* a,
                        int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, const void* c,
                        int64_t ldc, int64_t sc) {
    return gemm_thin_view_fits(ta, tb, m, n, k, batch, 1, ThinView{static_cast<const float*>(a), lda, sa, 0},
                               ThinView{static_cast<const float*>(b), ldb, sb, 0},
                               ThinView{static_cast<const float*>(c), ldc, sc, 0});
}

int gemm_thin_f32(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const float* a, int64_t lda,
                  int64_t sa, const float* b, int64_t ldb, int64_t sb, float* c, int64_t ldc, int64_t sc,
                  hipStream_t s) {
    return gemm_thin_view(ta, tb, m, n, k, batch, 1, ThinView{a, lda, sa, 0}, ThinView{b, ldb, sb, 0},
                          ThinView{c, ldc, sc, 0}, s);
}

}  // namespace mlxhip
