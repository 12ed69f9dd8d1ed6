// gemm16_small.hip — bf16 / f16 GEMM in one launch for products whose
// operands the direct-to-LDS kernel cannot read as they are (rows that are
// not whole 16-byte chunks: odd K or N, offset pointers) or that have too
// few 128 x 128 tiles to occupy the chip; replaces the pack / split-K /
// partial-sum sequence there.
//
// C_b[M,N] = op(A_b) * op(B_b), f32 accumulation, C in f32 / bf16 / f16
// (round to nearest even); replaces matmul (crates/mlx-core/src/
// cpu_kernels.rs:197-230) at these shapes (config 3's 1000 x 777 x 1531).
//
// Work decomposition
//   * One workgroup per 64 x 64 tile of C, gridDim.y = batch: KS groups of 4
//     waves (2 x 2 waves of 32 x 32, one v_mfma_f32_32x32x16 accumulator
//     each), group i over the i-th part of K; the groups' partial tiles meet
//     in LDS and are added in group order. The odd config-3 product makes 208
//     workgroups of 16 waves (4 per SIMD), so no second kernel.
//   * K tiles of 64. Each thread moves two 8-element chunks of each operand
//     per K tile: chunk = 8 consecutive elements along the operand's
//     contiguous axis. A chunk is read as one 16-byte buffer load from the
//     dword boundary at or below its first element and shifted down by one
//     element when that element sits at an odd position (any 2-byte-aligned
//     operand), then elements past the matrix edge are zeroed. Dwords past
//     the descriptor's range (the slice) read as zeros. The fifth dword an
//     odd chunk needs is the next lane's first: taken from it with a DPP
//     row shift, and loaded (4 bytes) only by the last lane of each group of
//     8 and where the next chunk lies outside the matrix.
//   * Loads run DEPTH K tiles ahead in registers (20 VGPRs per tile), so the
//     L2 / HBM latency overlaps DEPTH tiles of work per group; LDS is
//     double-buffered per group with one barrier per K tile.
//   * LDS holds both operands K-contiguous, [64 rows][64 k], 16-byte chunks
//     XOR-swizzled per row (lds_at): a K-contiguous chunk is one
//     ds_write_b128, an MN-contiguous chunk is written transposed as 8
//     ds_write_b16. Fragments are ds_read_b128 (lane = row l % 32, k-group
//     l / 32).
//   * MFMA roles are swapped (src_a = B fragment) as in the 16-bit kernel of
//     gemm16_impl.hpp: lane l then holds C[m][n .. n+3] for m = l % 32.
#include "../common.hpp"
#include "../kernels.hpp"

namespace mlxhip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
#define SMALL16_LDS __attribute__((address_space(3)))

constexpr int TILE = 64, BK = 64;
constexpr uint32_t OOB_OFF = 0xFFFFFF00u;      // beyond every descriptor range
constexpr int BUF_FLAGS = 0x00020000;          // gfx9 buffer descriptor word 3 (32-bit data format)

struct Small16Args {
    int64_t m, n, k;
    const void* a;
    int64_t lda, sa;
    const void* b;
    int64_t ldb, sb;
    void* c;
    int64_t ldc, sc;
    int tiles_n;
};

// One operand of one batch slice: a buffer descriptor from the dword
// boundary at or below the slice's first element to its last byte, and the
// element index (from that boundary) of the slice's element 0.
struct Operand {
    __amdgpu_buffer_rsrc_t rsrc;
    int64_t e0;
    uint32_t nrec;  // descriptor range: the slice's bytes rounded up to whole dwords
};

__device__ inline Operand make_operand(const void* p, int64_t slice_off, int64_t rows, int64_t cols, int64_t ld) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(p) + (uintptr_t)(slice_off * 2);
    const uintptr_t base = addr & ~uintptr_t(3);
    const int64_t e0 = (int64_t)((addr - base) >> 1);
    const int64_t bytes = rows > 0 && cols > 0 ? (e0 + (rows - 1) * ld + cols) * 2 : 0;
    Operand o;
    o.nrec = (uint32_t)((bytes + 3) & ~int64_t(3));
    o.rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)o.nrec, BUF_FLAGS);
    o.e0 = e0;
    return o;
}

// The raw dwords of one chunk: 5 dwords from the dword boundary at or below
// element e (or zeros for an out-of-range chunk).
struct Raw {
    u32x4 lo;
    uint32_t hi;
};

// Keep-masks of a chunk's 4 dwords (element 2j in the low half of dword
// j) when only its first `valid` elements (0 .. 8) are inside the matrix.
__device__ inline u32x4 chunk_keep(int valid) {
    auto keep = [valid](int j) {
        return (2 * j + 1 < valid ? 0xFFFF0000u : 0u) | (2 * j < valid ? 0x0000FFFFu : 0u);
    };
    return u32x4{keep(0), keep(1), keep(2), keep(3)};
}

// LDS position (in elements) of the 8-element chunk c (k = 8c .. 8c+7) of
// tile row `row`: rows of 64 elements (128 bytes), chunks XOR-swizzled by
// the row's low three bits (8 consecutive rows, as a fragment read takes
// them, land in 8 distinct 16-byte bank groups) and by the row's group of 8
// (8 rows 8 apart, as a transposed chunk writes them, do too).
__device__ inline int lds_at(int row, int c) { return row * TILE + 8 * (c ^ (row & 7) ^ ((row >> 3) & 7)); }

// One of a thread's two chunks of one operand, for the whole K loop. Chunk i
// of thread q covers, in every K tile: KC (operand stored [R][K]) row q / 8
// and k = 8 (q % 8) .. +7 of the tile; otherwise (stored [K][R]) k = q / 8
// and rows 8 (q % 8) .. +7. Everything that does not change from one K tile
// to the next is worked out once, in 32-bit arithmetic: the byte offset of
// the chunk's first dword in tile 0 (the next tile's is a fixed step
// further: 64 elements along K), the funnel-shift amount (the element's
// parity, the same in every tile since a tile step is an even number of
// elements), and whether its rows / columns are inside the matrix.
template <bool KC, bool SHARE = true>
struct Chunk {
    uint32_t off0;  // byte offset of the dword at or below the first element, tile 0
    uint32_t sh;    // 16 when that element is the upper half of its dword, else 0
    int k0;         // k of the chunk's first element in tile 0 (group-relative tile index 0)
    int lrow, lc;   // tile-local row (KC) / first row (MN), and 8-element chunk index along K
    bool ok;        // KC: its row is inside the matrix; MN: its first row is
    bool last;      // the last of the 8 lanes that share a row (KC) or a k (MN)
    bool nb_ok;     // MN: the next lane's first row is inside the matrix (KC: same row)
    u32x4 keep;     // MN: masks of the rows past the matrix edge (fixed)

    __device__ inline void init(const Operand& o, int q, int64_t r0, int64_t R, int64_t ld, int64_t kg) {
        int64_t e;
        last = (q & 7) == 7;
        nb_ok = true;
        if constexpr (KC) {
            lrow = q >> 3;
            lc = q & 7;
            k0 = (int)(kg + 8 * lc);
            const int64_t r = r0 + lrow;
            ok = r < R;
            e = o.e0 + (ok ? r : 0) * ld + k0;
            keep = u32x4{~0u, ~0u, ~0u, ~0u};
        } else {
            lrow = 8 * (q & 7);
            lc = (q >> 3) >> 3;
            k0 = (int)(kg + (q >> 3));
            const int64_t r = r0 + lrow;
            ok = r < R;
            e = o.e0 + (int64_t)k0 * ld + (ok ? r : 0);
            keep = chunk_keep((int)max<int64_t>(0, min<int64_t>(8, R - r)));
            nb_ok = r + 8 < R;
        }
        off0 = (uint32_t)((e >> 1) << 2);
        sh = (uint32_t)(e & 1) * 16;
    }

    // Whether this lane loads the fifth dword of its chunk in K tile t itself
    // (below).
    __device__ inline bool own(int t, int K) const {
        if constexpr (!SHARE) return true;
        else if constexpr (KC) return last || !(k0 + 8 + t * BK < K);
        else return last || !nb_ok;
    }

    // One 16-byte load (dword-aligned) of the chunk in K tile t
    // (group-relative), and the fifth dword, which only a chunk starting at
    // an odd element uses: it is the first dword of the next lane's chunk,
    // so only the last lane of each group of 8 (its neighbour's chunk is
    // not loaded here) and a lane whose neighbour's chunk lies outside the
    // matrix (read as zeros) load it themselves, 4 bytes; the others take
    // it from the neighbour in store(). `step` is the byte distance between
    // two K tiles.
    // Out-of-range chunks read through an offset past the descriptor's
    // range: zeros. The descriptor's range check is per dword, so a chunk
    // that ends its slice keeps its in-range dwords and reads zeros past
    // them (established on MI355X by an in-bounds probe); every dword read
    // lies inside the slice's last dword.
    __device__ inline void issue(const Operand& o, int t, uint32_t step, int K, Raw& r) const {
        const bool in = ok && k0 + t * BK < K;
        const uint32_t off = in ? off0 + (uint32_t)t * step : OOB_OFF;
        r.lo = __builtin_amdgcn_raw_buffer_load_b128(o.rsrc, off, 0, 0);
        r.hi = __builtin_amdgcn_raw_buffer_load_b32(o.rsrc, own(t, K) && sh ? off + 16 : OOB_OFF, 0, 0);
    }

    // The chunk's 8 elements of K tile t, shifted down one element when the
    // first one is at an odd position and masked past the matrix edge, into
    // the group's LDS stage. `tail`: K tile t holds the end of K (uniform
    // across the workgroup), where a K-contiguous chunk can straddle it.
    __device__ inline void store(const Raw& r, int t, int K, bool tail, SMALL16_LDS uint16_t* s) const {
        // The fifth dword: the next lane's first (DPP row_shl:1, lanes of a
        // group of 8 are consecutive within a row of 16), or this lane's own.
        const uint32_t nb = (uint32_t)__builtin_amdgcn_mov_dpp((int)r.lo.x, 0x101, 0xF, 0xF, false);
        const uint32_t hi = own(t, K) ? r.hi : nb;
        // Branch-free funnel shift by 0 or 16 bits, so the loads of later K
        // tiles stay in flight across it.
        u32x4 v{__builtin_amdgcn_alignbit(r.lo.y, r.lo.x, sh), __builtin_amdgcn_alignbit(r.lo.z, r.lo.y, sh),
                __builtin_amdgcn_alignbit(r.lo.w, r.lo.z, sh), __builtin_amdgcn_alignbit(hi, r.lo.w, sh)};
        if constexpr (KC) {
            // Elements past K belong to the next row: zero them (only in the
            // tile holding the end of K; chunks wholly past K read zeros).
            if (tail) v &= chunk_keep(max(0, min(8, K - (k0 + t * BK))));
            *(SMALL16_LDS u32x4*)(s + lds_at(lrow, lc)) = v;
        } else {
            v &= keep;
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            const int kk = (k0 & 63) & 7;
#pragma unroll
            for (int j = 0; j < 8; ++j) s[lds_at(lrow + j, lc) + kk] = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
        }
    }
};

template <int DT>
__device__ inline void mfma16(const u32x4& a, const u32x4& b, f32x16& acc) {
    if constexpr (DT == MLXHIP_DTYPE_BF16)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                      acc, 0, 0, 0);
    else
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                     acc, 0, 0, 0);
}

template <int CT>
__device__ inline void store_elem(void* c, int64_t idx, float v) {
    if constexpr (CT == MLXHIP_DTYPE_F32) {
        static_cast<float*>(c)[idx] = v;
    } else if constexpr (CT == MLXHIP_DTYPE_BF16) {
        static_cast<__bf16*>(c)[idx] = (__bf16)v;  // round to nearest even
    } else {
        static_cast<_Float16*>(c)[idx] = (_Float16)v;
    }
}

template <int DT, int CT, bool KCA, bool KCB, int KS, int DEPTH>
__global__ __attribute__((amdgpu_flat_work_group_size(256 * KS, 256 * KS), amdgpu_waves_per_eu(KS, KS)))
void gemm16_small_kernel(Small16Args g) {
    // KS groups of 4 waves, group i over its own contiguous range of K tiles
    // with its own double-buffered LDS stages; the groups' partial tiles are
    // added in group order at the end (deterministic).
    __shared__ __attribute__((aligned(16))) uint16_t smem[KS][2][2][TILE * TILE];  // [group][stage][A, B]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, lw = wave & 3, ltid = tid & 255;
    const int wm = lw >> 1, wn = lw & 1;
    // XCD-aware tile order: the hardware hands consecutive workgroup ids
    // to the 8 XCDs in turn; give each XCD a contiguous range of (slice,
    // tile) ids, i.e. whole rows of tiles, so its L2 holds the few A panels
    // and the B panels its tiles share (the odd config-3 product: 2 tile
    // rows per XCD, 2.8 MB, instead of all of A and B in every XCD's 4 MB L2).
    const int64_t nt = (int64_t)gridDim.x * gridDim.y;
    int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    if ((nt & 7) == 0) lin = (lin & 7) * (nt >> 3) + (lin >> 3);
    const int64_t batch = lin / gridDim.x;
    const int64_t tile = lin - batch * gridDim.x;
    const int64_t m0 = (tile / g.tiles_n) * TILE, n0 = (tile % g.tiles_n) * TILE;

    // A: op(A) is [M][K]; stored [M][K] (KCA) or [K][M]. B: op(B) is [K][N];
    // stored [N][K] (KCB) or [K][N].
    const Operand oa = make_operand(g.a, batch * g.sa, KCA ? g.m : g.k, KCA ? g.k : g.m, g.lda);
    const Operand ob = make_operand(g.b, batch * g.sb, KCB ? g.n : g.k, KCB ? g.k : g.n, g.ldb);
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;

    // Every group runs the same number of K tiles, a whole number of DEPTH
    // groups, so the loop body has no conditional steps (tiles past K load
    // and multiply zeros), the barriers line up across groups, and the
    // compiler's load-wait counts stay those of the steady state.
    const int K = (int)g.k;
    const int nkt = (K + BK - 1) / BK;
    const int ntg = (((nkt + KS - 1) / KS) + DEPTH - 1) / DEPTH * DEPTH;
    const int kg = grp * ntg * BK;  // first k of this group
    // Byte distance between consecutive K tiles of a chunk: 64 elements
    // along K (K-contiguous) or 64 rows of the leading dimension.
    const uint32_t step_a = KCA ? 2u * BK : (uint32_t)(2 * BK * g.lda);
    const uint32_t step_b = KCB ? 2u * BK : (uint32_t)(2 * BK * g.ldb);
    // With both operands M/N-contiguous (8 transposed LDS writes per chunk
    // each) every lane loads its own fifth dwords: sharing them spilled
    // registers at 4 waves per SIMD.
    Chunk<KCA, KCA || KCB> ca[2];
    Chunk<KCB, KCA || KCB> cb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ca[i].init(oa, ltid + 256 * i, m0, g.m, g.lda, kg);
        cb[i].init(ob, ltid + 256 * i, n0, g.n, g.ldb, kg);
    }
    Raw ra[DEPTH][2], rb[DEPTH][2];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            ca[i].issue(oa, d, step_a, K, ra[d][i]);
            cb[i].issue(ob, d, step_b, K, rb[d][i]);
        }
    const int fr = lane & 31, fc = lane >> 5;
    for (int t0 = 0; t0 < ntg; t0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int t = t0 + d;
            SMALL16_LDS uint16_t* sa = (SMALL16_LDS uint16_t*)smem[grp][t & 1][0];
            SMALL16_LDS uint16_t* sb = (SMALL16_LDS uint16_t*)smem[grp][t & 1][1];
            const bool tail = kg + (t + 1) * BK > K;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ca[i].store(ra[d][i], t, K, tail, sa);
                cb[i].store(rb[d][i], t, K, tail, sb);
            }
            __syncthreads();
            // Tile t + DEPTH into the registers just consumed (zeros past K).
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ca[i].issue(oa, t + DEPTH, step_a, K, ra[d][i]);
                cb[i].issue(ob, t + DEPTH, step_b, K, rb[d][i]);
            }
#pragma unroll
            for (int s = 0; s < BK / 16; ++s) {
                const u32x4 af = *(const SMALL16_LDS u32x4*)(sa + lds_at(32 * wm + fr, 2 * s + fc));
                const u32x4 bf = *(const SMALL16_LDS u32x4*)(sb + lds_at(32 * wn + fr, 2 * s + fc));
                mfma16<DT>(bf, af, acc);
            }
        }
    }

    if constexpr (KS > 1) {
        // Groups 1 .. KS-1 hand their partial tiles to group 0 through LDS
        // (reusing the stages once every group is done with them).
        __syncthreads();
        float* red = reinterpret_cast<float*>(&smem[0][0][0][0]);
        if (grp > 0) {
#pragma unroll
            for (int v = 0; v < 16; ++v) red[(((grp - 1) * 4 + lw) * 16 + v) * 64 + lane] = acc[v];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int j = 0; j < KS - 1; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] += red[((j * 4 + lw) * 16 + v) * 64 + lane];
    }

    // lane l: C[m][n + 8q + 4(l/32) + r] = acc[4q + r], m = 32 wm + l % 32.
    const int64_t m = m0 + 32 * wm + (lane & 31);
    if (m >= g.m) return;
    char* cbase = static_cast<char*>(g.c);
    const int64_t row = batch * g.sc + m * g.ldc;
    constexpr int ES = CT == MLXHIP_DTYPE_F32 ? 4 : 2;
    const bool vec = (reinterpret_cast<uintptr_t>(cbase) % (4 * ES)) == 0 && g.ldc % 4 == 0 && g.sc % 4 == 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + 32 * wn + 8 * q + 4 * (lane >> 5);
        if (vec && n + 3 < g.n) {
            if constexpr (CT == MLXHIP_DTYPE_F32) {
                *reinterpret_cast<float4*>(cbase + (row + n) * 4) =
                    float4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) store_elem<CT>(cbase, row + n + r, acc[4 * q + r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (n + r < g.n) store_elem<CT>(cbase, row + n + r, acc[4 * q + r]);
        }
    }
}

// K split over 4 groups of waves when K holds 8 or more K tiles, over 2 from
// 4 (MLXHIP_SMALL16_KSPLIT = 1, 2 or 4 forces it; tuning).
int small16_ksplit(int64_t k) {
    if (const char* e = getenv("MLXHIP_SMALL16_KSPLIT")) {
        const int v = atoi(e);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    const int64_t nkt = (k + BK - 1) / BK;
    return nkt >= 8 ? 4 : nkt >= 4 ? 2 : 1;
}

template <int DT, int CT, bool KCA, bool KCB>
void launch_ks(const Small16Args& a, dim3 grid, hipStream_t s) {
    switch (small16_ksplit(a.k)) {
        case 4: hipLaunchKernelGGL((gemm16_small_kernel<DT, CT, KCA, KCB, 4, 2>), grid, dim3(1024), 0, s, a); break;
        case 2: hipLaunchKernelGGL((gemm16_small_kernel<DT, CT, KCA, KCB, 2, 3>), grid, dim3(512), 0, s, a); break;
        default: hipLaunchKernelGGL((gemm16_small_kernel<DT, CT, KCA, KCB, 1, 3>), grid, dim3(256), 0, s, a);
    }
}

template <int DT, int CT>
int launch_small16(int ta, int tb, const Small16Args& a, int64_t batch, hipStream_t s) {
    const dim3 grid((unsigned)(ceil_div(a.m, TILE) * a.tiles_n), (unsigned)batch);
    // KCA: A stored [M][K] (not transposed); KCB: B stored [N][K] (transposed).
    if (!ta && !tb) launch_ks<DT, CT, true, false>(a, grid, s);
    else if (!ta && tb) launch_ks<DT, CT, true, true>(a, grid, s);
    else if (ta && !tb) launch_ks<DT, CT, false, false>(a, grid, s);
    else launch_ks<DT, CT, false, true>(a, grid, s);
    return launch_check("gemm16_small_kernel");
}

template <int DT>
int dispatch_ct(int c_dtype, int ta, int tb, const Small16Args& a, int64_t batch, hipStream_t s) {
    switch (c_dtype) {
        case MLXHIP_DTYPE_F32: return launch_small16<DT, MLXHIP_DTYPE_F32>(ta, tb, a, batch, s);
        case MLXHIP_DTYPE_BF16: return launch_small16<DT, MLXHIP_DTYPE_BF16>(ta, tb, a, batch, s);
        default: return launch_small16<DT, MLXHIP_DTYPE_F16>(ta, tb, a, batch, s);
    }
}

}  // namespace

bool gemm16_small_fits(int64_t m, int64_t n, int64_t k, int64_t batch, int64_t lda, int64_t ldb, int ta,
                       int tb) {
    if (m <= 0 || n <= 0 || k <= 0 || k > INT32_MAX / 4 || batch <= 0 || batch > 65535) return false;
    if (ceil_div(m, TILE) * ceil_div(n, TILE) > INT32_MAX / 2) return false;
    // 32-bit buffer offsets: every slice (plus alignment slack and the 20
    // bytes a chunk reads) well below the out-of-range offset.
    const int64_t a_ext = ((ta ? k : m) - 1) * lda + (ta ? m : k) + 2;
    const int64_t b_ext = ((tb ? n : k) - 1) * ldb + (tb ? k : n) + 2;
    return a_ext * 2 + 64 < (int64_t)OOB_OFF && b_ext * 2 + 64 < (int64_t)OOB_OFF;
}

int gemm16_small(int ab_dtype, int c_dtype, int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch,
                 const void* a, int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, void* c,
                 int64_t ldc, int64_t sc, hipStream_t s) {
    if (!gemm16_small_fits(m, n, k, batch, lda, ldb, ta, tb))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm16_small: %lld x %lld x %lld (batch %lld) out of range",
                    (long long)m, (long long)n, (long long)k, (long long)batch);
    if (reinterpret_cast<uintptr_t>(a) % 2 || reinterpret_cast<uintptr_t>(b) % 2 ||
        reinterpret_cast<uintptr_t>(c) % (c_dtype == MLXHIP_DTYPE_F32 ? 4 : 2))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm16_small: operands must be element-aligned");
    Small16Args g{m, n, k, a, lda, batch > 1 ? sa : 0, b, ldb, batch > 1 ? sb : 0, c, ldc, batch > 1 ? sc : 0,
                  (int)ceil_div(n, TILE)};
    return ab_dtype == MLXHIP_DTYPE_BF16 ? dispatch_ct<MLXHIP_DTYPE_BF16>(c_dtype, ta, tb, g, batch, s)
                                         : dispatch_ct<MLXHIP_DTYPE_F16>(c_dtype, ta, tb, g, batch, s);
}

}  // namespace mlxhip
