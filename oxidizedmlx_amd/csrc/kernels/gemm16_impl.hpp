// gemm16_impl.hpp — MFMA GEMM for 16-bit operands (bf16 / f16) on gfx950,
// fed by direct global->LDS loads.
//
// C_b[M,N] = op(A_b) * op(B_b), row-major, f32 accumulation; replaces matmul
// (crates/mlx-core/src/cpu_kernels.rs:197-230) for the bf16/f16 GEMMs of the
// hot path (plain, batched, and the NT/TN forms autograd's MatMul VJP
// produces, crates/mlx-autograd/src/vjp.rs:71-80).
//
// Work decomposition (Cfg below; two configurations are instantiated)
//   * CfgLarge: block tile 256 x 256, 512 threads = 8 wave64s in a 2 x 4
//     grid, each wave owning 128 x 64 = 4 x 2 tiles of
//     v_mfma_f32_32x32x16_{bf16,f16} (128 f32 accumulators per lane), two
//     waves per SIMD so one wave's LDS traffic overlaps the other's MFMAs.
//   * CfgMid: block tile 128 x 128, 4 waves of 64 x 64, two workgroups per
//     CU, for problems with too few 256 x 256 tiles to occupy 256 CUs.
//   * K tile 32 (two MFMA k-steps of 16).
//   * Operand tiles move HBM -> LDS with buffer_load_dwordx4 ... lds: each
//     wave instruction writes 1 KiB of LDS at (base + 16 * lane), no VGPR
//     staging. The swizzles below are applied by choosing which global
//     16-byte chunk each lane fetches.
//   * STAGES LDS stages (32 KiB each for 256 x 256); the loads for tile
//     kt+STAGES are issued as soon as tile kt's stage is released, so each
//     load has STAGES-1 K tiles of MFMA work to land. One barrier per K tile,
//     placed between the two MFMA batches of the tile (one per k-step) so
//     the matrix pipe never drains.
//   * Out-of-range 16-byte chunks (M/N/K edges, and the tiles the pipeline
//     requests past the end of K) are loaded with a buffer offset beyond the
//     descriptor's range; the hardware returns zeros for them without a
//     memory access.
//
// LDS layouts (per stage, per operand: R rows or columns of the block tile)
//   K-contiguous operand ([rows][K] in HBM: A when not transposed, B when
//   transposed): R rows x 64 bytes; logical chunk c (8 k-values) of row r
//   sits at physical chunk c ^ ((r >> 2) & 3). Fragment reads are
//   ds_read_b128 (lane = row, 8 consecutive k); 16 consecutive rows hit 16
//   distinct 16-byte bank groups.
//   MN-contiguous operand ([K][cols] in HBM): 32 k-rows x 2R bytes; logical
//   chunk q of k-row k sits at q ^ ((k & 3) << 2). Fragment reads are
//   ds_read_b64_tr_b16: within each 16-lane group, output lane i element e is
//   source lane (4e + i/4)'s element (i % 4). Source lane t of group g points
//   at k = k0 + 8*(g/2) + t/4, column c0 + 16*(g%2) + 4*(t%4), so lane l
//   receives column c0 + l%32 at k0 + 8*(l/32) + {0..3}; two reads give the
//   8 consecutive k an MFMA operand lane needs. 32 lanes touch 4 k-rows x 64
//   bytes, spread over 16 bank groups by the swizzle (R >= 128 so that a
//   k-row holds the 16 chunks the swizzle permutes).
//
// MFMA operand roles are swapped (src_a = B fragment, src_b = A fragment):
// the accumulator then holds C^T, so lane l owns C[m][n .. n+3] for
// m = l % 32 and 4 consecutive n, and the epilogue stores 4 elements at once.
#pragma once

#include "../common.hpp"

namespace mlxhip {
namespace gemm16 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
#define MLXHIP_LDS __attribute__((address_space(3)))

constexpr int BK = 32;
constexpr uint32_t OOB = 0xFFFFFF00u;     // beyond every descriptor range
constexpr int BUF_FLAGS = 0x00020000;     // gfx9 buffer descriptor word 3 (32-bit data format)

// Block configuration: WM x WN waves, each owning TM x TN 32x32 MFMA tiles;
// STAGES LDS stages; WPE waves per SIMD the kernel is compiled for (bounds
// the registers per wave: 512 / WPE).
template <int WM_, int WN_, int TM_, int TN_, int STAGES_, int WPE_>
struct Cfg {
    static constexpr int WM = WM_, WN = WN_, TM = TM_, TN = TN_, STAGES = STAGES_, WPE = WPE_;
    static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES;
    static constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;  // one stage
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LA = A_BYTES / (THREADS * 16), LB = B_BYTES / (THREADS * 16);  // loads per thread
    static_assert(BM >= 128 && BN >= 128, "MN-contiguous LDS rows need >= 16 chunks for the swizzle");
    static_assert(LA * THREADS * 16 == A_BYTES && LB * THREADS * 16 == B_BYTES, "whole 1 KiB blocks per wave");
    static_assert(STAGES >= 3 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS budget");
};

// 256 x 256 block, 8 waves of 128 x 64 (two waves per SIMD): large problems.
using CfgLarge = Cfg<2, 4, 4, 2, 4, 2>;
// 128 x 128 block, 4 waves of 64 x 64 (two workgroups per CU): problems
// with too few 256 x 256 tiles to occupy the chip.
using CfgMid = Cfg<2, 2, 2, 2, 4, 2>;
// 256 x 128 block, 8 waves of 64 x 64 (two waves per SIMD): one workgroup
// per CU for problems with 256 such tiles.
using CfgWide = Cfg<4, 2, 2, 2, 4, 2>;

struct Args {
    int64_t m, n, k;
    const void* a;
    int64_t lda, sa;
    const void* b;
    int64_t ldb, sb;
    void* c;
    int64_t ldc, sc;
    uint32_t a_bytes, b_bytes;  // byte extent of one batch slice (descriptor range)
    int tiles_m, tiles_n;
    // Split-K (splits > 1): gridDim.y = batch * splits; split s of batch b
    // covers k in [s * k_chunk, min(k, (s + 1) * k_chunk)) and writes its
    // f32 partial to c + (b * splits + s) * sc (the kernel is instantiated
    // with an f32 C; c / ldc / sc describe the workspace); a second kernel
    // sums the partials in split order.
    int splits = 1;
    int64_t k_chunk = 0;
    // Split-f32 mode (kernel template X6): a and b each hold three bf16
    // planes (hi, mid, lo with hi + mid + lo == the f32 value) plane_a /
    // plane_b bytes apart, in the layout a plain bf16 operand would have;
    // k is the (padded) K of one plane. The product runs over 6 k segments,
    // one per plane pair (see seg_plane_a / seg_plane_b); k_chunk and the
    // split ranges count k over those 6 segments. When *flag == gen the
    // split found a value that is not finite (or rounds out of range) and
    // the kernel instead forms C from the f32 operands fa / fb directly
    // (flag_a / gen_a: A's split, flag_b / gen_b: B's).
    uint32_t plane_a = 0, plane_b = 0;
    const float* fa = nullptr;
    const float* fb = nullptr;
    int64_t flda = 0, fsa = 0, fldb = 0, fsb = 0, fk = 0;
    const uint32_t* flag_a = nullptr;
    const uint32_t* flag_b = nullptr;
    uint32_t gen_a = 0, gen_b = 0;
    // Split-f32 mode, interleaved kernel, one split: bias[n] is added to
    // every element of C's column n as it is stored (the row-broadcast bias
    // of a linear layer; nullptr: none).
    const float* bias = nullptr;
    // Grouped products (interleaved split-f32 kernel only, one split): with
    // groups > 0, batch index b runs product grp[b] of the same shapes and
    // layouts, its planes, C and f32 operands at the pointers given here
    // instead of base + b * stride.
    struct Group {
        const void* a;
        const void* b;
        void* c;
        const float* fa;
        const float* fb;
        const uint32_t* flag_a;
        const uint32_t* flag_b;
        uint32_t gen_a, gen_b;
        const float* bias;
    };
    static constexpr int MAX_GROUPS = 4;
    int groups = 0;
    Group grp[MAX_GROUPS] = {};
};

// Group b of a grouped launch, read with constant offsets (a run-time index
// into the kernel arguments would copy them to scratch).
__device__ inline Args::Group group_of(const Args& g, int b) {
    switch (b) {
        case 0: return g.grp[0];
        case 1: return g.grp[1];
        case 2: return g.grp[2];
        default: return g.grp[3];
    }
}

// Plane pairs of the 6 k segments, smallest products first so the f32
// accumulators add the large hi*hi terms last: (mid, mid), (lo, hi),
// (hi, lo), (mid, hi), (hi, mid), (hi, hi); plane 0 = hi, 1 = mid, 2 = lo.
// With the planes rounded to nearest, |mid| <= 2^-8 |x| and |lo| <= 2^-16 |x|,
// so the three dropped pairs (mid*lo, lo*mid, lo*lo) add up to at most about
// 2^-23 of |a b| (one f32 rounding of the product is 2^-24 of it).
__host__ __device__ constexpr int seg_plane_a(int seg) { return (0x001021 >> (4 * seg)) & 3; }
__host__ __device__ constexpr int seg_plane_b(int seg) { return (0x010201 >> (4 * seg)) & 3; }
constexpr int X6_SEGS = 6;

// Position of the next K tile in split-f32 mode: segment, k inside it, and
// how many tiles of the workgroup's range are left (this one included).
struct SegCursor {
    int seg, kin, left;
    __device__ inline void init(int64_t vtile0, int tiles_per_seg, int ntiles) {
        seg = (int)(vtile0 / tiles_per_seg);
        kin = (int)(vtile0 - (int64_t)seg * tiles_per_seg) * BK;
        left = ntiles;
    }
    __device__ inline void next(int seg_k) {
        kin += BK;
        if (kin >= seg_k) {
            kin = 0;
            ++seg;
        }
        --left;
    }
    // k to hand the loaders: past the range, one no chunk accepts.
    __device__ inline int k() const { return left > 0 ? kin : INT32_MAX; }
    __device__ inline uint32_t base_a(uint32_t plane) const {
        return left > 0 ? (uint32_t)seg_plane_a(seg) * plane : 0u;
    }
    __device__ inline uint32_t base_b(uint32_t plane) const {
        return left > 0 ? (uint32_t)seg_plane_b(seg) * plane : 0u;
    }
};

template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// All LDS reads of this wave done, then a workgroup barrier. No wait on
// vector-memory loads: in-flight LDS-bound loads stay in flight. The wait is
// the compiler's own s_waitcnt (0xC07F = lgkmcnt(0), vmcnt/expcnt at their
// maxima), so its wait-count bookkeeping knows every LDS read has completed;
// the empty asm statements keep memory accesses on their side of the barrier.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 16 bytes per lane from buffer offset `voff` into LDS at dst + 16 * lane.
// Issued as inline assembly on purpose: the compiler cannot tell which LDS
// bytes an LDS-bound load writes, so for its own builtin it waits for every
// such load to finish before any later LDS read, which would serialise the
// pipeline. The kernel orders these loads itself (wait_vmcnt + barrier).
__device__ inline void lds_load16(__amdgpu_buffer_rsrc_t rsrc, MLXHIP_LDS char* dst, uint32_t voff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(m0) : "memory");
}

// One operand's global->LDS loader for a block tile of ROWS rows (KC) or
// columns (!KC). KC: operand is K-contiguous in HBM. Each wave instruction
// fills one 1 KiB block of the operand's stage; block q = i * WAVES + wave.
template <bool KC, int ROWS, int WAVES>
struct Loader {
    static constexpr int L = ROWS * BK * 2 / (WAVES * 1024);  // loads per thread per K tile
    static constexpr int ROWB = ROWS * 2;                     // !KC: bytes per k-row
    static constexpr int CPR = ROWB / 16;                     // !KC: 16-byte chunks per k-row
    uint32_t off[L];          // byte offset of the chunk for k0 = 0
    int lim[L];               // the chunk is in range iff k0 < lim (INT_MIN: never)
    uint32_t k_stride_bytes;  // bytes per unit of k (KC: 2, !KC: 2 * ld)

    // rows0: first tile row (KC) / column (!KC); R: valid rows / columns.
    __device__ inline void init(int tid, int64_t rows0, int64_t R, int64_t ld, int64_t K) {
        const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int q = i * WAVES + wave;
            if constexpr (KC) {
                // 16 rows x 64 bytes per block.
                const int r = 16 * q + (lane >> 2);
                const int c = (lane & 3) ^ ((r >> 2) & 3);
                const int64_t row = rows0 + r;
                const bool ok = row < R;
                off[i] = ok ? (uint32_t)((row * ld + 8 * c) * 2) : 0u;
                lim[i] = ok ? (int)(K - 8 * c) : INT32_MIN;
            } else {
                // 64 / CPR k-rows x ROWB bytes per block.
                const int kr = (64 / CPR) * q + lane / CPR;
                const int cc = (lane % CPR) ^ ((kr & 3) << 2);
                const int64_t col = rows0 + 8 * cc;
                const bool ok = col < R;
                off[i] = ok ? (uint32_t)((kr * ld + col) * 2) : 0u;
                lim[i] = ok ? (int)(K - kr) : INT32_MIN;
            }
        }
        k_stride_bytes = KC ? 2u : (uint32_t)(ld * 2);
    }

    // Load i (0 .. L-1) of the tile starting at k0.
    // `base`: byte offset added to every in-range chunk (split-f32 mode:
    // the plane of the tile's segment).
    __device__ inline void issue_one(__amdgpu_buffer_rsrc_t rsrc, MLXHIP_LDS char* stage_op, int wave,
                                     int k0, int i, uint32_t base = 0) const {
        const uint32_t v = k0 < lim[i] ? off[i] + base + (uint32_t)k0 * k_stride_bytes : OOB;
        lds_load16(rsrc, stage_op + (i * WAVES + wave) * 1024, v);
    }

    __device__ inline void issue(__amdgpu_buffer_rsrc_t rsrc, MLXHIP_LDS char* stage_op, int wave,
                                 int k0, uint32_t base = 0) const {
#pragma unroll
        for (int i = 0; i < L; ++i) issue_one(rsrc, stage_op, wave, k0, i, base);
    }
};

// Per-lane LDS byte offsets of one wave's T fragments (32 rows / columns
// each) of one operand inside a stage; ROWB: bytes per k-row (!KC).
//   KC : off(x, s) = base_s + x * 2048            (x: 32-row block, s: k-step)
//   !KC: off(x, s, r) = base_x[x] + (16 s + 4 r) * ROWB
template <bool KC, int T, int ROWB>
struct FragAddr {
    uint32_t base[KC ? 2 : T];
    __device__ inline void init(int lane, int wave_off /* first row / column of the wave */) {
        if constexpr (KC) {
            const int r = lane & 31;
            const int sw = (r >> 2) & 3;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int c = 2 * s + (lane >> 5);
                base[s] = (uint32_t)((wave_off + r) * 64 + ((c ^ sw) * 16));
            }
        } else {
            const int g = lane >> 4, t = lane & 15;
            const int krow = 8 * (g >> 1) + (t >> 2);  // krow & 3 == (t >> 2) & 3
#pragma unroll
            for (int x = 0; x < T; ++x) {
                const int logical = (wave_off >> 3) + 4 * x + 2 * (g & 1) + ((t >> 1) & 1);
                const int chunk = logical ^ ((t >> 2) << 2);
                base[x] = (uint32_t)(krow * ROWB + chunk * 16 + (t & 1) * 8);
            }
        }
    }
};

template <int DT>
__device__ inline void mfma(const u32x4& a, const u32x4& b, f32x16& acc) {
    if constexpr (DT == MLXHIP_DTYPE_BF16)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    else
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}

// Read `idx` of one operand's T fragments for k-step s: KC: fragment idx
// (ds_read_b128, T reads); !KC: half idx % 2 of fragment idx / 2
// (ds_read_b64_tr_b16, k offsets 0-3 or 4-7; 2T reads).
template <bool KC, int T, int ROWB>
__device__ inline void read_one(const MLXHIP_LDS char* op, const FragAddr<KC, T, ROWB>& fa, int s, int idx,
                                u32x4* f) {
    if constexpr (KC) {
        f[idx] = *(const MLXHIP_LDS u32x4*)(op + fa.base[s] + idx * 2048);
    } else {
        const int x = idx >> 1, r = idx & 1;
        const MLXHIP_LDS char* p = op + fa.base[x] + (16 * s + 4 * r) * ROWB;
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((MLXHIP_LDS i16x4*)p));
        if (r == 0) {
            f[x].x = v.x;
            f[x].y = v.y;
        } else {
            f[x].z = v.x;
            f[x].w = v.y;
        }
    }
}

// All T fragments of one operand for k-step s of the stage at `op`.
template <bool KC, int T, int ROWB>
__device__ inline void read_frags(const MLXHIP_LDS char* op, const FragAddr<KC, T, ROWB>& fa, int s, u32x4* f) {
#pragma unroll
    for (int idx = 0; idx < (KC ? T : 2 * T); ++idx) read_one<KC, T, ROWB>(op, fa, s, idx, f);
}

// Two f32 -> two 16-bit outputs packed in one dword (low = first), rounded
// to nearest even: bf16 by v_cvt_pk_bf16_f32, f16 by v_cvt_f16_f32.
template <int CT>
__device__ inline uint32_t pack2(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    if constexpr (CT == MLXHIP_DTYPE_BF16) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    } else {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
    }
}

// Epilogue staging: rows of one wave's sub-tile converted per pass, the
// largest power-of-two multiple of 32 (at most the wave's rows) whose
// padded rows for all waves fit in `budget` bytes of LDS.
template <class C, int ES>
constexpr int pass_rows(int budget) {
    int r = 32 * C::TM;
    while (r > 32 && C::WAVES * r * (32 * C::TN * ES + 16) > budget) r /= 2;
    return r;
}

// The workgroup's C tile. XCD-aware order over the whole grid (every tile
// of every batch slice): the hardware hands consecutive workgroup ids (x
// fastest) to the 8 XCDs round-robin; give each XCD a contiguous range of
// (slice, tile) ids so the tiles of a slice share one L2, then order a
// slice's tiles in groups of 4 tile rows so neighbours share A rows / B
// columns.
struct TileId {
    int64_t slice, batch, split;  // slice = batch * splits + split
    int64_t m0, n0;
};
template <class C>
__device__ inline TileId tile_of(const Args& g) {
    const int nwg = g.tiles_m * g.tiles_n;
    const int64_t total = (int64_t)nwg * gridDim.y;
    int64_t lin = (int64_t)blockIdx.y * nwg + blockIdx.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    TileId t;
    t.slice = lin / nwg;
    const int id = (int)(lin - t.slice * nwg);
    t.batch = t.slice / g.splits;
    t.split = t.slice - t.batch * g.splits;
    constexpr int GROUP_M = 4;
    const int in_group = GROUP_M * g.tiles_n;
    const int first_m = (id / in_group) * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int tm = first_m + (id % in_group) % gsz;
    const int tn = (id % in_group) / gsz;
    t.m0 = (int64_t)tm * C::BM;
    t.n0 = (int64_t)tn * C::BN;
    return t;
}

// Epilogue of the kernels below (C tile of one workgroup, after its last
// MFMA), through the first bytes of the operand stages' LDS.
template <int CT, class C, int PIPE_BYTES, bool NT = true>
__device__ inline void store_c(const Args& g, const f32x16 (&acc)[C::TM][C::TN], MLXHIP_LDS char* smem, char* Cp,
                               int64_t m0, int64_t n0, int wave, int lane, const float* bias = nullptr) {
    // Through LDS. acc[i][j][v] = C[m][n] with m = WR wm + 32 i +
    // lane % 32 and n = WC wn + 32 j + 8 (v / 4) + 4 (lane / 32) + v % 4
    // inside the tile (WR x WC: the wave's sub-tile). Each wave converts its
    // sub-tile into padded LDS rows (PITCH = row bytes + 16: consecutive rows
    // fall in distinct bank groups for the 8/16-byte writes) and reads it
    // back row by row, so every global store instruction writes whole row
    // segments instead of 16-byte pieces of 32 rows. With NT the row
    // segments are stored non-temporally (C is written once, so it streams
    // out instead of filling the L2s that later tiles' operands need);
    // otherwise as plain write-back stores.
    constexpr int TM = C::TM, TN = C::TN;
    constexpr int ES = CT == MLXHIP_DTYPE_F32 ? 4 : 2;
    constexpr int PASS_ROWS = pass_rows<C, ES>(PIPE_BYTES);
    constexpr int ROW_BYTES = 32 * TN * ES;  // one wave sub-tile row
    constexpr int PITCH = ROW_BYTES + 16;
    const int wm = wave / C::WN, wn = wave % C::WN;
    wait_vmcnt<0>();
    lds_barrier();  // every wave is done with the operand stages
    constexpr int LANES_PER_ROW = ROW_BYTES / 16;
    constexpr int ROWS_PER_READ = 64 / LANES_PER_ROW;
    static_assert(LANES_PER_ROW <= 64 && 64 % LANES_PER_ROW == 0, "epilogue read shape");
    MLXHIP_LDS char* region = smem + wave * PASS_ROWS * PITCH;
    const int64_t row0 = m0 + 32 * TM * wm, col0 = n0 + 32 * TN * wn;
    const bool vec_ok = (g.ldc * ES) % 16 == 0 && (reinterpret_cast<uintptr_t>(Cp) % 16) == 0;
    // A lane stores the same 16-byte column range of every row it stores:
    // its four bias values are loaded once, before the first store.
    float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (ES == 4) {
        if (bias) {
            const int64_t nb = col0 + ((lane % LANES_PER_ROW) * 16) / ES;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (nb + e < g.n) bv[e] = bias[nb + e];
        }
    }
#pragma unroll
    for (int pass = 0; pass < 32 * TM / PASS_ROWS; ++pass) {
#pragma unroll
        for (int i = 0; i < PASS_ROWS / 32; ++i) {
            const int ii = pass * (PASS_ROWS / 32) + i;
            const int r = 32 * i + (lane & 31);
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = 32 * j + 8 * q + 4 * (lane >> 5);
                    MLXHIP_LDS char* p = region + r * PITCH + c * ES;
                    const f32x16& a = acc[ii][j];
                    if constexpr (ES == 4) {
                        *(MLXHIP_LDS f32x4*)p = f32x4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
                    } else {
                        *(MLXHIP_LDS u32x2*)p =
                            u32x2{pack2<CT>(a[4 * q], a[4 * q + 1]), pack2<CT>(a[4 * q + 2], a[4 * q + 3])};
                    }
                }
        }
        // The staged rows are read back by the same wave: LDS accesses of one
        // wave complete in order, so no barrier is needed.
#pragma unroll 4
        for (int rr = 0; rr < PASS_ROWS; rr += ROWS_PER_READ) {
            const int r = rr + lane / LANES_PER_ROW;
            const int cb = (lane % LANES_PER_ROW) * 16;  // byte offset inside the row
            u32x4 v = *(const MLXHIP_LDS u32x4*)(region + r * PITCH + cb);
            const int64_t m = row0 + pass * PASS_ROWS + r;
            const int64_t n = col0 + cb / ES;
            if (m >= g.m || n >= g.n) continue;
            if constexpr (ES == 4) {
                // The bias term: the f32 value of C, then one f32 addition,
                // as a separate elementwise Add would give.
                if (bias) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = __float_as_uint(__uint_as_float(v[e]) + bv[e]);
                }
            }
            char* dst = Cp + (m * g.ldc + n) * ES;
            if (vec_ok && n + 16 / ES <= g.n) {
                if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
                else *reinterpret_cast<u32x4*>(dst) = v;
            } else {
                // Row end or unaligned C: element stores.
#pragma unroll
                for (int e = 0; e < 16 / ES; ++e) {
                    if (n + e >= g.n) break;
                    const uint32_t w = v[(e * ES) / 4];
                    if constexpr (ES == 4) reinterpret_cast<uint32_t*>(dst)[e] = w;
                    else reinterpret_cast<uint16_t*>(dst)[e] = (uint16_t)(w >> (16 * (e & 1)));
                }
            }
        }
    }
}

// LDS bytes the epilogue stages (it reuses the operand stages' LDS).
template <int CT, class C, int PIPE_BYTES>
constexpr int epi_bytes() {
    constexpr int ES = CT == MLXHIP_DTYPE_F32 ? 4 : 2;
    return C::WAVES * pass_rows<C, ES>(PIPE_BYTES) * (32 * C::TN * ES + 16);
}

// Split-f32 mode, inputs flagged as not finite: the workgroup's tile of C
// (f32) straight from the f32 operands, one FMA chain per element over the
// whole K, so infinities and NaNs combine as in an f32 product. Split 0 of a
// split-K launch holds the product, the other splits zeros.
template <int TA, int TB, class C>
__device__ void x6_direct(const Args& g, const float* A, const float* B, float* Cp, int64_t split, int64_t m0,
                          int64_t n0, int tid, const float* bias = nullptr) {
    for (int e = tid; e < C::BM * C::BN; e += C::THREADS) {
        const int64_t m = m0 + e / C::BN, n = n0 + e % C::BN;
        if (m >= g.m || n >= g.n) continue;
        float acc = 0.0f;
        if (split == 0)
            for (int64_t k = 0; k < g.fk; ++k)
                acc = fmaf(TA ? A[k * g.flda + m] : A[m * g.flda + k], TB ? B[n * g.fldb + k] : B[k * g.fldb + n],
                           acc);
        Cp[m * g.ldc + n] = bias ? acc + bias[n] : acc;
    }
}

template <int DT, int CT, int TA, int TB, class C, bool SPREAD, bool X6 = false, bool NTC = true>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(C::WPE, C::WPE)))
void gemm16_kernel(Args g) {
    static_assert(!X6 || (DT == MLXHIP_DTYPE_BF16 && CT == MLXHIP_DTYPE_F32), "split-f32 mode: bf16 planes, f32 C");
    constexpr bool KCA = (TA == 0);  // A stored [M][K]
    constexpr bool KCB = (TB == 1);  // B stored [N][K]
    constexpr int STAGES = C::STAGES, TM = C::TM, TN = C::TN, WAVES = C::WAVES;
    constexpr int PIPE_BYTES = STAGES * C::STAGE_BYTES;
    constexpr int EPI_BYTES = epi_bytes<CT, C, PIPE_BYTES>();
    constexpr int SMEM_BYTES = PIPE_BYTES > EPI_BYTES ? PIPE_BYTES : EPI_BYTES;
    __shared__ __attribute__((aligned(1024))) char smem_raw[SMEM_BYTES];
    MLXHIP_LDS char* smem = (MLXHIP_LDS char*)smem_raw;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WN, wn = wave % C::WN;

    const TileId tl = tile_of<C>(g);
    const int64_t slice = tl.slice, batch = tl.batch, split = tl.split, m0 = tl.m0, n0 = tl.n0;

    if constexpr (X6) {
        if (__atomic_load_n(g.flag_a, __ATOMIC_RELAXED) == g.gen_a ||
            __atomic_load_n(g.flag_b, __ATOMIC_RELAXED) == g.gen_b) {
            x6_direct<TA, TB, C>(g, g.fa + batch * g.fsa, g.fb + batch * g.fsb, static_cast<float*>(g.c) + slice * g.sc,
                                 split, m0, n0, tid);
            return;
        }
    }

    // A split starts k_chunk * split into K: its operands are the slices'
    // sub-matrices from that k on (descriptor ranges shortened to match).
    // Split-f32 mode: K counts over the 6 segments; the tiles find their
    // segment's planes through a SegCursor and the descriptors start at the
    // slice.
    const int64_t kb = split * g.k_chunk;
    const int64_t kv = X6 ? X6_SEGS * g.k : g.k;
    const int64_t klen = g.splits > 1 ? min(kv - kb, g.k_chunk) : kv;
    const int64_t a_koff = X6 ? 0 : (KCA ? kb : kb * g.lda) * 2, b_koff = X6 ? 0 : (KCB ? kb : kb * g.ldb) * 2;
    const char* A = static_cast<const char*>(g.a) + batch * g.sa * 2 + a_koff;
    const char* B = static_cast<const char*>(g.b) + batch * g.sb * 2 + b_koff;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)(g.a_bytes - (uint32_t)a_koff), BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)(g.b_bytes - (uint32_t)b_koff), BUF_FLAGS);

    constexpr int ROWB_A = C::BM * 2, ROWB_B = C::BN * 2;
    Loader<KCA, C::BM, WAVES> la;
    Loader<KCB, C::BN, WAVES> lb;
    la.init(tid, m0, g.m, g.lda, X6 ? g.k : klen);
    lb.init(tid, n0, g.n, g.ldb, X6 ? g.k : klen);
    FragAddr<KCA, TM, ROWB_A> fa;
    FragAddr<KCB, TN, ROWB_B> fb;
    fa.init(lane, 32 * TM * wm);
    fb.init(lane, 32 * TN * wn);

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int nk = (int)((klen + BK - 1) / BK);
    constexpr int LA = C::LA, LB = C::LB, LPT = LA + LB;
    constexpr int B_OFF = C::A_BYTES;  // stage layout: A block, then B block

    // Prologue: tiles 0 .. STAGES-1 into stages 0 .. STAGES-1.
    // With SPREAD, B's loads of tile t+STAGES are issued in the first half of
    // iteration t+1 instead (spread over its MFMAs) and the prologue leaves
    // out B of tile STAGES-1; the count of loads younger than any tile is
    // unchanged.
    // Split-f32 mode: ca walks the tiles A (and, without SPREAD, B) loads
    // next, cb the tiles of B's spread loads (one tile behind).
    SegCursor ca{}, cb{};
    const int seg_k = (int)g.k;
    if constexpr (X6) ca.init(kb / BK, seg_k / BK, nk);
#pragma unroll
    for (int t = 0; t < STAGES; ++t) {
        MLXHIP_LDS char* st = smem + t * C::STAGE_BYTES;
        if constexpr (X6) {
            if (t == STAGES - 1) cb = ca;
            la.issue(ra, st, wave, ca.k(), ca.base_a(g.plane_a));
            if (!SPREAD || t < STAGES - 1) lb.issue(rb, st + B_OFF, wave, ca.k(), ca.base_b(g.plane_b));
            ca.next(seg_k);
        } else {
            la.issue(ra, st, wave, t * BK);
            if (!SPREAD || t < STAGES - 1) lb.issue(rb, st + B_OFF, wave, t * BK);
        }
    }
    if constexpr (SPREAD) wait_vmcnt<(STAGES - 2) * LPT + LA>();
    else wait_vmcnt<(STAGES - 1) * LPT>();
    lds_barrier();

    u32x4 af[2][TM], bf[2][TN];
    read_frags<KCA, TM, ROWB_A>(smem, fa, 0, af[0]);
    read_frags<KCB, TN, ROWB_B>(smem + B_OFF, fb, 0, bf[0]);

    // Each half-tile issues NM MFMAs with the LDS reads / LDS-bound loads of
    // the next half placed between them; the scheduling barriers keep that
    // order (the compiler would otherwise sink each read next to its first
    // use and expose the LDS latency).
    constexpr int NM = TM * TN;
    constexpr int NA = KCA ? TM : 2 * TM, NB = KCB ? TN : 2 * TN, NR = NA + NB;
    constexpr int OPS2 = NR + LA + (SPREAD ? 0 : LB);
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt % STAGES;
        const MLXHIP_LDS char* st = smem + cur * C::STAGE_BYTES;
        MLXHIP_LDS char* spread_dst = smem + ((kt + STAGES - 1) % STAGES) * C::STAGE_BYTES + B_OFF;
        // k and plane offsets of the loads of this iteration: B's spread
        // loads (tile kt-1+STAGES), then A's and B's (tile kt+STAGES).
        const int k_sp = X6 ? cb.k() : (kt - 1 + STAGES) * BK;
        const uint32_t base_sp = X6 ? cb.base_b(g.plane_b) : 0u;
        const int k_ld = X6 ? ca.k() : (kt + STAGES) * BK;
        const uint32_t base_la = X6 ? ca.base_a(g.plane_a) : 0u, base_lb = X6 ? ca.base_b(g.plane_b) : 0u;
        if constexpr (X6) {
            cb.next(seg_k);
            ca.next(seg_k);
        }
        // First half: MFMAs of k-step 0, reads of k-step 1 of this tile.
#pragma unroll
        for (int q = 0; q < NM; ++q) {
            mfma<DT>(bf[0][q % TN], af[0][q / TN], acc[q / TN][q % TN]);
#pragma unroll
            for (int o = NR <= NM ? q : (q * NR) / NM; o < (NR <= NM ? q + 1 : ((q + 1) * NR) / NM); ++o) {
                if (o < NA) read_one<KCA, TM, ROWB_A>(st, fa, 1, o, af[1]);
                else if (o < NR) read_one<KCB, TN, ROWB_B>(st + B_OFF, fb, 1, o - NA, bf[1]);
            }
            if constexpr (SPREAD) {
                // B of tile kt-1+STAGES into the stage released in iteration kt-1.
                if (((q + 1) * LB) / NM > (q * LB) / NM)
                    lb.issue_one(rb, spread_dst, wave, k_sp, (q * LB) / NM, base_sp);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // Tile kt+1 has landed for every wave; every wave is done reading
        // this tile's stage, which then receives tile kt+STAGES.
        wait_vmcnt<(STAGES - 2) * LPT>();
        lds_barrier();
        MLXHIP_LDS char* dst = smem + cur * C::STAGE_BYTES;
        const MLXHIP_LDS char* nx = smem + ((kt + 1) % STAGES) * C::STAGE_BYTES;
        // Second half: MFMAs of k-step 1; the k-step 0 reads of tile kt+1
        // and the loads of tile kt+STAGES.
#pragma unroll
        for (int q = 0; q < NM; ++q) {
            mfma<DT>(bf[1][q % TN], af[1][q / TN], acc[q / TN][q % TN]);
#pragma unroll
            for (int o = (q * OPS2) / NM; o < ((q + 1) * OPS2) / NM; ++o) {
                // Reads first: the next tile's first MFMAs consume them.
                if (o < NA) read_one<KCA, TM, ROWB_A>(nx, fa, 0, o, af[0]);
                else if (o < NR) read_one<KCB, TN, ROWB_B>(nx + B_OFF, fb, 0, o - NA, bf[0]);
                else if (o < NR + LA) la.issue_one(ra, dst, wave, k_ld, o - NR, base_la);
                else if (!SPREAD) lb.issue_one(rb, dst + B_OFF, wave, k_ld, o - NR - LA, base_lb);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    store_c<CT, C, PIPE_BYTES, NTC>(g, acc, smem, static_cast<char*>(g.c) + slice * g.sc * (CT == MLXHIP_DTYPE_F32 ? 4 : 2),
                               m0, n0, wave, lane);
}

// Host-side check of what the kernel assumes about its operands; returns
// false when the general GEMM must run instead. `padded`: every row of both
// operands may be read up to its leading dimension (the zero-padded copies
// the dispatcher makes of unaligned operands); then an M or N extent need not
// be a multiple of 8 (the chunk that crosses it only feeds rows / columns of
// C that are never stored). K extents must be, in any case: a chunk crossing
// K would multiply what lies past it.
inline bool supported(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const void* a,
                      int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, uint32_t* a_bytes,
                      uint32_t* b_bytes, bool padded = false) {
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(b) % 16) return false;
    if (k >= (1 << 30)) return false;  // k offsets are 32-bit in the kernel
    if (lda % 8 || ldb % 8) return false;
    if (batch > 1 && (sa % 8 || sb % 8)) return false;
    // The contiguous extent of each operand must hold whole 16-byte chunks.
    if ((ta == 0 ? k : m) % 8 && !(padded && ta == 1)) return false;
    if ((tb == 1 ? k : n) % 8 && !(padded && tb == 0)) return false;
    const int64_t a_rows = ta ? k : m, b_rows = tb ? n : k;
    const int64_t a_ext = ((a_rows - 1) * lda + (padded ? lda : (ta ? m : k))) * 2;
    const int64_t b_ext = ((b_rows - 1) * ldb + (padded ? ldb : (tb ? k : n))) * 2;
    const int64_t lim = (int64_t)OOB - 4096;
    if (a_ext <= 0 || b_ext <= 0 || a_ext >= lim || b_ext >= lim) return false;
    *a_bytes = (uint32_t)a_ext;
    *b_bytes = (uint32_t)b_ext;
    return true;
}

template <int DT, int CT, int TA, int TB, class C, bool X6 = false>
int launch(const Args& a0, int64_t batch, hipStream_t s) {
    Args a = a0;
    a.tiles_m = (int)ceil_div(a.m, C::BM);
    a.tiles_n = (int)ceil_div(a.n, C::BN);
    dim3 grid((unsigned)(a.tiles_m * a.tiles_n), (unsigned)(batch * a.splits));
    // A grid that runs in one round of workgroups (one per CU for the
    // 256 x 256 blocks) stores C with plain stores: nothing runs after the
    // tiles' epilogues, and write-back stores drain faster at the kernel's
    // end (4096^3 bf16: 120.0-120.3 us against 121.9-122.1 us steady state,
    // alternating on one MI355X). Later rounds' operands need the L2s, so a
    // larger grid stores non-temporally (config 3, 512 tiles: 3-4 us faster
    // per call that way).
    // (The choice is a template parameter: a run-time flag in the store
    // loop cost config 3 3-9 us per call.) Split-f32 products keep
    // non-temporal stores.
    if constexpr (!X6) {
        if ((int64_t)grid.x * grid.y <= 256) {
            hipLaunchKernelGGL((gemm16_kernel<DT, CT, TA, TB, C, true, X6, false>), grid, dim3(C::THREADS), 0, s, a);
            return launch_check("gemm16_kernel");
        }
    }
    hipLaunchKernelGGL((gemm16_kernel<DT, CT, TA, TB, C, true, X6, true>), grid, dim3(C::THREADS), 0, s, a);
    return launch_check("gemm16_kernel");
}

template <int DT, int CT, class C, bool X6 = false>
int dispatch_layout(const Args& a, int64_t batch, int ta, int tb, hipStream_t s) {
    if (!ta && !tb) return launch<DT, CT, 0, 0, C, X6>(a, batch, s);
    if (!ta && tb) return launch<DT, CT, 0, 1, C, X6>(a, batch, s);
    if (ta && !tb) return launch<DT, CT, 1, 0, C, X6>(a, batch, s);
    return launch<DT, CT, 1, 1, C, X6>(a, batch, s);
}

// cfg: 0 = CfgLarge, 1 = CfgMid, 2 = CfgWide (split-f32 mode only).
template <int DT, int CT, bool X6 = false>
int dispatch(const Args& a, int64_t batch, int ta, int tb, int cfg, hipStream_t s) {
    if (cfg == 0) return dispatch_layout<DT, CT, CfgLarge, X6>(a, batch, ta, tb, s);
    if constexpr (X6)
        if (cfg == 2) return dispatch_layout<DT, CT, CfgWide, X6>(a, batch, ta, tb, s);
    return dispatch_layout<DT, CT, CfgMid, X6>(a, batch, ta, tb, s);
}

}  // namespace gemm16

// Per-dtype entry points (gemm16_bf16.hip, gemm16_f16.hip), and the
// split-f32 mode (gemm16_x6.hip; f32 C).
int gemm16_bf16(int c_dtype, int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s);
int gemm16_f16(int c_dtype, int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s);
int gemm16_x6(int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s);

// One f32 operand's split into three bf16 planes (gemm16_x6.hip). Each plane
// is [batch][rows_p][cols_p] with zeros beyond [rows][cols], so a plane
// product over the padded extents adds nothing for them.
struct X6SplitOp {
    const float* src;
    int64_t ld, stride;      // source row pitch and batch stride (elements)
    int64_t rows, cols;      // source extent of one batch slice
    int64_t rows_p, cols_p;  // plane extent of one slice; cols_p % 8 == 0
    uint16_t* dst;           // plane 0 (16-byte aligned); plane p at dst + p * plane
    int64_t plane;           // elements per plane: batch * rows_p * cols_p
    int64_t chunks;          // plane / 8, below 2^31
    uint32_t* flag;          // receives gen if a value is not finite or its
    uint32_t gen;            // hi plane rounds out of range
};
// Up to MAX operands in one launch (gridDim.y = n).
struct X6SplitPair {
    static constexpr int MAX = 5;
    X6SplitOp op[MAX];
    int n;
};
int x6_split(const X6SplitPair& sp, hipStream_t s);

}  // namespace mlxhip
