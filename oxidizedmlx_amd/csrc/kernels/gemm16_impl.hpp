// gemm16_impl.hpp — MFMA GEMM for 16-bit operands (bf16 / f16) on gfx950,
// fed by direct global->LDS loads.
//
// C_b[M,N] = op(A_b) * op(B_b), row-major, f32 accumulation; replaces matmul
// (crates/mlx-core/src/cpu_kernels.rs:197-230) for the bf16/f16 GEMMs of the
// hot path (plain, batched, and the NT/TN forms autograd's MatMul VJP
// produces, crates/mlx-autograd/src/vjp.rs:71-80).
//
// Work decomposition
//   * Block tile 256 x 256, K tile 32; 256 threads = 4 wave64s in a 2 x 2
//     grid, each wave owning a 128 x 128 quadrant = 4 x 4 tiles of
//     v_mfma_f32_32x32x16_{bf16,f16} (256 f32 accumulators per lane).
//   * Operand tiles move HBM -> LDS with buffer_load_dwordx4 ... lds: each
//     wave instruction writes 1 KiB of LDS at (base + 16 * lane), no VGPR
//     staging. The swizzles below are applied by choosing which global
//     16-byte chunk each lane fetches.
//   * STAGES LDS stages of 32 KiB; the loads for tile kt+STAGES are issued as
//     soon as tile kt's stage is released, so each load has STAGES-1 K tiles
//     of MFMA work to land. One barrier per K tile, placed between the two
//     16-deep MFMA batches of the tile so the matrix pipe never drains.
//   * Out-of-range 16-byte chunks (M/N/K edges, and the tiles the pipeline
//     requests past the end of K) are loaded with a buffer offset beyond the
//     descriptor's range; the hardware returns zeros for them without a
//     memory access.
//
// LDS layouts (per stage, per operand, 16 KiB)
//   K-contiguous operand ([rows][K] in HBM: A when not transposed, B when
//   transposed): 256 rows x 64 bytes; logical chunk c (8 k-values) of row r
//   sits at physical chunk c ^ ((r >> 2) & 3). Fragment reads are
//   ds_read_b128 (lane = row, 8 consecutive k); 16 consecutive rows hit 16
//   distinct 16-byte bank groups.
//   MN-contiguous operand ([K][cols] in HBM): 32 k-rows x 512 bytes; logical
//   chunk q of k-row k sits at q ^ ((k & 3) << 2). Fragment reads are
//   ds_read_b64_tr_b16: within each 16-lane group, output lane i element e is
//   source lane (4e + i/4)'s element (i % 4). Source lane t of group g points
//   at k = k0 + 8*(g/2) + t/4, column c0 + 16*(g%2) + 4*(t%4), so lane l
//   receives column c0 + l%32 at k0 + 8*(l/32) + {0..3}; two reads give the
//   8 consecutive k an MFMA operand lane needs. 32 lanes touch 4 k-rows x 64
//   bytes, spread over 16 bank groups by the swizzle.
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

constexpr int TILE = 256;                 // BM = BN
constexpr int BK = 32;
constexpr int THREADS = 256;
constexpr int OP_BYTES = TILE * BK * 2;   // 16 KiB: one operand, one stage
constexpr int STAGE_BYTES = 2 * OP_BYTES;
constexpr int LOADS_PER_OP = OP_BYTES / (THREADS * 16);  // 4 per thread
constexpr uint32_t OOB = 0xFFFFFF00u;     // beyond every descriptor range
constexpr int BUF_FLAGS = 0x00020000;     // gfx9 buffer descriptor word 3 (32-bit data format)

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

// One operand's global->LDS loader. KC: operand is K-contiguous in HBM.
// Per thread it issues LOADS_PER_OP 16-byte loads per K tile.
template <bool KC>
struct Loader {
    uint32_t off[LOADS_PER_OP];  // byte offset of the chunk for k0 = 0
    int lim[LOADS_PER_OP];       // the chunk is in range iff k0 < lim (INT_MIN: never)
    uint32_t k_stride_bytes;     // bytes per unit of k (KC: 2, !KC: 2 * ld)

    // rows0: first tile row (KC) / column (!KC); R: valid rows / columns.
    __device__ inline void init(int tid, int64_t rows0, int64_t R, int64_t ld, int64_t K) {
        const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
        for (int i = 0; i < LOADS_PER_OP; ++i) {
            const int q = i * 4 + wave;  // 1 KiB block of the operand's stage
            if constexpr (KC) {
                const int r = 16 * q + (lane >> 2);
                const int c = (lane & 3) ^ ((r >> 2) & 3);
                const int64_t row = rows0 + r;
                const bool ok = row < R;
                off[i] = ok ? (uint32_t)((row * ld + 8 * c) * 2) : 0u;
                lim[i] = ok ? (int)(K - 8 * c) : INT32_MIN;
            } else {
                const int kr = 2 * q + (lane >> 5);
                const int cc = (lane & 31) ^ ((kr & 3) << 2);
                const int64_t col = rows0 + 8 * cc;
                const bool ok = col < R;
                off[i] = ok ? (uint32_t)((kr * ld + col) * 2) : 0u;
                lim[i] = ok ? (int)(K - kr) : INT32_MIN;
            }
        }
        k_stride_bytes = KC ? 2u : (uint32_t)(ld * 2);
    }

    // Load i (0 .. LOADS_PER_OP-1) of the tile starting at k0.
    __device__ inline void issue_one(__amdgpu_buffer_rsrc_t rsrc, MLXHIP_LDS char* stage_op, int wave,
                                     int k0, int i) const {
        const uint32_t v = k0 < lim[i] ? off[i] + (uint32_t)k0 * k_stride_bytes : OOB;
        lds_load16(rsrc, stage_op + (i * 4 + wave) * 1024, v);
    }

    __device__ inline void issue(__amdgpu_buffer_rsrc_t rsrc, MLXHIP_LDS char* stage_op, int wave,
                                 int k0) const {
#pragma unroll
        for (int i = 0; i < LOADS_PER_OP; ++i) issue_one(rsrc, stage_op, wave, k0, i);
    }
};

// Per-lane LDS byte offsets of one operand's fragments inside a stage.
//   KC : off(x, s) = base_s + x * 2048            (x: 32-row block, s: k-step)
//   !KC: off(x, s, r) = base_x[x] + (16 s + 4 r) * 512
template <bool KC>
struct FragAddr {
    uint32_t base[KC ? 2 : 4];
    __device__ inline void init(int lane, int quad_off /* 128 * wave quadrant */) {
        if constexpr (KC) {
            const int r = lane & 31;
            const int sw = (r >> 2) & 3;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int c = 2 * s + (lane >> 5);
                base[s] = (uint32_t)((quad_off + r) * 64 + ((c ^ sw) * 16));
            }
        } else {
            const int g = lane >> 4, t = lane & 15;
            const int krow = 8 * (g >> 1) + (t >> 2);
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const int chunk = (quad_off >> 3) + 4 * (x ^ (t >> 2)) + 2 * (g & 1) + ((t >> 1) & 1);
                base[x] = (uint32_t)(krow * 512 + chunk * 16 + (t & 1) * 8);
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

// Number of LDS read instructions for one operand's 4 fragments of a k-step.
template <bool KC>
constexpr int reads_per_step() { return KC ? 4 : 8; }

// Read `idx` (0 .. reads_per_step-1) of one operand's fragments for k-step s:
// KC: fragment idx (ds_read_b128); !KC: half idx % 2 of fragment idx / 2
// (ds_read_b64_tr_b16, k offsets 0-3 or 4-7).
template <bool KC>
__device__ inline void read_one(const MLXHIP_LDS char* op, const FragAddr<KC>& fa, int s, int idx, u32x4* f) {
    if constexpr (KC) {
        f[idx] = *(const MLXHIP_LDS u32x4*)(op + fa.base[s] + idx * 2048);
    } else {
        const int x = idx >> 1, r = idx & 1;
        const MLXHIP_LDS char* p = op + fa.base[x] + (16 * s + 4 * r) * 512;
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

// Loads the 4 fragments of one operand for k-step s of the stage at `op`.
template <bool KC>
__device__ inline void read_frags(const MLXHIP_LDS char* op, const FragAddr<KC>& fa, int s, u32x4* f) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        if constexpr (KC) {
            f[x] = *(const MLXHIP_LDS u32x4*)(op + fa.base[s] + x * 2048);
        } else {
            const MLXHIP_LDS char* p = op + fa.base[x] + 16 * s * 512;
            i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((MLXHIP_LDS i16x4*)p);
            i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((MLXHIP_LDS i16x4*)(p + 4 * 512));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            f[x] = u32x4{l2.x, l2.y, h2.x, h2.y};
        }
    }
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

template <int DT, int CT, int TA, int TB, int STAGES, bool SPREAD>
__global__ __attribute__((amdgpu_flat_work_group_size(THREADS, THREADS), amdgpu_waves_per_eu(1, 1)))
void gemm16_kernel(Args g) {
    constexpr bool KCA = (TA == 0);  // A stored [M][K]
    constexpr bool KCB = (TB == 1);  // B stored [N][K]
    static_assert(STAGES >= 3 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS budget");
    constexpr int SMEM_BYTES = STAGES * STAGE_BYTES > 4 * 128 * (256 + 16) ? STAGES * STAGE_BYTES : 4 * 128 * (256 + 16);
    __shared__ __attribute__((aligned(1024))) char smem_raw[SMEM_BYTES];
    MLXHIP_LDS char* smem = (MLXHIP_LDS char*)smem_raw;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware tile order: consecutive workgroup ids go to the 8 XCDs
    // round-robin; give each XCD a contiguous range of tile ids, then order
    // the range in groups of 4 tile rows so neighbours share A rows / B
    // columns inside one XCD's L2.
    const int nwg = g.tiles_m * g.tiles_n;
    int id = blockIdx.x;
    if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
    constexpr int GROUP_M = 4;
    const int in_group = GROUP_M * g.tiles_n;
    const int first_m = (id / in_group) * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int tm = first_m + (id % in_group) % gsz;
    const int tn = (id % in_group) / gsz;
    const int64_t m0 = (int64_t)tm * TILE, n0 = (int64_t)tn * TILE;

    const int64_t batch = blockIdx.y;
    const char* A = static_cast<const char*>(g.a) + batch * g.sa * 2;
    const char* B = static_cast<const char*>(g.b) + batch * g.sb * 2;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)g.a_bytes, BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)g.b_bytes, BUF_FLAGS);

    Loader<KCA> la;
    Loader<KCB> lb;
    la.init(tid, m0, g.m, g.lda, g.k);
    lb.init(tid, n0, g.n, g.ldb, g.k);
    FragAddr<KCA> fa;
    FragAddr<KCB> fb;
    fa.init(lane, 128 * wm);
    fb.init(lane, 128 * wn);

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int nk = (int)((g.k + BK - 1) / BK);
    constexpr int LOADS_PER_TILE = 2 * LOADS_PER_OP;

    // Prologue: tiles 0 .. STAGES-1 into stages 0 .. STAGES-1.
    // With SPREAD, B's loads of tile t+STAGES are issued in the first half of
    // iteration t+1 instead (one per four MFMAs) and the prologue leaves out
    // B of tile STAGES-1; the count of loads younger than any tile is unchanged.
#pragma unroll
    for (int t = 0; t < STAGES; ++t) {
        MLXHIP_LDS char* st = smem + t * STAGE_BYTES;
        la.issue(ra, st, wave, t * BK);
        if (!SPREAD || t < STAGES - 1) lb.issue(rb, st + OP_BYTES, wave, t * BK);
    }
    if constexpr (SPREAD) wait_vmcnt<(STAGES - 2) * LOADS_PER_TILE + LOADS_PER_OP>();
    else wait_vmcnt<(STAGES - 1) * LOADS_PER_TILE>();
    lds_barrier();

    u32x4 af[2][4], bf[2][4];
    read_frags<KCA>(smem, fa, 0, af[0]);
    read_frags<KCB>(smem + OP_BYTES, fb, 0, bf[0]);

    // Each half-tile issues 16 MFMAs, one per 32-cycle MFMA slot, with the
    // LDS reads / LDS-bound loads of the next half placed between them; the
    // scheduling barriers keep that order (the compiler would otherwise sink
    // each read next to its first use and expose the LDS latency).
    constexpr int NA = reads_per_step<KCA>(), NB = reads_per_step<KCB>(), NR = NA + NB;
    constexpr int OPS2 = (SPREAD ? 1 : 2) * LOADS_PER_OP + NR;
    static_assert(NR <= 16, "one read per MFMA slot in the first half");
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt % STAGES;
        const MLXHIP_LDS char* st = smem + cur * STAGE_BYTES;
        // First half: MFMAs of k-step 0, reads of k-step 1 of this tile.
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            mfma<DT>(bf[0][q & 3], af[0][q >> 2], acc[q >> 2][q & 3]);
            if (q < NA) read_one<KCA>(st, fa, 1, q, af[1]);
            else if (q < NR) read_one<KCB>(st + OP_BYTES, fb, 1, q - NA, bf[1]);
            if constexpr (SPREAD) {
                // B of tile kt-1+STAGES into the stage released in iteration kt-1.
                if ((q & 3) == 3)
                    lb.issue_one(rb, smem + ((kt + STAGES - 1) % STAGES) * STAGE_BYTES + OP_BYTES, wave,
                                 (kt - 1 + STAGES) * BK, q >> 2);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // Tile kt+1 has landed for every wave; every wave is done reading
        // this tile's stage, which then receives tile kt+STAGES.
        wait_vmcnt<(STAGES - 2) * LOADS_PER_TILE>();
        lds_barrier();
        MLXHIP_LDS char* dst = smem + cur * STAGE_BYTES;
        const int k0 = (kt + STAGES) * BK;
        const MLXHIP_LDS char* nx = smem + ((kt + 1) % STAGES) * STAGE_BYTES;
        // Second half: MFMAs of k-step 1; the k-step 0 reads of tile kt+1
        // and the loads of tile kt+STAGES.
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            mfma<DT>(bf[1][q & 3], af[1][q >> 2], acc[q >> 2][q & 3]);
#pragma unroll
            for (int o = (q * OPS2) / 16; o < ((q + 1) * OPS2) / 16; ++o) {
                // Reads first: the next tile's first MFMAs consume them.
                if (o < NA) read_one<KCA>(nx, fa, 0, o, af[0]);
                else if (o < NR) read_one<KCB>(nx + OP_BYTES, fb, 0, o - NA, bf[0]);
                else if (o < NR + LOADS_PER_OP) la.issue_one(ra, dst, wave, k0, o - NR);
                else if (!SPREAD) lb.issue_one(rb, dst + OP_BYTES, wave, k0, o - NR - LOADS_PER_OP);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vmcnt<0>();

    // Epilogue through LDS. acc[i][j][v] = C[m][n] with m = 128 wm + 32 i +
    // lane % 32 and n = 128 wn + 32 j + 8 (v / 4) + 4 (lane / 32) + v % 4
    // inside the tile. Each wave converts its 128 x 128 quadrant into padded
    // LDS rows (PITCH = row bytes + 16: 16 consecutive rows fall in distinct
    // bank groups for the 8/16-byte writes) and reads it back row by row, so
    // every global store instruction writes whole 256- or 512-byte row
    // segments instead of 16-byte pieces of 32 rows.
    wait_vmcnt<0>();
    lds_barrier();  // every wave is done with the operand stages
    constexpr int ES = CT == MLXHIP_DTYPE_F32 ? 4 : 2;
    constexpr int ROW_BYTES = 128 * ES;
    constexpr int PITCH = ROW_BYTES + 16;
    constexpr int PASS_ROWS = ES == 2 ? 128 : 64;  // quadrant rows staged per pass
    constexpr int LANES_PER_ROW = ROW_BYTES / 16;
    constexpr int ROWS_PER_READ = 64 / LANES_PER_ROW;
    static_assert(4 * PASS_ROWS * PITCH <= SMEM_BYTES, "epilogue staging fits in LDS");
    MLXHIP_LDS char* region = smem + wave * PASS_ROWS * PITCH;
    char* C = static_cast<char*>(g.c) + batch * g.sc * ES;
    const int64_t row0 = m0 + 128 * wm, col0 = n0 + 128 * wn;
    const bool vec_ok = (g.ldc * ES) % 16 == 0 && (reinterpret_cast<uintptr_t>(C) % 16) == 0;
#pragma unroll
    for (int pass = 0; pass < 128 / PASS_ROWS; ++pass) {
#pragma unroll
        for (int i = 0; i < PASS_ROWS / 32; ++i) {
            const int ii = pass * (PASS_ROWS / 32) + i;
            const int r = 32 * i + (lane & 31);
#pragma unroll
            for (int j = 0; j < 4; ++j)
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
            const u32x4 v = *(const MLXHIP_LDS u32x4*)(region + r * PITCH + cb);
            const int64_t m = row0 + pass * PASS_ROWS + r;
            const int64_t n = col0 + cb / ES;
            if (m >= g.m || n >= g.n) continue;
            char* dst = C + (m * g.ldc + n) * ES;
            if (vec_ok && n + 16 / ES <= g.n) {
                *reinterpret_cast<u32x4*>(dst) = v;
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

// Host-side check of what the kernel assumes about its operands; returns
// false when the general GEMM must run instead.
inline bool supported(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const void* a,
                      int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, uint32_t* a_bytes,
                      uint32_t* b_bytes) {
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(b) % 16) return false;
    if (k >= (1 << 30)) return false;  // k offsets are 32-bit in the kernel
    if (lda % 8 || ldb % 8) return false;
    if (batch > 1 && (sa % 8 || sb % 8)) return false;
    // The contiguous extent of each operand must hold whole 16-byte chunks.
    if ((ta == 0 ? k : m) % 8) return false;
    if ((tb == 1 ? k : n) % 8) return false;
    const int64_t a_rows = ta ? k : m, b_rows = tb ? n : k;
    const int64_t a_ext = ((a_rows - 1) * lda + (ta ? m : k)) * 2;
    const int64_t b_ext = ((b_rows - 1) * ldb + (tb ? k : n)) * 2;
    const int64_t lim = (int64_t)OOB - 4096;
    if (a_ext <= 0 || b_ext <= 0 || a_ext >= lim || b_ext >= lim) return false;
    *a_bytes = (uint32_t)a_ext;
    *b_bytes = (uint32_t)b_ext;
    return true;
}

template <int DT, int CT, int TA, int TB>
int launch(const Args& a0, int64_t batch, hipStream_t s) {
    Args a = a0;
    a.tiles_m = (int)ceil_div(a.m, TILE);
    a.tiles_n = (int)ceil_div(a.n, TILE);
    dim3 grid((unsigned)(a.tiles_m * a.tiles_n), (unsigned)batch);
    hipLaunchKernelGGL((gemm16_kernel<DT, CT, TA, TB, 4, true>), grid, dim3(THREADS), 0, s, a);
    return launch_check("gemm16_kernel");
}

template <int DT, int CT>
int dispatch(const Args& a, int64_t batch, int ta, int tb, hipStream_t s) {
    if (!ta && !tb) return launch<DT, CT, 0, 0>(a, batch, s);
    if (!ta && tb) return launch<DT, CT, 0, 1>(a, batch, s);
    if (ta && !tb) return launch<DT, CT, 1, 0>(a, batch, s);
    return launch<DT, CT, 1, 1>(a, batch, s);
}

}  // namespace gemm16

// Per-dtype entry points (gemm16_bf16.hip, gemm16_f16.hip).
int gemm16_bf16(int c_dtype, int ta, int tb, const gemm16::Args& a, int64_t batch, hipStream_t s);
int gemm16_f16(int c_dtype, int ta, int tb, const gemm16::Args& a, int64_t batch, hipStream_t s);

}  // namespace mlxhip
