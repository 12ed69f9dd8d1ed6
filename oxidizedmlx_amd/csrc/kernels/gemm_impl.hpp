// gemm_impl.hpp — MFMA GEMM kernel template for gfx950 (CDNA4).
//
// C_b[M,N] = op(A_b) * op(B_b), row-major, f32 accumulation; replaces
// matmul (crates/mlx-core/src/cpu_kernels.rs:197-230) and the Metal
// tiled_gemm_f32 (crates/mlx-metal/src/kernels/gemm.metal:32-77).
//
// Work decomposition
//   * 256 threads = 4 wavefronts in a 2x2 grid; each wave owns WTM x WTN
//     32x32 MFMA tiles, so the block tile is BM = 64*WTM by BN = 64*WTN.
//   * K advances in LDS tiles of 8 "chunks" per row, a chunk being 16 bytes
//     (8 bf16/f16 or 4 f32): BK = 64 for 16-bit inputs, 32 for f32.
//   * Both operands sit in LDS K-contiguous ([row][k]), the layout MFMA
//     fragments want (a lane holds consecutive k of one row / column).
//     Operands whose K is the strided dimension in HBM (A^T stored [K,M],
//     B stored [K,N]) are transposed in registers on the way to LDS
//     (CHxCH blocks), so NN/TN/NT/TT all run from the same inner loop.
//   * LDS chunk c of tile row r lives at physical chunk c ^ ((r ^ r>>3) & 7):
//     conflict-free for the fragment reads (8 consecutive rows, same chunk)
//     and for the transposed writes (8 rows 8 apart, same chunk).
//   * Two LDS stages; global loads for tile k+1 are issued into registers
//     before the MFMAs of tile k, written to the other stage afterwards;
//     one barrier per K tile.
//   * Workgroups are numbered so that consecutive hardware workgroup ids,
//     which land on the 8 XCDs round-robin, map to tiles that share rows
//     of A / columns of B inside one XCD's L2 (grouped ordering, 4 tile rows).
//
// MFMA (wave64): 16-bit inputs use v_mfma_f32_32x32x16_{bf16,f16} (lanes
// 0-31 hold k 0-7 of the 16-k step, lanes 32-63 k 8-15, 8 elements each);
// f32 inputs use v_mfma_f32_32x32x2_f32 four times per 8-k step, lane group
// g supplying k = 4c+t of its chunk. Accumulator element v of lane l is
// C[8*(v/4) + 4*(l/32) + v%4][l%32].
#pragma once

#include "../common.hpp"

namespace mlxhip {
namespace gemm_detail {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct GemmArgs {
    int64_t m, n, k;
    const void* a;
    int64_t lda, sa;
    const void* b;
    int64_t ldb, sb;
    void* c;
    int64_t ldc, sc;
    int tiles_m, tiles_n;
    // Split-K: blockIdx.y = batch * splits + split; split s covers
    // k in [s * k_chunk, min(k, (s + 1) * k_chunk)) and writes its f32
    // partial product to ws + blockIdx.y * m * n (row pitch n); a second
    // kernel sums the partials in split order.
    int splits = 1;
    int64_t k_chunk = 0;
    float* ws = nullptr;
};

template <int DT>
struct Elem;
template <>
struct Elem<MLXHIP_DTYPE_BF16> {
    using T = uint16_t;
    static constexpr int CH = 8;
};
template <>
struct Elem<MLXHIP_DTYPE_F16> {
    using T = uint16_t;
    static constexpr int CH = 8;
};
template <>
struct Elem<MLXHIP_DTYPE_F32> {
    using T = uint32_t;
    static constexpr int CH = 4;
};

__device__ inline int phys_chunk(int r, int c) { return c ^ ((r ^ (r >> 3)) & 7); }

// One 16-byte chunk of row r, elements [c, c+CH) of a row-major matrix with
// R valid rows and Cn valid columns; out-of-range elements read as zero.
template <typename T, int CH, bool ALIGNED>
__device__ inline uint4 load_chunk(const T* __restrict__ base, int64_t ld, int64_t r, int64_t c,
                                   int64_t R, int64_t Cn) {
    uint4 z = make_uint4(0, 0, 0, 0);
    if (r >= R || c >= Cn) return z;
    const T* p = base + r * ld + c;
    if (ALIGNED && c + CH <= Cn) return *reinterpret_cast<const uint4*>(p);
    union {
        uint4 v;
        T e[CH];
    } u;
    u.v = z;
#pragma unroll
    for (int e = 0; e < CH; ++e)
        if (c + e < Cn) u.e[e] = p[e];
    return u.v;
}

// Transposes a CHxCH block held as CH row chunks (row i = k0+i, element j =
// column j) into CH column chunks (chunk j = column j, element i = row i).
template <int CH>
__device__ inline void transpose_block(const uint4* in, uint4* out);

template <>
__device__ inline void transpose_block<8>(const uint4* in, uint4* out) {
    // 16-bit elements: dword d of a chunk holds elements 2d (low) and 2d+1 (high).
    const uint32_t* w = reinterpret_cast<const uint32_t*>(in);  // w[i*4 + d]
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = w[(2 * e) * 4 + j / 2];
            const uint32_t hi = w[(2 * e + 1) * 4 + j / 2];
            o[e] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        out[j] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

template <>
__device__ inline void transpose_block<4>(const uint4* in, uint4* out) {
    out[0] = make_uint4(in[0].x, in[1].x, in[2].x, in[3].x);
    out[1] = make_uint4(in[0].y, in[1].y, in[2].y, in[3].y);
    out[2] = make_uint4(in[0].z, in[1].z, in[2].z, in[3].z);
    out[3] = make_uint4(in[0].w, in[1].w, in[2].w, in[3].w);
}

__device__ inline uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int CT>
__device__ inline void store_c(void* c, int64_t idx, float v) {
    if constexpr (CT == MLXHIP_DTYPE_F32) static_cast<float*>(c)[idx] = v;
    else if constexpr (CT == MLXHIP_DTYPE_BF16) static_cast<uint16_t*>(c)[idx] = f32_to_bf16(v);
    else static_cast<_Float16*>(c)[idx] = (_Float16)v;
}

template <int DT>
__device__ inline void mfma_step(const uint4& a, const uint4& b, f32x16& acc) {
    if constexpr (DT == MLXHIP_DTYPE_BF16) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    } else if constexpr (DT == MLXHIP_DTYPE_F16) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
    } else {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
    }
}

// Stages one operand tile (ROWS tile rows x 8 chunks) from HBM into registers.
//   KCONTIG: the operand is stored [rows][K] (K contiguous): chunk q of the
//            tile is row q/8, chunk q%8, one 16-byte load each.
//   else   : stored [K][rows]: CHxCH blocks, block b = (kb, rb) with rb
//            fastest so a wave reads whole 16-byte runs of a K row.
template <typename T, int CH, int ROWS, bool KCONTIG, bool ALIGNED>
struct OperandTile {
    static constexpr int CHUNKS = ROWS * 8;                    // K-contiguous case
    static constexpr int NBLK = (8 * CH / CH) * (ROWS / CH);   // = 8 * ROWS / CH blocks
    static constexpr int PER_THREAD = KCONTIG ? CHUNKS / 256 : (NBLK + 255) / 256;
    static constexpr int REGS = KCONTIG ? PER_THREAD : PER_THREAD * CH;
    uint4 r[REGS];

    // base: operand of this batch; row0: first tile row (M or N index);
    // k0: first k of the tile; R / Kn: valid rows / k.
    __device__ inline void load(const T* __restrict__ base, int64_t ld, int64_t row0, int64_t k0,
                                int64_t R, int64_t Kn, int tid) {
        if constexpr (KCONTIG) {
#pragma unroll
            for (int i = 0; i < PER_THREAD; ++i) {
                const int q = i * 256 + tid;
                const int row = q >> 3, ch = q & 7;
                r[i] = load_chunk<T, CH, ALIGNED>(base, ld, row0 + row, k0 + ch * CH, R, Kn);
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_THREAD; ++i) {
                const int bidx = i * 256 + tid;
                if (NBLK % 256 == 0 || bidx < NBLK) {
                    const int rb = bidx % (ROWS / CH), kb = bidx / (ROWS / CH);
#pragma unroll
                    for (int e = 0; e < CH; ++e)
                        r[i * CH + e] = load_chunk<T, CH, ALIGNED>(base, ld, k0 + kb * CH + e,
                                                                   row0 + rb * CH, Kn, R);
                }
            }
        }
    }

    __device__ inline void store(uint4 (*lds)[8], int tid) const {
        if constexpr (KCONTIG) {
#pragma unroll
            for (int i = 0; i < PER_THREAD; ++i) {
                const int q = i * 256 + tid;
                const int row = q >> 3, ch = q & 7;
                lds[row][phys_chunk(row, ch)] = r[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_THREAD; ++i) {
                const int bidx = i * 256 + tid;
                if (NBLK % 256 == 0 || bidx < NBLK) {
                    const int rb = bidx % (ROWS / CH), kb = bidx / (ROWS / CH);
                    uint4 t[CH];
                    transpose_block<CH>(&r[i * CH], t);
                    // For CH = 4 a chunk holds 4 k; the 8-chunk LDS row then
                    // spans k 0..31 and block kb covers chunk kb.
#pragma unroll
                    for (int e = 0; e < CH; ++e) {
                        const int row = rb * CH + e;
                        lds[row][phys_chunk(row, kb)] = t[e];
                    }
                }
            }
        }
    }
};

template <int DT, int CT, int TA, int TB, int WTM, int WTN, bool ALIGNED>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 2)))
void gemm_kernel(GemmArgs g) {
    using T = typename Elem<DT>::T;
    constexpr int CH = Elem<DT>::CH;
    constexpr int BM = 64 * WTM, BN = 64 * WTN;
    constexpr int BK = 8 * CH;
    __shared__ uint4 lds[2][BM + BN][8];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware grouped tile order.
    const int nwg = g.tiles_m * g.tiles_n;
    int id = blockIdx.x;
    if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
    constexpr int GROUP_M = 4;
    const int in_group = GROUP_M * g.tiles_n;
    const int first_m = (id / in_group) * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int tm = first_m + (id % in_group) % gsz;
    const int tn = (id % in_group) / gsz;

    const int64_t by = blockIdx.y;
    const int64_t batch = by / g.splits, split = by % g.splits;
    const int64_t kb = split * g.k_chunk;                       // first k of this split
    const int64_t klen = g.splits > 1 ? min(g.k - kb, g.k_chunk) : g.k;
    const T* A = static_cast<const T*>(g.a) + batch * g.sa + (TA ? kb * g.lda : kb);
    const T* B = static_cast<const T*>(g.b) + batch * g.sb + (TB ? kb : kb * g.ldb);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    // A is K-contiguous unless transposed; B is K-contiguous only when transposed.
    OperandTile<T, CH, BM, TA == 0, ALIGNED> at;
    OperandTile<T, CH, BN, TB == 1, ALIGNED> bt;

    f32x16 acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int64_t nk = (klen + BK - 1) / BK;
    at.load(A, g.lda, m0, 0, g.m, klen, tid);
    bt.load(B, g.ldb, n0, 0, g.n, klen, tid);
    at.store(lds[0], tid);
    bt.store(lds[0] + BM, tid);
    __syncthreads();

    const int lrow = lane & 31, lgrp = lane >> 5;
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int cur = (int)(kt & 1);
        const bool more = kt + 1 < nk;
        if (more) {
            at.load(A, g.lda, m0, (kt + 1) * BK, g.m, klen, tid);
            bt.load(B, g.ldb, n0, (kt + 1) * BK, g.n, klen, tid);
        }
        uint4(*As)[8] = lds[cur];
        uint4(*Bs)[8] = lds[cur] + BM;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int c = 2 * s + lgrp;
            uint4 af[WTM], bf[WTN];
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                const int r = wm * 32 * WTM + i * 32 + lrow;
                af[i] = As[r][phys_chunk(r, c)];
            }
#pragma unroll
            for (int j = 0; j < WTN; ++j) {
                const int r = wn * 32 * WTN + j * 32 + lrow;
                bf[j] = Bs[r][phys_chunk(r, c)];
            }
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j) mfma_step<DT>(af[i], bf[j], acc[i][j]);
        }
        if (more) {
            at.store(lds[cur ^ 1], tid);
            bt.store(lds[cur ^ 1] + BM, tid);
        }
        __syncthreads();
    }

    // Epilogue: accumulator element v of lane l is C[8*(v/4) + 4*(l/32) + v%4][l%32].
    if (g.splits > 1) {
        // f32 partial of this split into its workspace slice.
        float* P = g.ws + by * g.m * g.n;
#pragma unroll
        for (int i = 0; i < WTM; ++i)
#pragma unroll
            for (int j = 0; j < WTN; ++j) {
                const int64_t col = n0 + wn * 32 * WTN + j * 32 + lrow;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t row = m0 + wm * 32 * WTM + i * 32 + 8 * (v >> 2) + 4 * lgrp + (v & 3);
                    if (row < g.m && col < g.n) P[row * g.n + col] = acc[i][j][v];
                }
            }
        return;
    }
    void* C = g.c;
    const int64_t cbase = batch * g.sc;
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int64_t col = n0 + wn * 32 * WTN + j * 32 + lrow;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = m0 + wm * 32 * WTM + i * 32 + 8 * (v >> 2) + 4 * lgrp + (v & 3);
                if (row < g.m && col < g.n) store_c<CT>(C, cbase + row * g.ldc + col, acc[i][j][v]);
            }
        }
}

template <int DT, int CT, int TA, int TB, int WTM, int WTN, bool ALIGNED>
int launch(const GemmArgs& a0, int64_t batch, hipStream_t s) {
    GemmArgs a = a0;
    a.tiles_m = (int)ceil_div(a.m, 64 * WTM);
    a.tiles_n = (int)ceil_div(a.n, 64 * WTN);
    dim3 grid((unsigned)(a.tiles_m * a.tiles_n), (unsigned)(batch * a.splits));
    hipLaunchKernelGGL((gemm_kernel<DT, CT, TA, TB, WTM, WTN, ALIGNED>), grid, dim3(256), 0, s, a);
    return launch_check("gemm_kernel");
}

// Block tile edge of the general kernel: 64 * wt (wt = 1, 2 or 4 MFMA tiles
// per wave and dimension). The host picks wt and the split-K factor.
template <int DT, int CT, int TA, int TB>
int dispatch_layout(const GemmArgs& a, int64_t batch, bool aligned, int wt, hipStream_t s) {
    if (!aligned) return launch<DT, CT, TA, TB, 2, 2, false>(a, batch, s);
    if (wt == 4) return launch<DT, CT, TA, TB, 4, 4, true>(a, batch, s);
    if (wt == 1) return launch<DT, CT, TA, TB, 1, 1, true>(a, batch, s);
    return launch<DT, CT, TA, TB, 2, 2, true>(a, batch, s);
}

template <int DT, int CT>
int dispatch_trans(const GemmArgs& a, int64_t batch, int ta, int tb, bool aligned, int wt, hipStream_t s) {
    if (!ta && !tb) return dispatch_layout<DT, CT, 0, 0>(a, batch, aligned, wt, s);
    if (!ta && tb) return dispatch_layout<DT, CT, 0, 1>(a, batch, aligned, wt, s);
    if (ta && !tb) return dispatch_layout<DT, CT, 1, 0>(a, batch, aligned, wt, s);
    return dispatch_layout<DT, CT, 1, 1>(a, batch, aligned, wt, s);
}

}  // namespace gemm_detail

// Per-input-dtype entry points (one translation unit each, compiled in parallel).
int gemm_f32(int c_dtype, int ta, int tb, const gemm_detail::GemmArgs& a, int64_t batch,
             bool aligned, int wt, hipStream_t s);
int gemm_bf16(int c_dtype, int ta, int tb, const gemm_detail::GemmArgs& a, int64_t batch,
              bool aligned, int wt, hipStream_t s);
int gemm_f16(int c_dtype, int ta, int tb, const gemm_detail::GemmArgs& a, int64_t batch,
             bool aligned, int wt, hipStream_t s);

}  // namespace mlxhip
