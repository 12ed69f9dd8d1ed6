// decode.hip — the kernels of one greedy decode step of a decoder-only
// language model whose weights live in HBM as bf16 and whose activations and
// KV cache are f32 (the caller is csrc/decoder.cpp).
//
// One step for a batch of B <= 8 sequences at position t (t is read from a
// device counter, so one captured HIP graph serves every step), starting
// from x[b] = f32(E[token[t][b]]) (embedding_lookup,
// crates/mlx-core/src/cpu_kernels.rs:317-336: index clamped to [0, vocab-1]):
//   per layer:
//     gemv<QKV,norm> [q|k|v] = rms_norm(x)·Wqkv^T + b; k, v stored into the
//                    layer's KV cache at position t
//     decode_attn    o = softmax(q·K^T·scale)·V over positions 0..t, per
//                    (sequence, head) (cpu_attention, cpu_kernels.rs:738-812
//                    with Tq = 1, i.e. the decode loop of
//                    crates/mlx-conformance/tests/ttft_behavior.rs:101-216)
//     gemv<RESID>    x = x + (o·Wo^T + bo)
//     gemv<SILU,norm> u = silu(rms_norm(x)·W1^T + b1)
//     gemv<RESID>    x = x + (u·W2^T + b2)
//   gemv<ARGMAX,norm> logits = rms_norm(x)·Wlm^T, per-workgroup maxima
//   decode_finish    argmax, next token, its embedding into x, t += 1
// (decode_embed writes x for position 0 before the first step.)
//
// The GEMV (Y[B,N] = X[B,K]·W[N,K]^T) is HBM-bound on W. It runs on MFMA
// (v_mfma_f32_16x16x32_bf16) without rounding the f32 activations to bf16:
// each activation is kept as three bf16 terms x = hi + mid + lo (each term
// the round-to-nearest-even bf16 of what the previous ones left; the
// differences are exact in f32), so hi/mid/lo carry 24 significant bits
// between them and bf16·bf16 products are exact in the f32 accumulator. The
// 24 columns [hi b0..7 | mid b0..7 | lo b0..7] fill two 16-column MFMA tiles
// (the last 8 columns are zero) and y = hi + (mid + lo) per (row, b).
//
// Split activations: whatever produces an activation that a GEMV consumes
// (the residual updates, the SiLU, the attention, the embedding lookups)
// also writes it as three bf16 planes Xs[3][DEC_MAX_BATCH][ld] (plane 0 hi,
// 1 mid, 2 lo; row b of a plane is sequence b). The consuming GEMV loads its
// MFMA B operand straight from those planes, so no workgroup re-splits or
// stages X. RMS normalisation is a per-sequence scale: the GEMV runs on the
// raw activation and divides the dot product by the row's RMS, which it
// sums from the f32 activation while the MFMAs run.
#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "../common.hpp"
#include "../kernels.hpp"
#include "device_math.hpp"

#pragma clang fp contract(off)

namespace mlxhip {
namespace {

using dev::div_by;
using dev::shared_divisor;
using dev::sigmoid_ref;
using dev::wave_max;
using dev::wave_sum;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr int KSTEP = 32;                 // k per MFMA
constexpr int NSTEP = 6;                  // MFMA steps per pass (W and X fragments of a pass held in registers)
constexpr int TILE_N = 16;                // output features per wave tile
constexpr int MAX_WAVES = 16;
constexpr int XN = 4;                     // X units (8 k of 3 planes) per thread per round
// The LM head's shape: one k-slice per wave over the whole K in one pass (up
// to WIDE_NSTEP steps), up to WIDE_WAVES row tiles per workgroup, fewer X
// units per thread (more threads per unit of X).
constexpr int WIDE_NSTEP = 24;
constexpr int WIDE_XN = 2;
constexpr int WIDE_WAVES = 8;
constexpr int XPAD = 8;                   // bf16 padding of each LDS plane row (spreads rows over the banks)
constexpr int XROWS = 3 * DEC_MAX_BATCH;  // hi, mid, lo rows of the batch
constexpr int WSS_FLOATS = 2 * DEC_MAX_BATCH;  // rms, 1/rms

__device__ inline uint32_t bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ inline float bf16_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Writes v as its hi/mid/lo bf16 terms into the planes of `xs` (row b, column n).
__device__ inline void store_split(uint16_t* xs, int64_t ld, int b, int64_t n, float v) {
    const uint32_t h = bf16_rne(v);
    const float r1 = v - bf16_f32(h);
    const uint32_t m = bf16_rne(r1);
    const float r2 = r1 - bf16_f32(m);
    xs[(int64_t)b * ld + n] = (uint16_t)h;
    xs[(int64_t)(DEC_MAX_BATCH + b) * ld + n] = (uint16_t)m;
    xs[(int64_t)(2 * DEC_MAX_BATCH + b) * ld + n] = (uint16_t)bf16_rne(r2);
}

// Row b of x (and its planes) = f32 of the bf16 embedding row `src`, 8
// values per unit (the planes: hi = the bf16 value, mid = lo = 0).
__device__ inline void store_embedding_unit(const uint4 e, float* x, uint16_t* xs, int64_t ld, int b, int k) {
    float* xr = x + (int64_t)b * ld + k;
    const uint32_t w[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
    for (int j = 0; j < 2; ++j)
        reinterpret_cast<float4*>(xr)[j] =
            make_float4(bf16_f32(w[2 * j] & 0xFFFFu), bf16_f32(w[2 * j] >> 16), bf16_f32(w[2 * j + 1] & 0xFFFFu),
                        bf16_f32(w[2 * j + 1] >> 16));
    *reinterpret_cast<uint4*>(xs + (int64_t)b * ld + k) = e;
    *reinterpret_cast<uint4*>(xs + (int64_t)(DEC_MAX_BATCH + b) * ld + k) = make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(xs + (int64_t)(2 * DEC_MAX_BATCH + b) * ld + k) = make_uint4(0u, 0u, 0u, 0u);
}

// Maximum over the lanes of a wave that share lane % 8 (one sequence each).
__device__ inline uint64_t wave_max_u64_by8(uint64_t v) {
#pragma unroll
    for (int o = 8; o < WAVE; o <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)v, o, WAVE);
        const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, WAVE);
        const uint64_t w = ((uint64_t)hi << 32) | lo;
        v = w > v ? w : v;
    }
    return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)v, o, WAVE);
        const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, WAVE);
        const uint64_t w = ((uint64_t)hi << 32) | lo;
        v = w > v ? w : v;
    }
    return v;
}

// Total order of finite floats as unsigned integers, larger value = larger key.
__device__ inline uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ── the split-activation GEMV ──────────────────────────────────────────────
//
// Workgroup = R row tiles x KS k-slices, one wave each (R*KS <= 16). Wave
// (r, s) computes the 16 output features of tile blockIdx.x*R + r over k in
// [s*kw, (s+1)*kw). Partials of the KS slices are summed in slice order
// (deterministic).
//
// The workgroup first stages the X planes (rows of the B <= 8 sequences) in
// LDS with contiguous 16-byte loads, one (sequence, 8-k unit) of all three
// planes per thread, so each load instruction covers 1 KB of consecutive
// memory; the MFMA B operands are then read from LDS. Loading them straight
// from memory in MFMA layout (16 rows x 64 bytes per instruction, repeated
// by every row tile of the workgroup) measured 1-5 us slower per launch.
// With NORM the same thread also sums the squares of its unit's values
// (hi + mid + lo reproduces the f32 value exactly), and wave b (mod waves)
// adds the units of row b in k order, then across lanes, for the RMS of
// sequence b; the GEMV runs on the raw activation and its dot products are
// divided by the RMS.
//
// The kernel is latency-bound at decode sizes (a few MB per launch), so every
// global load whose address does not depend on this kernel's own results is
// issued at the start, before the first wait: the X units, the W fragments
// of the first pass, the step position and the epilogue's bias and residual
// values.
//
// ARGMAX (the LM head) publishes each workgroup's per-sequence maximum key
// for decode_finish.
//
// groups > 1 splits the batch: the workgroups of one row-tile set each take
// ceil(B/groups) consecutive sequences, staging only their planes (the other
// LDS rows hold whatever was there; an MFMA output column depends only on its
// own B column, and those columns are never stored). A launch with few row
// tiles (N = 768: 48 workgroups) then spreads its X traffic, which at
// K = 3072 is larger than its W, over 4x the CUs. When the row-tile sets are a
// multiple of 8, the groups of one set share an XCD (workgroup i runs on XCD
// i % 8), so its W comes from HBM once per set and from that L2 after.
//
// NS, XNT: MFMA steps per pass and X units per thread per round (the LM
// head's wide shape holds a whole K of 768 in registers: 8 waves at most).
template <int EPI, bool NORM, int NS = NSTEP, int XNT = XN>
__global__ __launch_bounds__((NS > NSTEP ? WIDE_WAVES : MAX_WAVES) * WAVE) void gemv_kernel(DecGemv p, int ks,
                                                                                            int r_tiles, int kw,
                                                                                            int groups) {
    constexpr int KP = NS * KSTEP;  // k per wave per pass
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int K = p.k, N = p.n, B = p.batch;
    constexpr int TB = TILE_N * DEC_MAX_BATCH;  // outputs of one row tile
    const int pitch = K + XPAD;                 // bf16 per LDS plane row
    uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                                    // [24][pitch]
    float* red = reinterpret_cast<float*>(smem + (size_t)XROWS * pitch * 2);            // [r_tiles * ks][TB]
    float* wss = red + r_tiles * ks * TB;                                                // [2][8]: rms, 1/rms
    uint64_t* keys = reinterpret_cast<uint64_t*>(wss + WSS_FLOATS);                     // ARGMAX: [nwaves][8] of [r_tiles * TB]
    float* psum = reinterpret_cast<float*>(keys + (EPI == DEC_EPI_ARGMAX ? r_tiles * TB : 0));  // NORM: [8][K/8]

    const int tid = threadIdx.x, nthr = blockDim.x;
    const int wave = tid / WAVE, lane = tid % WAVE;
    const int nwaves = nthr / WAVE;
    const int ksl = wave % ks, rl = wave / ks;
    int tset = blockIdx.x, grp = 0;
    if (groups > 1) {
        const int nsets = gridDim.x / groups;
        if (nsets % 8 == 0) {
            const int j = blockIdx.x / 8;
            tset = (j / groups) * 8 + blockIdx.x % 8;
            grp = j % groups;
        } else {
            tset = blockIdx.x / groups;
            grp = blockIdx.x % groups;
        }
    }
    const int bg = (B + groups - 1) / groups;
    const int b0 = min(B, grp * bg), b1 = min(B, b0 + bg), nb = b1 - b0;  // this workgroup's sequences
    const int tile0 = tset * r_tiles;
    const int n0 = (tile0 + rl) * TILE_N;
    const int kb = ksl * kw;
    const int ke = min(K, kb + kw);
    const bool active = n0 < N && kb < K;
    const int nitems = r_tiles * TB;

    // ── loads issued up front ───────────────────────────────────────────────
    // X unit u (u < nb*K/8): sequence b0 + u / (K/8), k = 8 * (u % (K/8)), three planes.
    const int k8 = K / 8, nunits = nb * k8;
    u32x4 xu[XNT][3];
    auto load_units = [&](int u0) {
#pragma unroll
        for (int i = 0; i < XNT; ++i) {
            const int u = u0 + tid + i * nthr;
            if (u < nunits) {
                const int bl = u / k8, k = 8 * (u - bl * k8);
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    xu[i][q] =
                        *reinterpret_cast<const u32x4*>(p.xs + (int64_t)(q * DEC_MAX_BATCH + b0 + bl) * p.ldxs + k);
            }
        }
    };
    load_units(0);
    // A operand (W, stored in fragment order): lane l's 8 k of feature
    // n0 + l%16 at k block l/16 are 16 consecutive bytes, and the 64 lanes'
    // fragments of one 32-k step are 1 KB of consecutive memory.
    const int col = lane & 15, kg = lane >> 4;
    const uint16_t* wp = p.w + ((int64_t)(n0 / TILE_N) * (K / KSTEP) * WAVE + lane) * 8;
    u32x4 a[NS];
    auto load_pass = [&](int k0) {
        const int steps = active ? min(NS, (ke - k0) / KSTEP) : 0;
#pragma unroll
        for (int s = 0; s < NS; ++s)
            if (s < steps) a[s] = *reinterpret_cast<const u32x4*>(wp + (int64_t)(k0 / KSTEP + s) * WAVE * 8);
    };
    load_pass(kb);

    const int t = p.tctr ? *p.tctr : 0;
    float pre_bias[2] = {0.0f, 0.0f}, pre_res[2] = {0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int i = tid + e * nthr;
        if (i < nitems) {
            const int rr = i / TB, row = (i % TB) / DEC_MAX_BATCH, b = i % DEC_MAX_BATCH;
            const int n = (tile0 + rr) * TILE_N + row;
            if (n < N && b >= b0 && b < b1) {
                if (p.bias) pre_bias[e] = bf16_f32(p.bias[n]);
                if constexpr (EPI == DEC_EPI_RESID) pre_res[e] = p.out[(int64_t)b * p.ldo + n];
            }
        }
    }

    // ── X planes into LDS (and the squares of X) ───────────────────────────
    auto store_units = [&](int u0) {
#pragma unroll
        for (int i = 0; i < XNT; ++i) {
            const int u = u0 + tid + i * nthr;
            if (u < nunits) {
                const int bl = u / k8, c = u - bl * k8;
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    *reinterpret_cast<u32x4*>(xl + (q * DEC_MAX_BATCH + b0 + bl) * pitch + 8 * c) = xu[i][q];
                if constexpr (NORM) {
                    // rms_norm, cpu_kernels.rs:647-669: sqrt(sum(x*x)/d + eps), y = x / rms.
                    float ss = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int w32 = j / 2, sh = (j & 1) * 16;
                        const float x = bf16_f32((xu[i][0][w32] >> sh) & 0xFFFFu) +
                                        (bf16_f32((xu[i][1][w32] >> sh) & 0xFFFFu) +
                                         bf16_f32((xu[i][2][w32] >> sh) & 0xFFFFu));
                        ss += x * x;
                    }
                    psum[u] = ss;
                }
            }
        }
    };
    store_units(0);
    // Rows wider than XNT * nthr units (not met at decode sizes) take more rounds.
    for (int u0 = XNT * nthr; u0 < nunits; u0 += XNT * nthr) {
        load_units(u0);
        store_units(u0);
    }
    __syncthreads();
    if constexpr (NORM) {
        for (int bl = wave; bl < nb; bl += nwaves) {
            float ss = 0.0f;
            for (int c = lane; c < k8; c += WAVE) ss += psum[bl * k8 + c];
            ss = wave_sum(ss);
            if (lane == 0) {
                float rms = sqrtf(ss / (float)K + p.eps), r;
                shared_divisor(rms, r);
                wss[b0 + bl] = rms;
                wss[DEC_MAX_BATCH + b0 + bl] = r;
            }
        }
    }

    // ── main loop: 2 MFMAs per 16 features x 32 k ───────────────────────────
    // B operand (X) from LDS: lane l holds column l%16, k block l/16. Tile 0
    // column c is plane c/8 (hi, mid) of sequence c%8, tile 1 column c < 8
    // the lo plane of sequence c; columns 8..15 of tile 1 are zero.
    const uint16_t* x0 = xl + col * pitch + 8 * kg;
    const uint16_t* x1 = xl + (2 * DEC_MAX_BATCH + (col & 7)) * pitch + 8 * kg;
    const bool zero1 = col >= 8;
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    for (int k0 = kb; k0 < ke; k0 += KP) {
        if (k0 != kb) load_pass(k0);
        const int steps = active ? min(NS, (ke - k0) / KSTEP) : 0;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if (s < steps) {
                const int ko = k0 + s * KSTEP;
                const u32x4 b0 = *reinterpret_cast<const u32x4*>(x0 + ko);
                u32x4 b1 = *reinterpret_cast<const u32x4*>(x1 + ko);
                b1 = zero1 ? zero4 : b1;
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[s]),
                                                               __builtin_bit_cast(bf16x8, b0), acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[s]),
                                                               __builtin_bit_cast(bf16x8, b1), acc1, 0, 0, 0);
            }
        }
    }

    // D layout: lane l holds column l%16 and features 4*(l/16) + j, j < 4.
    // Column c < 8 of tile 0 is hi of sequence c, column c+8 its mid; column c
    // of tile 1 its lo.
    float* myred = red + (rl * ks + ksl) * TB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float mid = __shfl_xor(acc0[j], 8, WAVE);
        const float v = acc0[j] + (mid + acc1[j]);
        if (col < 8) myred[(4 * kg + j) * DEC_MAX_BATCH + col] = v;
    }
    __syncthreads();

    // ── epilogue: sum the k-slices in order, 1/rms, bias, then the op ──────
    // ARGMAX: the thread's items all belong to sequence tid % 8 (item i is
    // sequence i % 8, and nthr is a multiple of 8); kmax is their largest key.
    uint64_t kmax = 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int i = tid + e * nthr;
        if (i >= nitems) continue;
        const int rr = i / TB, ei = i % TB;
        const int row = ei / DEC_MAX_BATCH, b = ei % DEC_MAX_BATCH;
        const int n = (tile0 + rr) * TILE_N + row;
        float v = red[(rr * ks) * TB + ei];
        for (int s = 1; s < ks; ++s) v += red[(rr * ks + s) * TB + ei];
        const bool valid = n < N && b >= b0 && b < b1;
        if constexpr (NORM) {
            if (valid) v = div_by(v, wss[b], wss[DEC_MAX_BATCH + b]);
        }
        if (p.bias) v = v + pre_bias[e];
        if constexpr (EPI == DEC_EPI_SILU) {
            if (valid) {
                const float y = v * sigmoid_ref(v);
                if (p.out) p.out[(int64_t)b * p.ldo + n] = y;
                store_split(p.outs, p.ldos, b, n, y);
            }
        } else if constexpr (EPI == DEC_EPI_RESID) {
            if (valid) {
                const float y = pre_res[e] + v;
                p.out[(int64_t)b * p.ldo + n] = y;
                store_split(p.outs, p.ldos, b, n, y);
            }
        } else if constexpr (EPI == DEC_EPI_QKV) {
            if (valid) {
                const int d = p.dmodel, seg = n / d, nn = n - seg * d;
                const int h = nn / p.head_dim, dd = nn - h * p.head_dim;
                const int64_t bh = (int64_t)b * p.heads + h;
                if (seg == 0)
                    p.out[(int64_t)b * p.ldo + nn] = v;
                else if (seg == 1)
                    p.kc[(bh * p.head_dim + dd) * p.tmax + t] = v;  // K^T: [b][h][dd][pos]
                else
                    p.vc[(bh * p.tmax + t) * p.head_dim + dd] = v;  // V:   [b][h][pos][dd]
            }
        } else {  // DEC_EPI_ARGMAX
            if (valid && p.out) p.out[(int64_t)b * p.ldo + (int64_t)t * N + n] = v;
            const uint64_t key = valid ? ((uint64_t)order_key(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)n) : 0ull;
            kmax = key > kmax ? key : kmax;
        }
    }
    if constexpr (EPI == DEC_EPI_ARGMAX) {
        // Per sequence: across the wave's lanes of that sequence, then across
        // the waves (keys[w * 8 + b]); the maximum of the keys does not
        // depend on the order it is taken in.
        kmax = wave_max_u64_by8(kmax);
        if (lane < DEC_MAX_BATCH) keys[wave * DEC_MAX_BATCH + lane] = kmax;
        __syncthreads();
        if (tid < DEC_MAX_BATCH) {
            uint64_t m = 0;
            for (int w = 0; w < nwaves; ++w) m = keys[w * DEC_MAX_BATCH + tid] > m ? keys[w * DEC_MAX_BATCH + tid] : m;
            p.part[(int64_t)blockIdx.x * DEC_MAX_BATCH + tid] = m;
        }
    }
}

// ── end of the step: argmax, next token and its embedding, t += 1 ──────────
// One workgroup of 512 threads. Thread i reduces the keys of sequence i % 8
// from workgroups g = i/8, i/8 + 64, ... (all loaded before the first use),
// then lanes with equal i % 8 and the 8 waves combine theirs. Equal logits
// resolve to the lowest index (the key's low word is 0xFFFFFFFF - index). The
// next token is the prompt's while t+1 < prompt_len, else the argmax; its
// embedding row becomes the residual stream x (and its planes) of the next
// step, 8 values per thread and unit, every unit's load issued before the
// first store.
constexpr int FIN_BLOCK = DEC_MAX_BATCH * WAVE;
constexpr int FIN_KEYS = 8;  // keys per thread loaded at once
constexpr int FIN_UNITS = 4; // embedding units (8 bf16) per thread loaded at once

__global__ __launch_bounds__(FIN_BLOCK) void decode_finish_kernel(
    const uint64_t* __restrict__ part, int groups, int* __restrict__ tokens, int* __restrict__ argmax_out,
    const uint16_t* __restrict__ emb, float* __restrict__ x, uint16_t* __restrict__ xs, int d, int vocab,
    int batch, int prompt_len, int* __restrict__ tctr) {
    __shared__ uint64_t s_max[FIN_BLOCK / WAVE][DEC_MAX_BATCH];
    __shared__ int s_tok[DEC_MAX_BATCH];
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int b = tid % DEC_MAX_BATCH;
    constexpr int GSTRIDE = FIN_BLOCK / DEC_MAX_BATCH;
    const int t = *tctr;
    uint64_t m = 0;
    for (int g0 = tid / DEC_MAX_BATCH; g0 < groups; g0 += GSTRIDE * FIN_KEYS) {
        uint64_t k[FIN_KEYS];
#pragma unroll
        for (int j = 0; j < FIN_KEYS; ++j) {
            const int g = g0 + j * GSTRIDE;
            k[j] = g < groups ? part[(int64_t)g * DEC_MAX_BATCH + b] : 0ull;
        }
#pragma unroll
        for (int j = 0; j < FIN_KEYS; ++j) m = k[j] > m ? k[j] : m;
    }
#pragma unroll
    for (int o = 8; o < WAVE; o <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)m, o, WAVE);
        const uint32_t hi = __shfl_xor((uint32_t)(m >> 32), o, WAVE);
        const uint64_t w = ((uint64_t)hi << 32) | lo;
        m = w > m ? w : m;
    }
    if (lane < DEC_MAX_BATCH) s_max[wave][lane] = m;
    __syncthreads();
    if (tid < batch) {
        uint64_t mm = s_max[0][tid];
#pragma unroll
        for (int w = 1; w < FIN_BLOCK / WAVE; ++w) mm = s_max[w][tid] > mm ? s_max[w][tid] : mm;
        const int idx = (int)(0xFFFFFFFFu - (uint32_t)mm);
        argmax_out[(int64_t)t * batch + tid] = idx;
        int next = idx;
        if (t + 1 < prompt_len)
            next = tokens[(int64_t)(t + 1) * batch + tid];
        else
            tokens[(int64_t)(t + 1) * batch + tid] = idx;
        s_tok[tid] = next < 0 ? 0 : (next > vocab - 1 ? vocab - 1 : next);
    }
    __syncthreads();
    const int d8 = d / 8, units = batch * d8;
    for (int u0 = tid; u0 < units; u0 += FIN_UNITS * FIN_BLOCK) {
        uint4 e[FIN_UNITS];
#pragma unroll
        for (int j = 0; j < FIN_UNITS; ++j) {
            const int u = u0 + j * FIN_BLOCK;
            if (u < units) {
                const int bb = u / d8;
                e[j] = *reinterpret_cast<const uint4*>(emb + (int64_t)s_tok[bb] * d + 8 * (u - bb * d8));
            }
        }
#pragma unroll
        for (int j = 0; j < FIN_UNITS; ++j) {
            const int u = u0 + j * FIN_BLOCK;
            if (u < units) {
                const int bb = u / d8;
                store_embedding_unit(e[j], x, xs, d, bb, 8 * (u - bb * d8));
            }
        }
    }
    if (tid == 0) *tctr = t + 1;
}

// ── attention of one new query per (sequence, head) over the KV cache ────
//
// Block = 256 threads for one (b, h). Scores s_j = (q·k_j)·scale summed over
// the head dimension in order (as cpu_matmul_raw), softmax as
// cpu_kernels.rs:790-806 (max, exp(x - max), sum, divide), o = sum_j p_j v_j.
// The cache is K^T [hd][tmax] (thread j reads column j: consecutive threads,
// consecutive addresses) and V [tmax][hd] (a thread reads float4s of a row).
// The V rows of the P·V phase and the K columns of the thread's first
// position are loaded before anything is used and q (the same for the whole
// block) through the scalar cache, so the loads cost about one memory round
// trip. Each wave takes exp(s_j - m_w) against its own maximum m_w and sums
// them; one exchange of the waves' (m_w, l_w) gives the block maximum m and
// the sum l = sum_w l_w e^(m_w - m); the P·V phase accumulates
// e_j e^(m_w - m) v_j and divides by l at the end. Two barriers in all.
constexpr int ATT_BLOCK = 256;
constexpr int ATT_WAVES = ATT_BLOCK / WAVE;

// v[w] of (v0, v1, v2, v3) by value selects on the bits of w (0 <= w < 4).
__device__ inline float pick4(int w, float v0, float v1, float v2, float v3) {
    const float lo = (w & 1) ? v1 : v0;
    const float hi = (w & 1) ? v3 : v2;
    return (w & 2) ? hi : lo;
}

template <int HD>
__global__ __launch_bounds__(ATT_BLOCK) void decode_attn_kernel(const float* __restrict__ q,
                                                                const float* __restrict__ kc,
                                                                const float* __restrict__ vc,
                                                                uint16_t* __restrict__ os, int heads,
                                                                int tmax, float scale,
                                                                const int* __restrict__ tctr) {
    constexpr int C4 = HD / 4, G = ATT_BLOCK / C4, VCH = 16;
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* s = sm;                  // [tmax] scores
    float* part = s + ((tmax + 3) & ~3);  // [G][HD] P·V partials (16-byte aligned)
    float* slot = part + G * HD;    // [ATT_WAVES][2] (max, sum) of each wave
    const int bh = blockIdx.x, b = bh / heads, h = bh % heads;
    const int d = heads * HD;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const float* kT = kc + (int64_t)bh * HD * tmax;
    const float* vv = vc + (int64_t)bh * tmax * HD;
    const float* qp = q + (int64_t)b * d + h * HD;
    const int T = *tctr + 1;

    // P·V mapping: thread (c, g) owns columns 4c..4c+3 over positions
    // j = g (mod G). Its first VCH rows of V are loaded first. Rows past the
    // last position load row T-1 instead (no branch around the loads, which
    // would make the compiler wait for each one) and get probability 0.
    const int c = tid % C4, g = tid / C4;
    float4 vr[VCH];
#pragma unroll
    for (int u = 0; u < VCH; ++u) {
        const int j = min(g + u * G, T - 1);
        vr[u] = *reinterpret_cast<const float4*>(vv + (int64_t)j * HD + 4 * c);
    }

    // Scores of positions j = tid (mod 256), K loaded KCH values at a time.
    constexpr int KCH = HD < 64 ? HD : 64;
    float mloc = -INFINITY;
    for (int j = tid; j < T; j += ATT_BLOCK) {
        float acc = 0.0f;
#pragma unroll
        for (int d0 = 0; d0 < HD; d0 += KCH) {
            float kv[KCH];
#pragma unroll
            for (int u = 0; u < KCH; ++u) kv[u] = kT[(int64_t)(d0 + u) * tmax + j];
#pragma unroll
            for (int u = 0; u < KCH; ++u) acc += qp[d0 + u] * kv[u];
        }
        const float sc = acc * scale;
        s[j] = sc;
        mloc = fmaxf(mloc, sc);
    }
    // e_j = exp(s_j - m_w) against the maximum m_w of the wave that owns
    // position j (wave (j % 256) / 64), and the wave's sum l_w of them.
    const float mw = wave_max(mloc);
    float lloc = 0.0f;
    for (int j = tid; j < T; j += ATT_BLOCK) {
        const float e = expf(s[j] - mw);
        s[j] = e;
        lloc += e;
    }
    const float lw = wave_sum(lloc);
    if (lane == 0) {
        slot[2 * wave] = mw;
        slot[2 * wave + 1] = lw;
    }
    __syncthreads();  // e_j and the waves' (max, sum)
    // Block maximum m, factors f_w = exp(m_w - m) (0 for a wave without
    // positions), sum l = sum_w l_w f_w.
    float m = slot[0];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; ++w) m = fmaxf(m, slot[2 * w]);
    static_assert(ATT_WAVES == 4, "four wave factors");
    auto wave_factor = [&](int w) { return slot[2 * w] == -INFINITY ? 0.0f : expf(slot[2 * w] - m); };
    const float f0 = wave_factor(0), f1 = wave_factor(1), f2 = wave_factor(2), f3 = wave_factor(3);
    const float l = ((slot[1] * f0 + slot[3] * f1) + slot[5] * f2) + slot[7] * f3;
    // The factor of position j is wave ((j >> 6) & 3)'s, selected from four
    // values (a select over an array, or over references to the four, is
    // compiled to an indexed load from scratch memory).
    auto factor = [f0, f1, f2, f3](int w) { return pick4(w, f0, f1, f2, f3); };
    auto prob = [&](int j) { return j < T ? s[j] * factor((j >> 6) & 3) : 0.0f; };
    // In the first VCH rows, j = g + u*G with g < G: for G <= 64 (a power of
    // two, so g + (u*G mod 64) < 64) the wave of j is that of u*G, known at
    // compile time.
    auto prob_first = [&](int u) {
        const int j = g + u * G;
        const int w = G <= 64 ? ((u * G) >> 6) & 3 : (j >> 6) & 3;
        return j < T ? s[j] * factor(w) : 0.0f;
    };

    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int u = 0; u < VCH; ++u) {
        const float pj = prob_first(u);
        acc.x += pj * vr[u].x;
        acc.y += pj * vr[u].y;
        acc.z += pj * vr[u].z;
        acc.w += pj * vr[u].w;
    }
    for (int j0 = g + VCH * G; j0 < T; j0 += G * VCH) {
#pragma unroll
        for (int u = 0; u < VCH; ++u) {
            const int j = min(j0 + u * G, T - 1);
            vr[u] = *reinterpret_cast<const float4*>(vv + (int64_t)j * HD + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < VCH; ++u) {
            const float pj = prob(j0 + u * G);
            acc.x += pj * vr[u].x;
            acc.y += pj * vr[u].y;
            acc.z += pj * vr[u].z;
            acc.w += pj * vr[u].w;
        }
    }
    *reinterpret_cast<float4*>(part + g * HD + 4 * c) = acc;
    __syncthreads();
    if (tid < HD) {
        float r = part[tid];
        for (int gg = 1; gg < G; ++gg) r += part[gg * HD + tid];
        store_split(os, d, b, h * HD + tid, r / l);
    }
}

// ── embedding of the step's tokens (x and its planes) ──────────────────────
__global__ __launch_bounds__(256) void decode_embed_kernel(const uint16_t* __restrict__ emb,
                                                           const int* __restrict__ tokens,
                                                           float* __restrict__ x, uint16_t* __restrict__ xs,
                                                           int d, int vocab, int batch,
                                                           const int* __restrict__ tctr) {
    const int b = blockIdx.x;
    const int t = *tctr;
    int tok = tokens[(int64_t)t * batch + b];
    tok = tok < 0 ? 0 : (tok > vocab - 1 ? vocab - 1 : tok);
    const uint16_t* src = emb + (int64_t)tok * d;
    for (int u = threadIdx.x; u < d / 8; u += blockDim.x)
        store_embedding_unit(*reinterpret_cast<const uint4*>(src + 8 * u), x, xs, d, b, 8 * u);
}

__global__ void decode_set_kernel(int* __restrict__ p, int v) { *p = v; }

// Launch shape: a problem with fewer than 512 row tiles gives each
// workgroup one row tile and splits K into slices of ~64 (up to 16 waves),
// so its W and X loads spread over many waves. The LM head (ARGMAX with 512
// or more row tiles) gives each wave a whole row tile over all of K in one
// pass and each workgroup up to 8 row tiles, keeping at least 256
// workgroups when that leaves a whole one-round grid: with the 1024-thread
// shape it had before (4 k-slices x 4 row tiles, 500 workgroups for a
// 32000-word vocabulary) its registers allowed one workgroup per CU, so the
// launch ran in two rounds. MLXHIP_DEC_WIDE="ks,r" overrides the wide shape
// (tuning; ks > 1 or r * ks > 8 takes the 1024-thread kernel).
//
// K is not split across workgroups: adding partial sums of several
// workgroups takes a device-scope fence per workgroup (an L2 write-back and
// invalidate of its XCD), measured at 15-20 us per launch over 300-400
// workgroups of a decode step, where a whole GEMV takes 5-12 us.
struct GemvShape {
    int ks, r, kw, grid;
    bool wide;   // the WIDE_NSTEP kernel
    int groups;  // batch groups (workgroups per row-tile set)
};

// MI355X's CU count: the batch is split while the launch still fits one
// workgroup per CU (a shape choice only; results do not depend on it).
constexpr int DEC_CUS = 256;

GemvShape gemv_shape(int n, int k, bool argmax, int batch) {
    GemvShape g{1, 1, 0, 0, false, 1};
    const int ntiles = (int)ceil_div(n, TILE_N);
    if (argmax && ntiles >= 512) {
        g.ks = 1;
        g.r = WIDE_WAVES;
        static const char* env = std::getenv("MLXHIP_DEC_WIDE");
        int eks = 0, er = 0;
        if (env && std::sscanf(env, "%d,%d", &eks, &er) == 2 && eks >= 1 && er >= 1 && eks * er <= MAX_WAVES) {
            g.ks = eks;
            g.r = er;
        }
        g.wide = g.ks == 1 && g.r <= WIDE_WAVES;
    } else {
        g.ks = std::max(1, std::min(MAX_WAVES, (int)ceil_div(k, 64)));
    }
    g.kw = (int)ceil_div(ceil_div(k, g.ks), KSTEP) * KSTEP;
    const int sets = (int)ceil_div(ntiles, g.r);
    if (!argmax) {
        static const char* genv = std::getenv("MLXHIP_DEC_GROUPS");
        const int want = genv ? std::atoi(genv) : 0;
        if (want >= 1) {
            g.groups = want;
        } else {
            while (g.groups * 2 <= DEC_MAX_BATCH && sets * g.groups * 2 <= DEC_CUS) g.groups *= 2;
        }
        // No empty group: groups = ceil(batch / ceil(batch / groups)).
        g.groups = std::max(1, std::min(g.groups, batch));
        g.groups = (int)ceil_div(batch, ceil_div(batch, g.groups));
    }
    g.grid = sets * g.groups;
    return g;
}

template <int EPI, bool NORM>
int launch_gemv(const DecGemv& p, hipStream_t s) {
    const GemvShape g = gemv_shape(p.n, p.k, EPI == DEC_EPI_ARGMAX, p.batch);
    const size_t lds = dec_gemv_lds_bytes(p.k, g.ks, g.r, EPI == DEC_EPI_ARGMAX, NORM);
    if (lds > DEC_LDS_LIMIT)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode gemv: K = %d needs %zu bytes of LDS (limit %d)", p.k,
                    lds, DEC_LDS_LIMIT);
    if (EPI == DEC_EPI_ARGMAX && g.grid > p.part_capacity)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode gemv: %d workgroups exceed the partial-max buffer (%d)",
                    g.grid, p.part_capacity);
    if constexpr (EPI == DEC_EPI_ARGMAX) {
        if (g.wide) {
            hipLaunchKernelGGL((gemv_kernel<EPI, NORM, WIDE_NSTEP, WIDE_XN>), dim3(g.grid), dim3(g.r * WAVE), lds, s,
                               p, g.ks, g.r, g.kw, g.groups);
            return launch_check("decode gemv_kernel (wide)");
        }
    }
    hipLaunchKernelGGL((gemv_kernel<EPI, NORM>), dim3(g.grid), dim3(g.r * g.ks * WAVE), lds, s, p, g.ks, g.r, g.kw,
                       g.groups);
    return launch_check("decode gemv_kernel");
}

template <int EPI, bool NORM, int NS = NSTEP, int XNT = XN>
int set_lds_attr() {
    MLXHIP_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<EPI, NORM, NS, XNT>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, DEC_LDS_LIMIT));
    return MLXHIP_OK;
}

}  // namespace

size_t dec_gemv_lds_bytes(int k, int ks, int r, bool argmax, bool norm) {
    size_t b = (size_t)XROWS * (k + XPAD) * 2;                           // X planes
    b += (size_t)r * ks * TILE_N * DEC_MAX_BATCH * sizeof(float);        // k-slice partials
    b += WSS_FLOATS * sizeof(float);                                     // row rms and 1 / rms
    if (argmax) b += (size_t)r * TILE_N * DEC_MAX_BATCH * sizeof(uint64_t);
    if (norm) b += (size_t)DEC_MAX_BATCH * (k / 8) * sizeof(float);      // squares of the X units
    return b;
}

int dec_gemv_groups(int n, int k) { return gemv_shape(n, k, true, DEC_MAX_BATCH).grid; }

size_t dec_tiled_index(int64_t n, int64_t k, int64_t K) {
    const int64_t tile = n / TILE_N, step = k / KSTEP;
    const int64_t lane = (n % TILE_N) + TILE_N * ((k % KSTEP) / 8);
    return (size_t)(((tile * (K / KSTEP) + step) * WAVE + lane) * 8 + k % 8);
}

int dec_prepare() {
    MLXHIP_TRY((set_lds_attr<DEC_EPI_QKV, true>()));
    MLXHIP_TRY((set_lds_attr<DEC_EPI_RESID, false>()));
    MLXHIP_TRY((set_lds_attr<DEC_EPI_SILU, true>()));
    MLXHIP_TRY((set_lds_attr<DEC_EPI_ARGMAX, true>()));
    MLXHIP_TRY((set_lds_attr<DEC_EPI_ARGMAX, true, WIDE_NSTEP, WIDE_XN>()));
    return MLXHIP_OK;
}

int dec_gemv(int epi, bool norm, const DecGemv& p, hipStream_t s) {
    if (p.k <= 0 || p.k % KSTEP || p.n <= 0 || p.batch <= 0 || p.batch > DEC_MAX_BATCH || p.ldxs % 8 ||
        p.ldxs < p.k || !p.xs)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode gemv: unsupported shape n=%d k=%d batch=%d", p.n, p.k,
                    p.batch);
    if ((epi == DEC_EPI_RESID || epi == DEC_EPI_SILU) && (!p.outs || p.ldos < p.n))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode gemv: epilogue %d needs the output planes", epi);
    if (epi == DEC_EPI_QKV && norm) return launch_gemv<DEC_EPI_QKV, true>(p, s);
    if (epi == DEC_EPI_RESID && !norm) return launch_gemv<DEC_EPI_RESID, false>(p, s);
    if (epi == DEC_EPI_SILU && norm) return launch_gemv<DEC_EPI_SILU, true>(p, s);
    if (epi == DEC_EPI_ARGMAX && norm) return launch_gemv<DEC_EPI_ARGMAX, true>(p, s);
    return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode gemv: no kernel for epilogue %d (norm=%d)", epi, (int)norm);
}

size_t dec_attn_lds_bytes(int hd, int tmax) {
    const size_t g = ATT_BLOCK / (hd / 4);  // P·V position groups
    return ((size_t)ceil_div(tmax, 4) * 4 + g * hd + 2 * ATT_WAVES) * sizeof(float);
}

int dec_attention(const float* q, const float* kc, const float* vc, uint16_t* os, int batch, int heads, int hd,
                  int tmax, float scale, const int* tctr, hipStream_t s) {
    if (batch <= 0 || heads <= 0 || tmax <= 0)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode attention: empty problem");
    const size_t lds = dec_attn_lds_bytes(hd, tmax);
    if (lds > 64 * 1024) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode attention: max_seq %d too long", tmax);
    const dim3 grid(batch * heads), block(ATT_BLOCK);
    switch (hd) {
        case 8: hipLaunchKernelGGL(decode_attn_kernel<8>, grid, block, lds, s, q, kc, vc, os, heads, tmax, scale, tctr); break;
        case 16: hipLaunchKernelGGL(decode_attn_kernel<16>, grid, block, lds, s, q, kc, vc, os, heads, tmax, scale, tctr); break;
        case 32: hipLaunchKernelGGL(decode_attn_kernel<32>, grid, block, lds, s, q, kc, vc, os, heads, tmax, scale, tctr); break;
        case 64: hipLaunchKernelGGL(decode_attn_kernel<64>, grid, block, lds, s, q, kc, vc, os, heads, tmax, scale, tctr); break;
        case 128: hipLaunchKernelGGL(decode_attn_kernel<128>, grid, block, lds, s, q, kc, vc, os, heads, tmax, scale, tctr); break;
        case 256: hipLaunchKernelGGL(decode_attn_kernel<256>, grid, block, lds, s, q, kc, vc, os, heads, tmax, scale, tctr); break;
        default: return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode attention: head_dim %d not in {8, 16, ..., 256}", hd);
    }
    return launch_check("decode_attn_kernel");
}

int dec_embed(const uint16_t* emb, const int* tokens, float* x, uint16_t* xs, int d, int vocab, int batch,
              const int* tctr, hipStream_t s) {
    if (d % 8) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode embed: d_model %d is not a multiple of 8", d);
    hipLaunchKernelGGL(decode_embed_kernel, dim3(batch), dim3(256), 0, s, emb, tokens, x, xs, d, vocab, batch, tctr);
    return launch_check("decode_embed_kernel");
}

int dec_finish(const uint64_t* part, int groups, int* tokens, int* argmax_out, const uint16_t* emb, float* x,
               uint16_t* xs, int d, int vocab, int batch, int prompt_len, int* tctr, hipStream_t s) {
    if (batch <= 0 || batch > DEC_MAX_BATCH)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode finish: batch %d outside [1, %d]", batch, DEC_MAX_BATCH);
    if (d % 8) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decode finish: d_model %d is not a multiple of 8", d);
    hipLaunchKernelGGL(decode_finish_kernel, dim3(1), dim3(FIN_BLOCK), 0, s, part, groups, tokens, argmax_out, emb,
                       x, xs, d, vocab, batch, prompt_len, tctr);
    return launch_check("decode_finish_kernel");
}

int dec_set_counter(int* p, int v, hipStream_t s) {
    hipLaunchKernelGGL(decode_set_kernel, dim3(1), dim3(1), 0, s, p, v);
    return launch_check("decode_set_kernel");
}

}  // namespace mlxhip
