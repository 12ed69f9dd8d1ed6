// attention.hip — fused scaled, masked attention for a batch of heads:
//   O_b = softmax(Q_b K_b^T * scale, causal) V_b,  Q_b [tq, dh], K_b, V_b [tk, dh]
// with the arithmetic of cpu_attention (crates/mlx-core/src/cpu_kernels.rs:
// 738-812): scores = (q . k) * scale, the causal entries j > i excluded (the
// reference writes -1e9 there, whose exp is 0 next to any finite score),
// softmax over the row, then P V.
//
// Streaming form. Queries are cut into blocks of 32 rows; a 256-thread
// workgroup owns one pair of blocks (b, nblk-1-b), so that under the causal
// mask every workgroup has the same number of key tiles, and processes them
// one after the other. Within a block, wave (g, h) owns rows 16g .. 16g+15
// and the key tiles of parity h (tiles of 32 keys, two per iteration, staged
// through LDS; the next pair is loaded into registers while the current one
// is computed). Per tile, a wave:
//   1. S^T = K Q^T on v_mfma_f32_16x16x4f32, A = 16 key rows from LDS, B = its
//      16 query rows held in registers; then * scale. The head-dimension
//      index is permuted (lane group g covers columns g*dh/4 .. g*dh/4 +
//      dh/4 - 1, MFMA step s picks one of them) so each lane reads contiguous
//      floats. Lane (i, g) then holds 8 scores of query row i: keys 16x +
//      4g + r of the tile.
//   2. Online softmax per row: running max m and running sum l of
//      exp(s - m); when the max grows, l and the output row are rescaled by
//      exp(m_old - m_new). The row's max and sum over its four lane groups use
//      the gfx950 lane-swap instructions (v_permlane16/32_swap). exp(d) is
//      computed as 2^(d * log2 e) on the subtracted, small argument d.
//   3. O^T += V^T P^T on the same MFMA: A = V^T from LDS, B = P^T straight
//      from the score registers (MFMA step r takes keys {4g + r}). The O^T
//      accumulator keeps lane (i, g) on query row i (output columns 16c + 4g +
//      r), so the rescaling and the final division need no lane exchange.
// The two waves of a row group then merge their (m, l, O) through LDS in a
// fixed order and divide by l. The reference takes the whole row's max first
// and divides every probability before P V; the orders differ by rounding
// only. Masks are applied only on tiles that cross tk or the causal diagonal.
// Workgroups are numbered so that the blocks of one head run on one XCD and
// share its L2.
#include <algorithm>

#include "../common.hpp"
#include "../kernels.hpp"
#include "device_math.hpp"

#pragma clang fp contract(off)

namespace mlxhip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr int ATT_THREADS = 4 * WAVE;
constexpr int QB = 32;  // query rows per block (two row groups of 16)
constexpr int KT = 32;  // keys per tile; a wave pair takes two tiles per iteration
constexpr int XCDS = 8;
constexpr float LOG2E = 1.44269504088896340736f;

using dev::div_by;
using dev::shared_divisor;

// Max and sum over the four 16-lane rows of the wave, lane by lane (lanes l,
// l ^ 16, l ^ 32, l ^ 48): one v_permlane16_swap and one v_permlane32_swap.
// Every lane gets the same bits (rows 0 and 1 are combined first, in that
// operand order, then rows 0-1 with rows 2-3).
__device__ inline float lanes_max(float x) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const unsigned w = __float_as_uint(x);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float lanes_sum(float x) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const unsigned w = __float_as_uint(x);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int DH>
struct Tile {
    // LDS row pitch (floats) of the K and V tiles. DH + 4: the float4 reads
    // of 16 consecutive key rows (step 1) and the column reads of keys
    // 4g + r (step 3) fall on distinct banks.
    static constexpr int P = DH + 4;
    static constexpr int FLOATS = KT * P;       // one K or V tile
    static constexpr int STAGE = 4 * FLOATS;    // K0 V0 K1 V1
    static constexpr int STAGES = DH <= 64 ? 2 : 1;  // two stages (and a register prefetch) up to dh 64
    static constexpr int F4 = KT * DH / 4;      // float4 of one tile
    static constexpr int LD4 = 2 * F4 / ATT_THREADS;  // float4 of K (and of V) per thread and iteration
    static_assert(2 * F4 % ATT_THREADS == 0, "tile pair must split evenly over the threads");
    static constexpr int CT = DH / 16;          // 16-column output tiles
    static constexpr int MERGE = 2 * WAVE * (4 * CT + 2);  // floats of the wave-pair merge
    static_assert(MERGE <= STAGE, "merge area must fit in one stage");
};

template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void attn_fused_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ v,
                                                                 float* __restrict__ o, int tq, int tk,
                                                                 int64_t sq, int64_t sk, int64_t sv,
                                                                 int64_t so, float scale, int causal,
                                                                 int npairs, int nblk) {
    using T = Tile<DH>;
    constexpr int DQ = DH / 4;  // head columns per lane group
    constexpr int CT = T::CT;
    __shared__ __attribute__((aligned(16))) float lds[T::STAGES * T::STAGE];

    // Workgroup -> (head, block pair). Consecutive workgroups go to
    // different XCDs; this numbering gives each XCD a contiguous range of
    // heads, so a head's K and V are fetched into one L2.
    const unsigned L = blockIdx.x, N = gridDim.x;
    const unsigned logical = N % XCDS == 0 ? (L % XCDS) * (N / XCDS) + L / XCDS : L;
    const int bh = (int)(logical / (unsigned)npairs), pair = (int)(logical % (unsigned)npairs);
    q += bh * sq;
    k += bh * sk;
    v += bh * sv;
    o += bh * so;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int li = lane & 15, lg = lane >> 4;
    const int g = wave & 1, h = wave >> 1;

    // Tile-pair loads: float4 f = tid + j*256 of an iteration is tile f / F4
    // of the pair, key row (f % F4) / (DH/4), columns 4 * (f % (DH/4)).
    // Loads are unconditional (keys clamped to tk - 1) and go straight into
    // registers; rows past tk are zeroed when stored (their scores are
    // masked, and 0 * V must not meet a non-finite V).
    int lkey[T::LD4], lcol[T::LD4], lat[T::LD4];
#pragma unroll
    for (int j = 0; j < T::LD4; ++j) {
        const int f = tid + j * ATT_THREADS;
        const int sub = f / T::F4, row = (f % T::F4) / (DH / 4);
        lkey[j] = sub * KT + row;
        lcol[j] = 4 * (f % (DH / 4));
        lat[j] = sub * 2 * T::FLOATS + row * T::P + lcol[j];
    }
    float4 kr[T::LD4], vr[T::LD4];
#define ATT_LOAD(it)                                                                  \
    do {                                                                              \
        const int kb_ = (it) * 2 * KT;                                                \
        _Pragma("unroll") for (int j = 0; j < T::LD4; ++j) {                          \
            const int64_t o_ = (int64_t)min(kb_ + lkey[j], tk - 1) * DH + lcol[j];    \
            kr[j] = *reinterpret_cast<const float4*>(k + o_);                         \
            vr[j] = *reinterpret_cast<const float4*>(v + o_);                         \
        }                                                                             \
    } while (0)
#define ATT_STORE(stage, it)                                                          \
    do {                                                                              \
        float* st_ = lds + (stage) * T::STAGE;                                        \
        _Pragma("unroll") for (int j = 0; j < T::LD4; ++j) {                          \
            const bool in_ = (it) * 2 * KT + lkey[j] < tk;                            \
            float4 w_;                                                                \
            w_.x = in_ ? vr[j].x : 0.0f;                                              \
            w_.y = in_ ? vr[j].y : 0.0f;                                              \
            w_.z = in_ ? vr[j].z : 0.0f;                                              \
            w_.w = in_ ? vr[j].w : 0.0f;                                              \
            *reinterpret_cast<float4*>(st_ + lat[j]) = kr[j];                         \
            *reinterpret_cast<float4*>(st_ + T::FLOATS + lat[j]) = w_;                \
        }                                                                             \
    } while (0)

    for (int bi = 0; bi < 2; ++bi) {
        const int blk = bi == 0 ? pair : nblk - 1 - pair;
        if (bi == 1 && blk == pair) break;  // the middle block of an odd count
        const int q0 = blk * QB, qw = q0 + 16 * g;
        const int kend = causal ? min(tk, q0 + QB) : tk;  // keys any row of the block sees
        const int niter = (kend + 2 * KT - 1) / (2 * KT);

        // This wave's query rows as B operands: lane holds row qw + li, columns lg*DQ + s.
        float qf[DQ];
        {
            const float* qr = q + (int64_t)min(qw + li, tq - 1) * DH + lg * DQ;
#pragma unroll
            for (int s = 0; s < DQ; s += 4) {
                const float4 t = *reinterpret_cast<const float4*>(qr + s);
                qf[s] = t.x; qf[s + 1] = t.y; qf[s + 2] = t.z; qf[s + 3] = t.w;
            }
        }
        float m_run = -INFINITY, l_run = 0.0f;  // of row qw + li (the 4 lane groups agree)
        f32x4 acc[CT];                          // O row qw + li, columns 16c + 4lg + r
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        // Tile t (this wave's half of an iteration) from LDS stage `stage`.
        // Tiles past the block's keys are fully masked and leave the state
        // unchanged.
        auto tile = [&](int t, int stage) {
            const float* ks = lds + stage * T::STAGE + h * 2 * T::FLOATS;
            const float* vs = ks + T::FLOATS;
            // 1. S^T of the two 16-key halves, their MFMA chains interleaved.
            f32x4 sa[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
            for (int s = 0; s < DQ; s += 4) {
                float4 kk[2];
#pragma unroll
                for (int x = 0; x < 2; ++x)
                    kk[x] = *reinterpret_cast<const float4*>(ks + (16 * x + li) * T::P + lg * DQ + s);
#pragma unroll
                for (int x = 0; x < 2; ++x) sa[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[x].x, qf[s], sa[x], 0, 0, 0);
#pragma unroll
                for (int x = 0; x < 2; ++x) sa[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[x].y, qf[s + 1], sa[x], 0, 0, 0);
#pragma unroll
                for (int x = 0; x < 2; ++x) sa[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[x].z, qf[s + 2], sa[x], 0, 0, 0);
#pragma unroll
                for (int x = 0; x < 2; ++x) sa[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[x].w, qf[s + 3], sa[x], 0, 0, 0);
            }
            float p[2][4];
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int r = 0; r < 4; ++r) p[x][r] = sa[x][r] * scale;
            // Keys past tk, or past a row's causal horizon, get -inf (weight 0).
            const int kt1 = (t + 1) * KT;
            if (kt1 > tk || (causal && kt1 - 1 > qw)) {
#pragma unroll
                for (int x = 0; x < 2; ++x)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = t * KT + 16 * x + 4 * lg + r;
                        if (key >= tk || (causal && key > qw + li)) p[x][r] = -INFINITY;
                    }
            }
            // 2. online softmax over the row's 32 keys of this tile (8 here,
            // 24 in the lanes 16, 32 and 48 apart).
            float mt = fmaxf(fmaxf(fmaxf(p[0][0], p[0][1]), fmaxf(p[0][2], p[0][3])),
                             fmaxf(fmaxf(p[1][0], p[1][1]), fmaxf(p[1][2], p[1][3])));
            mt = lanes_max(mt);
            const float m_new = fmaxf(m_run, mt);
            // m_new stays -inf while every key seen so far is masked: then
            // every weight is 0 and the state is untouched.
            const float m_sub = m_new == -INFINITY ? 0.0f : m_new;
            const float corr = __builtin_amdgcn_exp2f((m_run - m_sub) * LOG2E);
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int r = 0; r < 4; ++r) p[x][r] = __builtin_amdgcn_exp2f((p[x][r] - m_sub) * LOG2E);
            float ps = ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) + ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
            ps = lanes_sum(ps);
            l_run = l_run * corr + ps;
            m_run = m_new;
            // 3. O^T = O^T * corr + V^T P^T.
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[c][r] *= corr;
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float* vp = vs + (16 * x + 4 * lg + r) * T::P + li;
#pragma unroll
                    for (int c = 0; c < CT; ++c)
                        acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vp[16 * c], p[x][r], acc[c], 0, 0, 0);
                }
        };

        ATT_LOAD(0);
        ATT_STORE(0, 0);
        __syncthreads();
        for (int it = 0; it + 1 < niter; ++it) {
            if constexpr (T::STAGES == 2) {
                ATT_LOAD(it + 1);
                __builtin_amdgcn_sched_barrier(0);  // the scheduler would otherwise move the loads after the MFMAs
                tile(2 * it + h, it & 1);
                ATT_STORE((it + 1) & 1, it + 1);
            } else {
                // One stage, and no registers to spare for a prefetch: the
                // other workgroup on the CU covers the load latency.
                tile(2 * it + h, 0);
                __syncthreads();
                ATT_LOAD(it + 1);
                ATT_STORE(0, it + 1);
            }
            __syncthreads();
        }
        tile(2 * (niter - 1) + h, (niter - 1) % T::STAGES);
        __syncthreads();  // every wave is done with the stages: the merge area aliases them

        // Merge the wave pair (g, 1) into (g, 0): m = max, weights 2^((m_x - m) log2 e).
        float* mg = lds + g * WAVE * (4 * CT + 2) + lane * (4 * CT + 2);
        if (h == 1) {
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) mg[4 * c + r] = acc[c][r];
            mg[4 * CT] = m_run;
            mg[4 * CT + 1] = l_run;
        }
        __syncthreads();
        if (h == 0) {
            const float m1 = mg[4 * CT], l1 = mg[4 * CT + 1];
            const float m = fmaxf(m_run, m1);  // finite: tile 0 holds key 0, which every row sees
            const float a0 = __builtin_amdgcn_exp2f((m_run - m) * LOG2E);
            const float a1 = __builtin_amdgcn_exp2f((m1 - m) * LOG2E);
            float l = l_run * a0 + l1 * a1, rl;
            shared_divisor(l, rl);
            const int row = qw + li;
            if (row < tq) {
                float* orow = o + (int64_t)row * DH + 4 * lg;
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    float4 w;
                    w.x = div_by(acc[c][0] * a0 + mg[4 * c + 0] * a1, l, rl);
                    w.y = div_by(acc[c][1] * a0 + mg[4 * c + 1] * a1, l, rl);
                    w.z = div_by(acc[c][2] * a0 + mg[4 * c + 2] * a1, l, rl);
                    w.w = div_by(acc[c][3] * a0 + mg[4 * c + 3] * a1, l, rl);
                    *reinterpret_cast<float4*>(orow + 16 * c) = w;
                }
            }
        }
        __syncthreads();  // the next block's first tiles overwrite the merge area
    }
#undef ATT_LOAD
#undef ATT_STORE
}

int64_t blocks_of(int64_t tq) { return (tq + QB - 1) / QB; }
int64_t pairs_of(int64_t tq) { return (blocks_of(tq) + 1) / 2; }

template <int DH>
int launch(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq, int64_t tk,
           int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale, int causal, hipStream_t s) {
    const int64_t npairs = pairs_of(tq);
    const dim3 grid((unsigned)(npairs * batch));
    hipLaunchKernelGGL(attn_fused_kernel<DH>, grid, dim3(ATT_THREADS), 0, s, q, k, v, o, (int)tq, (int)tk, sq, sk,
                       sv, so, scale, causal, (int)npairs, (int)blocks_of(tq));
    return launch_check("attn_fused_kernel");
}

}  // namespace

bool attention_fused_supported(int64_t dh, int64_t tq, int64_t tk) {
    if (!(dh == 16 || dh == 32 || dh == 64 || dh == 128)) return false;
    return tq > 0 && tk > 0 && tq <= INT32_MAX - QB && tk <= INT32_MAX - 2 * KT;
}

int attention_fused(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq,
                    int64_t tk, int64_t dh, int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale,
                    int causal, hipStream_t s) {
    if (batch <= 0 || batch > 65535) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: batch %lld", (long long)batch);
    if (!attention_fused_supported(dh, tq, tk))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: fused kernel unsupported for dh=%lld tq=%lld tk=%lld",
                    (long long)dh, (long long)tq, (long long)tk);
    if (pairs_of(tq) * batch > INT32_MAX)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: %lld heads of %lld queries exceed one launch",
                    (long long)batch, (long long)tq);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
    if (al % 16 || (sq | sk | sv | so) % 4)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: Q, K, V and O need 16-byte aligned rows");
    switch (dh) {
        case 16: return launch<16>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
        case 32: return launch<32>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
        case 64: return launch<64>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
        default: return launch<128>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
    }
}

}  // namespace mlxhip
