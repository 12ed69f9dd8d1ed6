// attention.hip — fused scaled, masked attention for a batch of heads:
//   O_b = softmax(Q_b K_b^T * scale, causal) V_b,  Q_b [tq, dh], K_b, V_b [tk, dh]
// with the arithmetic of cpu_attention (crates/mlx-core/src/cpu_kernels.rs:
// 738-812): scores = (q . k) * scale, the causal entries j > i excluded (the
// reference writes -1e9 there, whose exp is 0 next to any finite score),
// softmax over the row, then P V.
//
// f32 products on the bf16 matrix cores. Every f32 operand x is split into
// three bf16 terms x = hi + mid + lo, exactly (hi keeps the top 8 significant
// bits, mid the next 8, lo the last 8; each step is a truncation and an exact
// f32 subtraction). A product a*b is then the sum of the six terms that reach
// f32 precision, hi*hi + (hi*mid + mid*hi) + (hi*lo + lo*hi + mid*mid); the
// dropped ones (mid*lo, lo*mid, lo*lo) are below 2^-24 of it. Each term is a
// v_mfma_f32_16x16x32_bf16 with f32 accumulation (bf16 x bf16 products are
// exact in f32), the small terms accumulated first. Six of these cost 96
// cycles against 256 for the same products on v_mfma_f32_16x16x4f32.
//
// Streaming form. Queries are cut into blocks of 64 rows; a 512-thread
// workgroup owns one pair of blocks (b, nblk-1-b), so that under the causal
// mask every workgroup has the same number of key tiles, and processes them
// one after the other. Within a block, wave (g, h) owns rows 16g .. 16g+15
// and the key tiles of parity h (tiles of 32 keys, two per iteration). The
// workgroup stages each pair of tiles in LDS already split: K as three bf16
// planes [key][dh], V transposed as three planes [dh][key] (keys permuted, see
// below); the next pair is loaded into registers while the current one is
// computed. Per tile, a wave:
//   1. S^T = K Q^T: A = 16 key rows of K (planes from LDS), B = its 16 query
//      rows (split once per block, held in registers); then * scale. Lane
//      (i, g) holds 8 scores of query row i: keys 16x + 4g + r, x < 2, r < 4.
//   2. Online softmax per row: running max m and running sum l of
//      exp(s - m); when the max grows, l and the output row are rescaled by
//      exp(m_old - m_new). The row's max and sum over its four lane groups use
//      the gfx950 lane-swap instructions (v_permlane16/32_swap). exp(d) is
//      computed as 2^(d * log2 e) on the subtracted, small argument d.
//   3. O^T += V^T P^T: B = P^T, the lane's 8 weights split in registers, as MFMA
//      k-indices 8g + 4x + r; the V^T planes hold key 16x + 4g + r at position
//      8g + 4x + r, so A = V^T is one 16-byte read per plane. The O^T
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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int WAVE = 64;
constexpr int ATT_WAVES = 8;
constexpr int ATT_THREADS = ATT_WAVES * WAVE;
constexpr int QB = 64;  // query rows per block (four row groups of 16)
constexpr int KT = 32;  // keys per tile; the two wave halves take one tile each per iteration
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

// x = hi + mid + lo exactly; each term's bits are the high half of the
// returned word (the low half is zero).
struct Split3 {
    uint32_t hi, mid, lo;
};
__device__ inline Split3 split3(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t h = u & 0xFFFF0000u;
    const float r1 = x - __uint_as_float(h);
    const uint32_t m = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(m);
    return {h, m, __float_as_uint(r2)};
}
// Two terms (first in the low half) as one word of bf16 pairs.
__device__ inline uint32_t pack_hi(uint32_t first, uint32_t second) {
    return (second & 0xFFFF0000u) | (first >> 16);
}

__device__ inline f32x4 mma(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
// acc += a * b for split operands, small terms first.
__device__ inline f32x4 mma6(const u32x4 (&a)[3], const u32x4 (&b)[3], f32x4 acc) {
    acc = mma(a[1], b[1], acc);
    acc = mma(a[0], b[2], acc);
    acc = mma(a[2], b[0], acc);
    acc = mma(a[0], b[1], acc);
    acc = mma(a[1], b[0], acc);
    return mma(a[0], b[0], acc);
}

template <int DH>
struct Tile {
    static constexpr int NS = DH < 32 ? 1 : DH / 32;  // MFMA k-steps over the head dim (dh 16: one, half zero)
    static constexpr int CT = DH / 16;                // 16-column output tiles
    // K planes: [32 keys][dh] bf16, row pitch 2 dh + 16 bytes (the 16-byte
    // reads of 16 consecutive rows fall on distinct banks).
    static constexpr int KP2 = 2 * DH + 16;
    static constexpr int KPLANE = KT * KP2;
    // V^T planes: [dh][32 key positions] bf16, row pitch 80 bytes (same).
    static constexpr int VP2 = 2 * KT + 16;
    static constexpr int VPLANE = DH * VP2;
    static constexpr int TILEB = 3 * KPLANE + 3 * VPLANE;  // one split tile
    static constexpr int STAGE = 2 * TILEB;                // the pair of tiles of one iteration
    static constexpr int STAGES = 2 * STAGE <= 150 * 1024 ? 2 : 1;
    // Loader: unit = (pair of adjacent keys, 4 columns) of an iteration's 64 keys.
    static constexpr int UNITS = (2 * KT / 2) * (DH / 4);
    static constexpr int LU = (UNITS + ATT_THREADS - 1) / ATT_THREADS;  // units per thread
    static constexpr int MERGE = 4 * WAVE * (4 * CT + 2) * 4;           // bytes of the wave-pair merge
    static_assert(MERGE <= STAGE, "merge area must fit in one stage");
};

// Position of tile-local key k in the V^T planes: key 16x + 4g + r sits at
// 8g + 4x + r, the k-index its weight takes in the lane (i, g) of P^T.
__device__ inline int vpos(int key) { return 8 * ((key & 15) >> 2) + 4 * (key >> 4) + (key & 3); }

template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void attn_fused_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ v,
                                                                 float* __restrict__ o, int tq, int tk,
                                                                 int64_t sq, int64_t sk, int64_t sv,
                                                                 int64_t so, float scale, int causal,
                                                                 int npairs, int nblk, int hg, int rs) {
    using T = Tile<DH>;
    constexpr int NS = T::NS, CT = T::CT;
    __shared__ __attribute__((aligned(16))) char lds[T::STAGES * T::STAGE];

    // Workgroup -> (head, block pair). Consecutive workgroups go to
    // different XCDs; this numbering gives each XCD a contiguous range of
    // heads, so a head's K and V are fetched into one L2.
    const unsigned L = blockIdx.x, N = gridDim.x;
    const unsigned logical = N % XCDS == 0 ? (L % XCDS) * (N / XCDS) + L / XCDS : L;
    // Head bh is head bh % hg of row group bh / hg: its rows are rs floats
    // apart, its columns start at (bh % hg) * DH (hg = 1, rs = DH: one
    // [t, DH] block per head, s* floats apart).
    const int bh = (int)(logical / (unsigned)npairs), pair = (int)(logical % (unsigned)npairs);
    const int64_t grp = bh / hg, hcol = (int64_t)(bh % hg) * DH;
    q += grp * sq + hcol;
    k += grp * sk + hcol;
    v += grp * sv + hcol;
    o += grp * so + hcol;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int li = lane & 15, lg = lane >> 4;
    const int g = wave & 3, h = wave >> 2;

    // Loader units: u = tid + j*512 -> keys 2p, 2p+1 of the iteration's 64
    // (p = u / (dh/4)), columns 4 * (u % (dh/4)) + 0..3. Loads are
    // unconditional (keys clamped to tk - 1) and go straight into registers;
    // keys past tk are stored as zero V (their scores are masked, and 0 * V
    // must not meet a non-finite V).
    int ukey[T::LU], ucol[T::LU];
    bool uon[T::LU];
#pragma unroll
    for (int j = 0; j < T::LU; ++j) {
        const int u = tid + j * ATT_THREADS;
        uon[j] = u < T::UNITS;
        ukey[j] = 2 * ((uon[j] ? u : 0) / (DH / 4));
        ucol[j] = 4 * (u % (DH / 4));
    }
    float4 kr[T::LU][2], vr[T::LU][2];
#define ATT_LOAD(it)                                                                         \
    do {                                                                                     \
        const int kb_ = (it) * 2 * KT;                                                       \
        _Pragma("unroll") for (int j = 0; j < T::LU; ++j) {                                  \
            _Pragma("unroll") for (int e = 0; e < 2; ++e) {                                  \
                const int64_t o_ = (int64_t)min(kb_ + ukey[j] + e, tk - 1) * rs + ucol[j];   \
                kr[j][e] = *reinterpret_cast<const float4*>(k + o_);                         \
                vr[j][e] = *reinterpret_cast<const float4*>(v + o_);                         \
            }                                                                                \
        }                                                                                    \
    } while (0)
    // Split and store the loaded pair of tiles into stage `stage`.
    auto att_store = [&](int stage, int it) {
        char* st = lds + stage * T::STAGE;
#pragma unroll
        for (int j = 0; j < T::LU; ++j) {
            if (T::UNITS % ATT_THREADS == 0 || uon[j]) {
                const int key = ukey[j];  // even, 0..62
                char* tb = st + (key >> 5) * T::TILEB;
                const int kl = key & 31;
                // K: rows kl, kl+1, columns ucol .. ucol+3 of each plane.
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float kv[4] = {kr[j][e].x, kr[j][e].y, kr[j][e].z, kr[j][e].w};
                    Split3 s4[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) s4[c] = split3(kv[c]);
                    char* kp = tb + (kl + e) * T::KP2 + 2 * ucol[j];
                    *reinterpret_cast<u32x2*>(kp) = u32x2{pack_hi(s4[0].hi, s4[1].hi), pack_hi(s4[2].hi, s4[3].hi)};
                    *reinterpret_cast<u32x2*>(kp + T::KPLANE) =
                        u32x2{pack_hi(s4[0].mid, s4[1].mid), pack_hi(s4[2].mid, s4[3].mid)};
                    *reinterpret_cast<u32x2*>(kp + 2 * T::KPLANE) =
                        u32x2{pack_hi(s4[0].lo, s4[1].lo), pack_hi(s4[2].lo, s4[3].lo)};
                }
                // V^T: columns ucol .. ucol+3, positions vpos(kl), vpos(kl)+1.
                const bool in0 = (it) * 2 * KT + key < tk, in1 = (it) * 2 * KT + key + 1 < tk;
                const float v0[4] = {vr[j][0].x, vr[j][0].y, vr[j][0].z, vr[j][0].w};
                const float v1[4] = {vr[j][1].x, vr[j][1].y, vr[j][1].z, vr[j][1].w};
                char* vp = tb + 3 * T::KPLANE + ucol[j] * T::VP2 + 2 * vpos(kl);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const Split3 a = split3(in0 ? v0[c] : 0.0f), b = split3(in1 ? v1[c] : 0.0f);
                    char* p = vp + c * T::VP2;
                    *reinterpret_cast<uint32_t*>(p) = pack_hi(a.hi, b.hi);
                    *reinterpret_cast<uint32_t*>(p + T::VPLANE) = pack_hi(a.mid, b.mid);
                    *reinterpret_cast<uint32_t*>(p + 2 * T::VPLANE) = pack_hi(a.lo, b.lo);
                }
            }
        }
    };

    for (int bi = 0; bi < 2; ++bi) {
        const int blk = bi == 0 ? pair : nblk - 1 - pair;
        if (bi == 1 && blk == pair) break;  // the middle block of an odd count
        const int q0 = blk * QB, qw = q0 + 16 * g;
        const int kend = causal ? min(tk, q0 + QB) : tk;  // keys any row of the block sees
        const int niter = (kend + 2 * KT - 1) / (2 * KT);

        // This wave's query rows as B operands, split: lane holds row qw + li,
        // columns 32s + 8lg .. +7 (zero past dh).
        u32x4 qb[NS][3];
        {
            const float* qr = q + (int64_t)min(qw + li, tq - 1) * rs;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                float x[8];
                if (DH >= 32 || 8 * lg < DH) {
                    const float4 a = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg);
                    const float4 b = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg + 4);
                    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
                }
                Split3 sp[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) sp[e] = split3(x[e]);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    qb[s][0][w] = pack_hi(sp[2 * w].hi, sp[2 * w + 1].hi);
                    qb[s][1][w] = pack_hi(sp[2 * w].mid, sp[2 * w + 1].mid);
                    qb[s][2][w] = pack_hi(sp[2 * w].lo, sp[2 * w + 1].lo);
                }
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
            const char* tb = lds + stage * T::STAGE + h * T::TILEB;
            // 1. S^T of the two 16-key halves.
            f32x4 sa[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
#pragma unroll
                for (int x = 0; x < 2; ++x) {
                    u32x4 ka[3];
                    const char* kp = tb + (16 * x + li) * T::KP2 + 2 * (32 * s + 8 * lg);
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl) {
                        if (DH >= 32 || 8 * lg < DH) ka[pl] = *reinterpret_cast<const u32x4*>(kp + pl * T::KPLANE);
                        else ka[pl] = u32x4{0u, 0u, 0u, 0u};
                    }
                    sa[x] = mma6(ka, qb[s], sa[x]);
                }
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
            // 3. O^T = O^T * corr + V^T P^T. P^T's k-index 8lg + 4x + r is key 16x + 4lg + r.
            u32x4 pb[3];
            {
                Split3 sp[8];
#pragma unroll
                for (int x = 0; x < 2; ++x)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sp[4 * x + r] = split3(p[x][r]);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    pb[0][w] = pack_hi(sp[2 * w].hi, sp[2 * w + 1].hi);
                    pb[1][w] = pack_hi(sp[2 * w].mid, sp[2 * w + 1].mid);
                    pb[2][w] = pack_hi(sp[2 * w].lo, sp[2 * w + 1].lo);
                }
            }
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[c][r] *= corr;
            const char* vt = tb + 3 * T::KPLANE + 16 * lg;
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                u32x4 va[3];
                const char* vp = vt + (16 * c + li) * T::VP2;
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) va[pl] = *reinterpret_cast<const u32x4*>(vp + pl * T::VPLANE);
                acc[c] = mma6(va, pb, acc[c]);
            }
        };

        ATT_LOAD(0);
        att_store(0, 0);
        __syncthreads();
        for (int it = 0; it + 1 < niter; ++it) {
            ATT_LOAD(it + 1);
            __builtin_amdgcn_sched_barrier(0);  // the scheduler would otherwise move the loads after the MFMAs
            if constexpr (T::STAGES == 2) {
                tile(2 * it + h, it & 1);
                att_store((it + 1) & 1, it + 1);
            } else {
                tile(2 * it + h, 0);
                __syncthreads();
                att_store(0, it + 1);
            }
            __syncthreads();
        }
        tile(2 * (niter - 1) + h, (niter - 1) % T::STAGES);
        __syncthreads();  // every wave is done with the stages: the merge area aliases them

        // Merge the wave pair (g, 1) into (g, 0): m = max, weights 2^((m_x - m) log2 e).
        float* mg = reinterpret_cast<float*>(lds) + (g * WAVE + lane) * (4 * CT + 2);
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
                float* orow = o + (int64_t)row * rs + 4 * lg;
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
}

int64_t blocks_of(int64_t tq) { return (tq + QB - 1) / QB; }
int64_t pairs_of(int64_t tq) { return (blocks_of(tq) + 1) / 2; }

template <int DH>
int launch(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq, int64_t tk,
           int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale, int causal, int hg, int rs,
           hipStream_t s) {
    const int64_t npairs = pairs_of(tq);
    const dim3 grid((unsigned)(npairs * batch));
    hipLaunchKernelGGL(attn_fused_kernel<DH>, grid, dim3(ATT_THREADS), 0, s, q, k, v, o, (int)tq, (int)tk, sq, sk,
                       sv, so, scale, causal, (int)npairs, (int)blocks_of(tq), hg, rs);
    return launch_check("attn_fused_kernel");
}

}  // namespace

bool attention_fused_supported(int64_t dh, int64_t tq, int64_t tk) {
    if (!(dh == 16 || dh == 32 || dh == 64 || dh == 128)) return false;
    return tq > 0 && tk > 0 && tq <= INT32_MAX - QB && tk <= INT32_MAX - 2 * KT;
}

int attention_fused(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq,
                    int64_t tk, int64_t dh, int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale,
                    int causal, hipStream_t s, int64_t hg, int64_t rs) {
    if (batch <= 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: batch %lld", (long long)batch);
    if (rs == 0) rs = dh;
    if (hg < 1 || batch % hg || rs < hg * dh || rs % 4 || rs > INT32_MAX || hg > INT32_MAX)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: %lld heads per row of %lld floats (dh %lld, batch %lld)",
                    (long long)hg, (long long)rs, (long long)dh, (long long)batch);
    if (!attention_fused_supported(dh, tq, tk))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: fused kernel unsupported for dh=%lld tq=%lld tk=%lld",
                    (long long)dh, (long long)tq, (long long)tk);
    // A dispatch counts its work-items in 32 bits: one launch holds at most
    // (2^32 - 1) / ATT_THREADS workgroups. Heads are independent, so a larger
    // batch runs as several launches.
    const int64_t max_wg = int64_t(UINT32_MAX) / ATT_THREADS, np = pairs_of(tq);
    if (np > max_wg)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: %lld queries exceed one launch", (long long)tq);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
    if (al % 16 || (sq | sk | sv | so) % 4)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: Q, K, V and O need 16-byte aligned rows");
    // Whole row groups per launch.
    const int64_t per = (max_wg / np) / hg * hg;
    if (per == 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: %lld heads per row exceed one launch", (long long)hg);
    const int ihg = (int)hg, irs = (int)rs;
    for (int64_t b0 = 0; b0 < batch; b0 += per) {
        const int64_t nb = std::min(per, batch - b0), g0 = b0 / hg;
        const float *qb = q + g0 * sq, *kb = k + g0 * sk, *vb = v + g0 * sv;
        float* ob = o + g0 * so;
        switch (dh) {
            case 16: MLXHIP_TRY(launch<16>(qb, kb, vb, ob, nb, tq, tk, sq, sk, sv, so, scale, causal, ihg, irs, s)); break;
            case 32: MLXHIP_TRY(launch<32>(qb, kb, vb, ob, nb, tq, tk, sq, sk, sv, so, scale, causal, ihg, irs, s)); break;
            case 64: MLXHIP_TRY(launch<64>(qb, kb, vb, ob, nb, tq, tk, sq, sk, sv, so, scale, causal, ihg, irs, s)); break;
            default: MLXHIP_TRY(launch<128>(qb, kb, vb, ob, nb, tq, tk, sq, sk, sv, so, scale, causal, ihg, irs, s)); break;
        }
    }
    return MLXHIP_OK;
}

}  // namespace mlxhip
