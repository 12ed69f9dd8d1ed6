// gemm16_x6.hip — f32 GEMM on the bf16 matrix cores: each f32 operand is
// split exactly into three bf16 planes (hi + mid + lo == x, each rounded to
// nearest from what the planes before it leave), and the direct-to-LDS bf16
// kernel (gemm16_impl.hpp) sums the six significant plane products in f32.
//
// Replaces matmul (crates/mlx-core/src/cpu_kernels.rs:197-230) for large f32
// products: v_mfma_f32_32x32x16_bf16 does 16 times the work per cycle of
// v_mfma_f32_32x32x2_f32, so six of them per f32 product still leave the
// f32 instruction behind, and the split itself is an elementwise pass over
// the operands (4 bytes read, 6 written per element).
//
// Values that are not finite, or whose hi plane would round past the bf16
// range (|x| above about 3.39e38), cannot be split; the split kernel then
// writes the call's generation number into a flag word and the GEMM kernel,
// seeing it, forms C from the f32 operands directly (x6_direct), so such
// inputs give what an f32 product gives.
#include "gemm16_impl.hpp"

namespace mlxhip {

namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// Round to nearest even (v_cvt_pk_bf16_f32), as raw bits and back.
__device__ inline uint16_t to_bf16(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
__device__ inline float from_bf16(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// One 8-element chunk of a plane row: the source values (zeros beyond the
// source extent).
struct SplitChunk {
    uint32_t row_all, c0;
    bool in;
};

__device__ inline SplitChunk locate(const X6SplitOp& o, uint32_t c, uint32_t cpr, uint32_t rows_p) {
    SplitChunk k;
    k.row_all = c / cpr;
    k.c0 = (c - k.row_all * cpr) * 8;
    k.in = c < o.chunks;
    return k;
}

__device__ inline void load_chunk(const X6SplitOp& o, const SplitChunk& k, uint32_t rows_p, bool vec, float (&x)[8]) {
    const uint32_t b = k.row_all / rows_p, r = k.row_all - b * rows_p;
    const float* src = o.src + (int64_t)b * o.stride + (int64_t)r * o.ld + k.c0;
    if (k.in && r < o.rows && k.c0 + 8 <= o.cols && vec) {
        const f32x4v v0 = *reinterpret_cast<const f32x4v*>(src);
        const f32x4v v1 = *reinterpret_cast<const f32x4v*>(src + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = v0[e];
            x[4 + e] = v1[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (k.in && r < o.rows && k.c0 + e < o.cols) ? src[e] : 0.0f;
    }
}

__device__ inline void split_store(const X6SplitOp& o, const SplitChunk& k, const float (&x)[8], bool& bad) {
    u16x8 hi, mid, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        // Each difference is exact in f32: x - hi has at most 16
        // significant bits and (x - hi) - mid at most 8.
        const uint16_t h = to_bf16(x[e]);
        const float r1 = x[e] - from_bf16(h);
        const uint16_t m = to_bf16(r1);
        const float r2 = r1 - from_bf16(m);
        hi[e] = h;
        mid[e] = m;
        lo[e] = to_bf16(r2);
        bad |= !__builtin_isfinite(from_bf16(h));
    }
    if (!k.in) return;
    uint16_t* dst = o.dst + (int64_t)k.row_all * o.cols_p + k.c0;
    *reinterpret_cast<u16x8*>(dst) = hi;
    *reinterpret_cast<u16x8*>(dst + o.plane) = mid;
    *reinterpret_cast<u16x8*>(dst + 2 * o.plane) = lo;
}

// The split of one operand by this workgroup: two chunks per thread per
// step, both loaded before either is split, so each wave keeps four 16-byte
// loads per lane in flight.
__device__ inline void split_op(const X6SplitOp& o) {
    const uint32_t cpr = (uint32_t)(o.cols_p / 8);  // 8-element chunks per plane row
    const uint32_t rows_p = (uint32_t)o.rows_p;
    const bool vec = o.ld % 4 == 0 && reinterpret_cast<uintptr_t>(o.src) % 16 == 0 && o.stride % 4 == 0;
    const uint32_t step = gridDim.x * 256;
    bool bad = false;
    for (uint32_t c = blockIdx.x * 512 + threadIdx.x; c < o.chunks; c += 2 * step) {
        const SplitChunk k0 = locate(o, c, cpr, rows_p), k1 = locate(o, c + 256, cpr, rows_p);
        float x0[8], x1[8];
        load_chunk(o, k0, rows_p, vec, x0);
        load_chunk(o, k1, rows_p, vec, x1);
        split_store(o, k0, x0, bad);
        split_store(o, k1, x1, bad);
    }
    // Every writer stores the same word, so the stores need no order.
    if (bad) *o.flag = o.gen;
}

// gridDim.y = operands; each case names its operand with a constant index (a
// run-time index into the kernel arguments would copy them to scratch).
__global__ void __launch_bounds__(256) x6_split_kernel(X6SplitPair sp) {
    switch (blockIdx.y) {
        case 0: split_op(sp.op[0]); break;
        case 1: split_op(sp.op[1]); break;
        case 2: split_op(sp.op[2]); break;
        case 3: split_op(sp.op[3]); break;
        default: split_op(sp.op[4]); break;
    }
}

}  // namespace

int x6_split(const X6SplitPair& sp, hipStream_t s) {
    if (sp.n < 0 || sp.n > X6SplitPair::MAX) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: split-f32 operand count");
    int64_t most = 0;
    for (int i = 0; i < sp.n; ++i) {
        const X6SplitOp& o = sp.op[i];
        if (o.cols_p % 8 || o.rows_p < o.rows || o.cols_p < o.cols || o.chunks != o.plane / 8 ||
            o.chunks >= ((int64_t)1 << 31) || reinterpret_cast<uintptr_t>(o.dst) % 16 || !o.flag)
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: split-f32 plane layout");
        most = std::max(most, o.chunks);
    }
    if (most == 0) return MLXHIP_OK;
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(most, 512), 4096);
    hipLaunchKernelGGL(x6_split_kernel, dim3(blocks, (unsigned)sp.n), dim3(256), 0, s, sp);
    return launch_check("x6_split_kernel");
}

namespace gemm16 {

// Interleaved split-f32 blocks: every stage holds the K tile of all three
// planes of both operands, and each k-step runs the six plane products from
// one set of fragment reads (half the operand loads and half the LDS reads
// per MFMA of the segment-by-segment order). WM x WN waves of TM x TN 32x32
// tiles, two waves per SIMD.
template <int WM_, int WN_, int TM_, int TN_, int STAGES_>
struct CfgI {
    static constexpr int WM = WM_, WN = WN_, TM = TM_, TN = TN_, STAGES = STAGES_, WPE = 2;
    static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES;
    static constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;  // one plane of one stage
    static constexpr int STAGE_BYTES = 3 * (A_BYTES + B_BYTES);        // A planes 0-2, then B planes 0-2
    static constexpr int LA = A_BYTES / (THREADS * 16), LB = B_BYTES / (THREADS * 16);  // per plane
    static_assert(BM >= 128 && BN >= 128, "MN-contiguous LDS rows need >= 16 chunks for the swizzle");
    static_assert(LA * THREADS * 16 == A_BYTES && LB * THREADS * 16 == B_BYTES, "whole 1 KiB blocks per wave");
    static_assert(STAGES >= 2 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS budget");
};
// 256 x 128, 8 waves of 64 x 64, two stages of 72 KiB.
using CfgIWide = CfgI<4, 2, 2, 2, 2>;
// 128 x 128, 8 waves of 64 x 32, three stages of 48 KiB.
using CfgIMid = CfgI<2, 4, 2, 1, 3>;

template <int TA, int TB, class C>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS), amdgpu_waves_per_eu(C::WPE, C::WPE)))
void gemm_x6i_kernel(Args g) {
    constexpr bool KCA = (TA == 0), KCB = (TB == 1);
    constexpr int STAGES = C::STAGES, TM = C::TM, TN = C::TN, WAVES = C::WAVES;
    constexpr int PIPE_BYTES = STAGES * C::STAGE_BYTES;
    constexpr int EPI_BYTES = epi_bytes<MLXHIP_DTYPE_F32, C, PIPE_BYTES>();
    constexpr int SMEM_BYTES = PIPE_BYTES > EPI_BYTES ? PIPE_BYTES : EPI_BYTES;
    __shared__ __attribute__((aligned(1024))) char smem_raw[SMEM_BYTES];
    MLXHIP_LDS char* smem = (MLXHIP_LDS char*)smem_raw;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WN, wn = wave % C::WN;
    const TileId tl = tile_of<C>(g);
    const int64_t slice = tl.slice, batch = tl.batch, split = tl.split, m0 = tl.m0, n0 = tl.n0;

    // This slice's planes, C and f32 operands (a group's, or base + stride).
    const char *pa, *pb;
    char* pc;
    const float *fa32, *fb32;
    const uint32_t *flag_a, *flag_b;
    uint32_t gen_a, gen_b;
    const float* bias;
    if (g.groups) {
        const Args::Group gr = group_of(g, (int)batch);
        pa = static_cast<const char*>(gr.a);
        pb = static_cast<const char*>(gr.b);
        pc = static_cast<char*>(gr.c);
        fa32 = gr.fa;
        fb32 = gr.fb;
        flag_a = gr.flag_a;
        flag_b = gr.flag_b;
        gen_a = gr.gen_a;
        gen_b = gr.gen_b;
        bias = gr.bias;
    } else {
        pa = static_cast<const char*>(g.a) + batch * g.sa * 2;
        pb = static_cast<const char*>(g.b) + batch * g.sb * 2;
        pc = static_cast<char*>(g.c) + slice * g.sc * 4;
        fa32 = g.fa + batch * g.fsa;
        fb32 = g.fb + batch * g.fsb;
        flag_a = g.flag_a;
        flag_b = g.flag_b;
        gen_a = g.gen_a;
        gen_b = g.gen_b;
        bias = g.bias;
    }

    if (__atomic_load_n(flag_a, __ATOMIC_RELAXED) == gen_a || __atomic_load_n(flag_b, __ATOMIC_RELAXED) == gen_b) {
        x6_direct<TA, TB, C>(g, fa32, fb32, reinterpret_cast<float*>(pc), split, m0, n0, tid, bias);
        return;
    }

    // Split over K as in gemm16_kernel (K here is the planes' K); plane p of
    // either operand sits p * plane bytes after plane 0.
    const int64_t kb = split * g.k_chunk;
    const int64_t klen = g.splits > 1 ? min(g.k - kb, g.k_chunk) : g.k;
    const int64_t a_koff = (KCA ? kb : kb * g.lda) * 2, b_koff = (KCB ? kb : kb * g.ldb) * 2;
    const char* A = pa + a_koff;
    const char* B = pb + b_koff;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)(g.a_bytes - (uint32_t)a_koff), BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)(g.b_bytes - (uint32_t)b_koff), BUF_FLAGS);

    constexpr int ROWB_A = C::BM * 2, ROWB_B = C::BN * 2;
    Loader<KCA, C::BM, WAVES> la;
    Loader<KCB, C::BN, WAVES> lb;
    la.init(tid, m0, g.m, g.lda, klen);
    lb.init(tid, n0, g.n, g.ldb, klen);
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
    constexpr int LA = C::LA, LB = C::LB, LPT = 3 * (LA + LB);
    constexpr int B0 = 3 * C::A_BYTES;  // first B plane in a stage

    // Prologue: tiles 0 .. STAGES-1 (all planes) into stages 0 .. STAGES-1.
#pragma unroll
    for (int t = 0; t < STAGES; ++t) {
        MLXHIP_LDS char* st = smem + t * C::STAGE_BYTES;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            la.issue(ra, st + p * C::A_BYTES, wave, t * BK, (uint32_t)p * g.plane_a);
            lb.issue(rb, st + B0 + p * C::B_BYTES, wave, t * BK, (uint32_t)p * g.plane_b);
        }
    }
    wait_vmcnt<(STAGES - 1) * LPT>();
    lds_barrier();

    // Fragments of k-step s: af[s][plane][i], bf[s][plane][j].
    constexpr int NA = KCA ? TM : 2 * TM, NB = KCB ? TN : 2 * TN, NR = 3 * (NA + NB);
    u32x4 af[2][3][TM], bf[2][3][TN];
    auto read_op = [&](const MLXHIP_LDS char* st, int s, int o) {
        if (o < 3 * NA) {
            const int p = o / NA;
            read_one<KCA, TM, ROWB_A>(st + p * C::A_BYTES, fa, s, o - p * NA, af[s][p]);
        } else {
            const int ob = o - 3 * NA, p = ob / NB;
            read_one<KCB, TN, ROWB_B>(st + B0 + p * C::B_BYTES, fb, s, ob - p * NB, bf[s][p]);
        }
    };
#pragma unroll
    for (int o = 0; o < NR; ++o) read_op(smem, 0, o);

    // Each half-tile: the 6 x TM x TN MFMAs of one k-step (pair-major, so
    // consecutive MFMAs feed different accumulators), with the next half's
    // LDS reads (and, in the second half, the loads of tile kt+STAGES) placed
    // between them.
    constexpr int NM = TM * TN, NMI = X6_SEGS * NM;
    constexpr int OPS2 = NR + 3 * (LA + LB);
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt % STAGES;
        const MLXHIP_LDS char* st = smem + cur * C::STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < NMI; ++q) {
            const int e = q / NM, t = q % NM;
            mfma<MLXHIP_DTYPE_BF16>(bf[0][seg_plane_b(e)][t % TN], af[0][seg_plane_a(e)][t / TN], acc[t / TN][t % TN]);
#pragma unroll
            for (int o = (q * NR) / NMI; o < ((q + 1) * NR) / NMI; ++o) read_op(st, 1, o);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Tile kt+1 has landed for every wave; every wave is done reading this
        // tile's stage, which then receives tile kt+STAGES.
        wait_vmcnt<(STAGES - 2) * LPT>();
        lds_barrier();
        MLXHIP_LDS char* dst = smem + cur * C::STAGE_BYTES;
        const int k0 = (kt + STAGES) * BK;
        const MLXHIP_LDS char* nx = smem + ((kt + 1) % STAGES) * C::STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < NMI; ++q) {
            const int e = q / NM, t = q % NM;
            mfma<MLXHIP_DTYPE_BF16>(bf[1][seg_plane_b(e)][t % TN], af[1][seg_plane_a(e)][t / TN], acc[t / TN][t % TN]);
#pragma unroll
            for (int o = (q * OPS2) / NMI; o < ((q + 1) * OPS2) / NMI; ++o) {
                if (o < NR) {
                    read_op(nx, 0, o);
                } else if (o < NR + 3 * LA) {
                    const int p = (o - NR) / LA;
                    la.issue_one(ra, dst + p * C::A_BYTES, wave, k0, o - NR - p * LA, (uint32_t)p * g.plane_a);
                } else {
                    const int ob = o - NR - 3 * LA, p = ob / LB;
                    lb.issue_one(rb, dst + B0 + p * C::B_BYTES, wave, k0, ob - p * LB, (uint32_t)p * g.plane_b);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    store_c<MLXHIP_DTYPE_F32, C, PIPE_BYTES>(g, acc, smem, pc, m0, n0, wave, lane, bias);
}

template <int TA, int TB, class C>
int launch_x6i(const Args& a0, int64_t batch, hipStream_t s) {
    Args a = a0;
    a.tiles_m = (int)ceil_div(a.m, C::BM);
    a.tiles_n = (int)ceil_div(a.n, C::BN);
    dim3 grid((unsigned)(a.tiles_m * a.tiles_n), (unsigned)(batch * a.splits));
    hipLaunchKernelGGL((gemm_x6i_kernel<TA, TB, C>), grid, dim3(C::THREADS), 0, s, a);
    return launch_check("gemm_x6i_kernel");
}

template <class C>
int dispatch_x6i(const Args& a, int64_t batch, int ta, int tb, hipStream_t s) {
    if (!ta && !tb) return launch_x6i<0, 0, C>(a, batch, s);
    if (!ta && tb) return launch_x6i<0, 1, C>(a, batch, s);
    if (ta && !tb) return launch_x6i<1, 0, C>(a, batch, s);
    return launch_x6i<1, 1, C>(a, batch, s);
}

}  // namespace gemm16

// cfg 0-2: segment-by-segment kernel (CfgLarge, CfgMid, CfgWide), k and
// splits over the 6 segments; cfg 3 / 4: interleaved kernel (CfgIWide,
// CfgIMid), k and splits over the planes' K.
int gemm16_x6(int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s) {
    if (cfg == 3) return gemm16::dispatch_x6i<gemm16::CfgIWide>(a, batch, ta, tb, s);
    if (cfg == 4) return gemm16::dispatch_x6i<gemm16::CfgIMid>(a, batch, ta, tb, s);
    return gemm16::dispatch<MLXHIP_DTYPE_BF16, MLXHIP_DTYPE_F32, true>(a, batch, ta, tb, cfg, s);
}

}  // namespace mlxhip
