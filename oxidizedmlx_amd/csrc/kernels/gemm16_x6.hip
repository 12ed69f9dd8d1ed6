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

// Two chunks per thread per step, both loaded before either is split, so
// each wave keeps four 16-byte loads per lane in flight.
__global__ void __launch_bounds__(256) x6_split_kernel(X6SplitPair sp) {
    const X6SplitOp& o = sp.op[blockIdx.y];
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

}  // namespace

int x6_split(const X6SplitPair& sp, hipStream_t s) {
    if (sp.n < 0 || sp.n > 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: split-f32 operand count");
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

int gemm16_x6(int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s) {
    return gemm16::dispatch<MLXHIP_DTYPE_BF16, MLXHIP_DTYPE_F32, true>(a, batch, ta, tb, cfg, s);
}

}  // namespace mlxhip
