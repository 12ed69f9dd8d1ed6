// gemm.hip — host-side validation and dispatch of the MFMA GEMM
// (kernel in gemm_impl.hpp, instantiated per input dtype in gemm_{f32,bf16,f16}.hip).
#include "../common.hpp"
#include "../kernels.hpp"
#include "gemm_impl.hpp"
#include "gemm16_impl.hpp"

#include <cstdlib>
#include <cstring>

namespace mlxhip {
namespace {

__global__ __launch_bounds__(256) void zero_c_kernel(char* c, int64_t ldc, int64_t sc, int64_t m,
                                                     int64_t n, int elem) {
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= m * n) return;
    const int64_t r = f / n, col = f % n;
    char* p = c + ((int64_t)blockIdx.y * sc + r * ldc + col) * elem;
    for (int e = 0; e < elem; ++e) p[e] = 0;
}

int elem_size(int dt) { return dt == MLXHIP_DTYPE_F32 ? 4 : 2; }

// MLXHIP_GEMM_PATH: unset/"auto" = choose by shape, "general" = always the
// general kernel, "lds16" = the direct-to-LDS 16-bit kernel whenever the
// operands allow it. Read on every call so one process (the tests) can
// cover both kernels.
int gemm_path() {
    const char* e = getenv("MLXHIP_GEMM_PATH");
    if (!e) return 0;
    if (!strcmp(e, "general")) return 1;
    if (!strcmp(e, "lds16")) return 2;
    return 0;
}

}  // namespace

int gemm(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
         int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
         int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s) {
    if (ab_dtype != MLXHIP_DTYPE_F32 && ab_dtype != MLXHIP_DTYPE_BF16 && ab_dtype != MLXHIP_DTYPE_F16)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: input dtype %d unsupported", ab_dtype);
    if (c_dtype != MLXHIP_DTYPE_F32 && c_dtype != MLXHIP_DTYPE_BF16 && c_dtype != MLXHIP_DTYPE_F16)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: output dtype %d unsupported", c_dtype);
    if (m < 0 || n < 0 || k < 0 || batch < 0)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: negative size");
    if (m == 0 || n == 0 || batch == 0) return MLXHIP_OK;
    if (!c) return fail(MLXHIP_ERR_NULL_PTR, "gemm: C is null");
    if (ldc < n) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: ldc %lld < n %lld", (long long)ldc, (long long)n);
    if (batch > 65535) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: batch %lld > 65535", (long long)batch);
    if (k == 0) {
        dim3 grid((unsigned)ceil_div(m * n, 256), (unsigned)batch);
        hipLaunchKernelGGL(zero_c_kernel, grid, dim3(256), 0, s, static_cast<char*>(c), ldc, stride_c,
                           m, n, elem_size(c_dtype));
        return launch_check("zero_c_kernel");
    }
    if (!a || !b) return fail(MLXHIP_ERR_NULL_PTR, "gemm: A or B is null");
    const int64_t a_cols = trans_a ? m : k, b_cols = trans_b ? k : n;
    if (lda < a_cols) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: lda %lld < %lld", (long long)lda, (long long)a_cols);
    if (ldb < b_cols) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: ldb %lld < %lld", (long long)ldb, (long long)b_cols);
    if (ceil_div(m, 64) * ceil_div(n, 64) > INT32_MAX)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: too many tiles");

    const int ch = 16 / elem_size(ab_dtype);
    const bool aligned = reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(b) % 16 == 0 && lda % ch == 0 &&
                         ldb % ch == 0 && (batch == 1 || (stride_a % ch == 0 && stride_b % ch == 0));

    gemm_detail::GemmArgs g{};
    g.m = m;
    g.n = n;
    g.k = k;
    g.a = a;
    g.lda = lda;
    g.sa = stride_a;
    g.b = b;
    g.ldb = ldb;
    g.sb = stride_b;
    g.c = c;
    g.ldc = ldc;
    g.sc = stride_c;
    const int ta = trans_a ? 1 : 0, tb = trans_b ? 1 : 0;
    // 16-bit operands on 256x256 tiles with direct-to-LDS loads when the
    // problem fills the chip and the operands meet that kernel's layout
    // requirements; the general kernel covers everything else.
    const int path = gemm_path();
    if (ab_dtype != MLXHIP_DTYPE_F32 && path != 1) {
        const int64_t big_tiles = ceil_div(m, 256) * ceil_div(n, 256) * batch;
        gemm16::Args h{};
        if ((path == 2 || big_tiles >= 200) &&
            gemm16::supported(ta, tb, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, &h.a_bytes,
                              &h.b_bytes)) {
            h.m = m;
            h.n = n;
            h.k = k;
            h.a = a;
            h.lda = lda;
            h.sa = stride_a;
            h.b = b;
            h.ldb = ldb;
            h.sb = stride_b;
            h.c = c;
            h.ldc = ldc;
            h.sc = stride_c;
            return ab_dtype == MLXHIP_DTYPE_BF16 ? gemm16_bf16(c_dtype, ta, tb, h, batch, s)
                                                 : gemm16_f16(c_dtype, ta, tb, h, batch, s);
        }
    }
    switch (ab_dtype) {
        case MLXHIP_DTYPE_F32: return gemm_f32(c_dtype, ta, tb, g, batch, aligned, s);
        case MLXHIP_DTYPE_BF16: return gemm_bf16(c_dtype, ta, tb, g, batch, aligned, s);
        default: return gemm_f16(c_dtype, ta, tb, g, batch, aligned, s);
    }
}

}  // namespace mlxhip
