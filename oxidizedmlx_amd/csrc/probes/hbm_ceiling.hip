// hbm_ceiling.hip — achievable HBM bandwidth of simple streaming kernels
// with cold caches: read-only, copy (1 read + 1 write, plain and
// non-temporal stores) and a 3-read/1-write stream, each over 64 MiB
// buffers rotated through a 2 GiB working set (well beyond the 256 MiB
// Infinity Cache), plus the same copy repeated on one buffer pair (warm).
//
// Measurement tool, not part of libmlxhip.so: it gives the ceilings the
// HBM-bound kernels of the library are compared with.
// Build: python -m oxidizedmlx_amd.build --probes; run: oxidizedmlx_amd/_build/hbm_ceiling
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x)                                                                         \
    do {                                                                              \
        hipError_t e = (x);                                                           \
        if (e != hipSuccess) {                                                        \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__); \
            std::exit(3);                                                             \
        }                                                                             \
    } while (0)

typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_sum(const f32x4* __restrict__ x, float* out, int64_t n) {
    f32x4 acc = {0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) acc += x[i];
    if (acc.x + acc.y + acc.z + acc.w == 1234.5f) out[0] = 1.f;
}

template <bool NT>
__global__ __launch_bounds__(256) void copy_k(const f32x4* __restrict__ x, f32x4* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const f32x4 v = x[i];
        if (NT) __builtin_nontemporal_store(v, y + i);
        else y[i] = v;
    }
}

__global__ __launch_bounds__(256) void fma3(const f32x4* __restrict__ a, const f32x4* __restrict__ b,
                                            const f32x4* __restrict__ c, f32x4* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = a[i] * b[i] + c[i];
}

template <typename F>
void timeit(const char* name, F f, double bytes) {
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    std::vector<float> t;
    for (int r = 0; r < 5; ++r) {
        CK(hipEventRecord(e0, 0));
        for (int i = 0; i < 8; ++i) f(i);
        CK(hipEventRecord(e1, 0));
        CK(hipEventSynchronize(e1));
        float ms = 0;
        CK(hipEventElapsedTime(&ms, e0, e1));
        t.push_back(ms * 1e3f / 8);
    }
    std::sort(t.begin(), t.end());
    std::printf("%-46s median %7.1f us  %7.0f GB/s  %5.1f%% of 8 TB/s\n", name, t[2], bytes / (t[2] * 1e-6) / 1e9,
                100 * bytes / (t[2] * 1e-6) / 8e12);
    std::fflush(stdout);
}

int main() {
    const int64_t n = 4096LL * 4096, nv = n / 4;  // 64 MiB per buffer
    const int SETS = 8;                            // 8 x 4 x 64 MiB = 2 GiB
    std::vector<f32x4*> a(SETS), b(SETS), c(SETS), y(SETS);
    for (int i = 0; i < SETS; ++i) {
        for (auto* p : {&a[i], &b[i], &c[i], &y[i]}) {
            CK(hipMalloc(reinterpret_cast<void**>(p), n * 4));
            CK(hipMemset(*p, 0, n * 4));
        }
    }
    float* o;
    CK(hipMalloc(&o, 4));
    const unsigned grid = (unsigned)(nv / 256);
    timeit("read only (cold)", [&](int i) { hipLaunchKernelGGL(read_sum, dim3(4096), dim3(256), 0, 0, a[i % SETS], o, nv); },
           4.0 * n);
    timeit("copy, plain store (cold)", [&](int i) { hipLaunchKernelGGL(copy_k<false>, dim3(grid), dim3(256), 0, 0, a[i % SETS], y[i % SETS], nv); },
           8.0 * n);
    timeit("copy, non-temporal store (cold)", [&](int i) { hipLaunchKernelGGL(copy_k<true>, dim3(grid), dim3(256), 0, 0, a[i % SETS], y[i % SETS], nv); },
           8.0 * n);
    timeit("3 reads + 1 write, a*b+c (cold)",
           [&](int i) { hipLaunchKernelGGL(fma3, dim3(grid), dim3(256), 0, 0, a[i % SETS], b[i % SETS], c[i % SETS], y[i % SETS], nv); },
           16.0 * n);
    timeit("copy, plain store (warm, one buffer pair)", [&](int) { hipLaunchKernelGGL(copy_k<false>, dim3(grid), dim3(256), 0, 0, a[0], y[0], nv); },
           8.0 * n);
    return 0;
}
