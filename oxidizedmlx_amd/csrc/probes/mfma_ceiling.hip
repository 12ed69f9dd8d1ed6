// mfma_ceiling.hip — sustained v_mfma_f32_32x32x16_bf16 / 16x16x32_bf16 rate
// on every SIMD of the GPU, with random and with all-zero operands.
//
// Measurement tool, not part of libmlxhip.so. It bounds what any bf16 GEMM
// can reach on this part: each wave issues independent MFMAs back to back on
// register-resident operands (no memory traffic), so the only limits are the
// matrix pipe and the clock the chip holds under that load, which depends on
// how much the operand bits toggle.
// Build: python -m oxidizedmlx_amd.build --probes; run: oxidizedmlx_amd/_build/mfma_ceiling
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define CK(x)                                                                         \
    do {                                                                              \
        hipError_t e = (x);                                                           \
        if (e != hipSuccess) {                                                        \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__); \
            std::exit(3);                                                             \
        }                                                                             \
    } while (0)

// NACC independent 32x32x16 accumulators per wave, issued back to back.
template <int NACC>
__global__ __launch_bounds__(256) void mfma32(const bf16x8* in, float* out, int iters) {
    const bf16x8 a = in[threadIdx.x], b = in[threadIdx.x + 256];
    f32x16 acc[NACC];
    for (int i = 0; i < NACC; ++i)
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < NACC; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i], 0, 0, 0);
    }
    float s = 0;
    for (int i = 0; i < NACC; ++i)
        for (int v = 0; v < 16; ++v) s += acc[i][v];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <int NACC>
__global__ __launch_bounds__(256) void mfma16(const bf16x8* in, float* out, int iters) {
    const bf16x8 a = in[threadIdx.x], b = in[threadIdx.x + 256];
    f32x4 acc[NACC];
    for (int i = 0; i < NACC; ++i)
        for (int v = 0; v < 4; ++v) acc[i][v] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < NACC; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[i], 0, 0, 0);
    }
    float s = 0;
    for (int i = 0; i < NACC; ++i)
        for (int v = 0; v < 4; ++v) s += acc[i][v];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <typename F>
void timeit(const char* name, F launch, double flops) {
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    launch();
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0, 0));
    for (int r = 0; r < 5; ++r) launch();
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, e0, e1));
    ms /= 5;
    const double tf = flops / (ms * 1e-3) / 1e12;
    std::printf("%-50s %8.1f us %8.1f TFLOP/s %5.1f%% of 2516.6\n", name, ms * 1e3, tf, 100 * tf / 2516.6);
    std::fflush(stdout);
}

int main() {
    // bf16 operands with random sign and mantissa bits, exponent near 1.0.
    std::vector<uint16_t> h(512 * 8);
    uint32_t s = 7;
    for (auto& v : h) {
        s = s * 1664525u + 1013904223u;
        v = (uint16_t)((0x3f00 + ((s >> 20) & 0xff)) ^ ((s >> 8) & 0x8000));
    }
    bf16x8 *rnd, *zero;
    float* out;
    CK(hipMalloc(&rnd, h.size() * 2));
    CK(hipMalloc(&zero, h.size() * 2));
    CK(hipMalloc(&out, 1 << 24));
    CK(hipMemcpy(rnd, h.data(), h.size() * 2, hipMemcpyHostToDevice));
    CK(hipMemset(zero, 0, h.size() * 2));
    const int iters = 2048;
    const double f32x = 2.0 * 32 * 32 * 16, f16x = 2.0 * 16 * 16 * 32;
    for (int z = 0; z < 2; ++z) {
        const bf16x8* in = z ? zero : rnd;
        const char* tag = z ? "zero operands" : "random operands";
        char nm[128];
        std::snprintf(nm, sizeof nm, "32x32x16, 16 acc, 1 wave/SIMD, %s", tag);
        timeit(nm, [&] { hipLaunchKernelGGL(mfma32<16>, dim3(256), dim3(256), 0, 0, in, out, iters); },
               256.0 * 4 * 16 * iters * f32x);
        std::snprintf(nm, sizeof nm, "32x32x16, 8 acc, 2 waves/SIMD, %s", tag);
        timeit(nm, [&] { hipLaunchKernelGGL(mfma32<8>, dim3(512), dim3(256), 0, 0, in, out, iters); },
               512.0 * 4 * 8 * iters * f32x);
        std::snprintf(nm, sizeof nm, "16x16x32, 16 acc, 2 waves/SIMD, %s", tag);
        timeit(nm, [&] { hipLaunchKernelGGL(mfma16<16>, dim3(512), dim3(256), 0, 0, in, out, iters); },
               512.0 * 4 * 16 * iters * f16x);
    }
    return 0;
}
