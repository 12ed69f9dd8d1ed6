// attention.hip — fused scaled, masked attention for a batch of heads:
//   O_b = softmax(Q_b K_b^T * scale, causal) V_b,  Q_b [tq, dh], K_b, V_b [tk, dh]
// with the arithmetic of cpu_attention (crates/mlx-core/src/cpu_kernels.rs:
// 738-812): scores scaled, the causal entries j > i replaced by -1e9, row
// max, e = exp(x - max), sum, e / sum, then P V.
//
// One 256-thread workgroup (4 waves) owns 16 query rows of one head. Its
// scores stay in LDS for the whole computation, so every score row is
// normalised exactly as the reference does (no running-max rescaling):
//   1. S = Q K^T: the 16 query rows are held in registers as MFMA A
//      fragments; waves take 16-key tiles round-robin and run
//      v_mfma_f32_16x16x4f32 over the head dimension. The reduction index is
//      permuted (lane group g covers head columns g*dh/4 .. g*dh/4 + dh/4 - 1,
//      step s picks one of them), so each lane loads dh/4 contiguous floats
//      of its key row. S*scale goes to LDS.
//   2. Each wave normalises 4 rows: max, exp, sum, divide (the reference's
//      order of operations; sums are taken lane-parallel; the quotient is
//      the correctly rounded one, from the reciprocal and one remainder
//      correction). Masked entries are 0, as exp(-1e9 - max) is.
//   3. O = P V: waves split the keys in four ranges; for 4 keys per step,
//      A = P (LDS), B = V rows (global), one MFMA per 16 output columns. The
//      four partial O tiles are added in wave order (deterministic).
// Keys past the causal horizon of the block's last row are never touched.
#include <algorithm>

#include "../common.hpp"
#include "../kernels.hpp"
#include "device_math.hpp"

#pragma clang fp contract(off)

namespace mlxhip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr int ATT_WAVES = 4;
constexpr int ATT_THREADS = ATT_WAVES * WAVE;
constexpr int QB = 16;  // query rows per workgroup

using dev::div_by;
using dev::shared_divisor;
using dev::wave_max;
using dev::wave_sum;


template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void attn_fused_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ v,
                                                                 float* __restrict__ o, int tq, int tk,
                                                                 int64_t sq, int64_t sk, int64_t sv,
                                                                 int64_t so, float scale, int causal) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    constexpr int DQ = DH / 4;   // head columns per lane group
    constexpr int CT = DH / 16;  // 16-column output tiles
    const int pitch = tk + 1;    // odd: the 16 rows of a column read hit distinct banks
    float* sc = lds;    // [QB][pitch] scores, then probabilities
    float* part = lds;  // [ATT_WAVES][QB][DH] partial O tiles, after the last read of sc

    const int bh = blockIdx.y, q0 = blockIdx.x * QB;
    q += bh * sq;
    k += bh * sk;
    v += bh * sv;
    o += bh * so;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int li = lane & 15, lg = lane >> 4;
    const int kend = causal ? min(tk, q0 + QB) : tk;  // keys any row of the block sees

    // ── 1. scores ─────────────────────────────────────────────────────────
    float qf[DQ];
    {
        const int row = q0 + li;
        const float* qr = q + (int64_t)min(row, tq - 1) * DH + lg * DQ;
#pragma unroll
        for (int s = 0; s < DQ; s += 4) {
            const float4 t = *reinterpret_cast<const float4*>(qr + s);
            qf[s] = t.x; qf[s + 1] = t.y; qf[s + 2] = t.z; qf[s + 3] = t.w;
        }
    }
    // KT key tiles per iteration: all their loads are in flight before the
    // first MFMA.
    constexpr int KT = DH <= 64 ? 4 : 2;
    for (int kt = wave; kt * 16 < kend; kt += KT * ATT_WAVES) {
        float kf[KT][DQ];
#pragma unroll
        for (int h = 0; h < KT; ++h) {
            const int key = (kt + h * ATT_WAVES) * 16 + li;
            const float* kr = k + (int64_t)min(key, tk - 1) * DH + lg * DQ;
#pragma unroll
            for (int s = 0; s < DQ; s += 4) {
                const float4 t = *reinterpret_cast<const float4*>(kr + s);
                kf[h][s] = t.x; kf[h][s + 1] = t.y; kf[h][s + 2] = t.z; kf[h][s + 3] = t.w;
            }
        }
#pragma unroll
        for (int h = 0; h < KT; ++h) {
            const int tile = kt + h * ATT_WAVES;
            const int key = tile * 16 + li;
            if (tile * 16 >= kend) break;
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < DQ; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[s], kf[h][s], acc, 0, 0, 0);
            // D: lane holds key tile*16 + li for query rows 4*lg + r.
            if (key < kend) {
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[(4 * lg + r) * pitch + key] = acc[r] * scale;
            }
        }
    }
    __syncthreads();

    // ── 2. row softmax in LDS ─────────────────────────────────────────────
    // Rows of up to 64*SU keys are normalised in registers (one LDS read and
    // one write per element); longer rows take three passes over LDS.
    constexpr int SU = 8;
    for (int i = wave; i < QB; i += ATT_WAVES) {
        const int row = q0 + i;
        float* sr = sc + i * pitch;
        const int n = causal ? min(kend, row + 1) : kend;  // unmasked keys of this row
        if (row >= tq) {
            for (int j = lane; j < kend; j += WAVE) sr[j] = 0.0f;
            continue;
        }
        if (kend <= WAVE * SU) {
            float x[SU];
            float m = -INFINITY;
#pragma unroll
            for (int u = 0; u < SU; ++u) {
                const int j = lane + WAVE * u;
                x[u] = j < n ? sr[j] : -INFINITY;
                m = fmaxf(m, x[u]);
            }
            m = wave_max(m);
            float sum = 0.0f;
#pragma unroll
            for (int u = 0; u < SU; ++u) {
                const int j = lane + WAVE * u;
                x[u] = j < n ? expf(x[u] - m) : 0.0f;
                sum += x[u];
            }
            sum = wave_sum(sum);
            float r;
            shared_divisor(sum, r);
#pragma unroll
            for (int u = 0; u < SU; ++u) {
                const int j = lane + WAVE * u;
                if (j < kend) sr[j] = div_by(x[u], sum, r);
            }
            continue;
        }
        float m = -INFINITY;
        for (int j = lane; j < n; j += WAVE) m = fmaxf(m, sr[j]);
        m = wave_max(m);
        float sum = 0.0f;
        for (int j = lane; j < n; j += WAVE) {
            const float e = expf(sr[j] - m);
            sr[j] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        for (int j = lane; j < kend; j += WAVE) sr[j] = j < n ? sr[j] / sum : 0.0f;
    }
    __syncthreads();

    // ── 3. O = P V over four key ranges ───────────────────────────────────
    const int k4 = (kend + 3) / 4;                       // 4-key steps
    const int per = (k4 + ATT_WAVES - 1) / ATT_WAVES;    // steps per wave
    const int st0 = wave * per, st1 = min(k4, st0 + per);
    f32x4 acc[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // VB steps per iteration: all their V and P values are loaded first.
    constexpr int VB = DH <= 64 ? 16 : 8;
    for (int st = st0; st < st1; st += VB) {
        float a[VB], b[VB][CT];
#pragma unroll
        for (int u = 0; u < VB; ++u) {
            const int j = 4 * (st + u) + lg;  // this lane's key of the step
            const bool jv = st + u < st1 && j < kend;
            a[u] = jv ? sc[li * pitch + j] : 0.0f;
            const float* vr = v + (int64_t)min(j, tk - 1) * DH + li;
#pragma unroll
            for (int c = 0; c < CT; ++c) b[u][c] = jv ? vr[16 * c] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < VB; ++u)
#pragma unroll
            for (int c = 0; c < CT; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u][c], acc[c], 0, 0, 0);
    }
    __syncthreads();  // every wave is done with sc
    // D: lane holds column 16c + li for query rows 4*lg + r.
    float* pw = part + wave * QB * DH;
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) pw[(4 * lg + r) * DH + 16 * c + li] = acc[c][r];
    __syncthreads();
    for (int e = tid; e < QB * DH; e += ATT_THREADS) {
        const int i = e / DH;
        if (q0 + i >= tq) continue;
        float r = part[e];
#pragma unroll
        for (int w = 1; w < ATT_WAVES; ++w) r += part[w * QB * DH + e];
        o[(int64_t)(q0 + i) * DH + (e - i * DH)] = r;
    }
}

template <int DH>
int launch(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq, int64_t tk,
           int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale, int causal, hipStream_t s) {
    const size_t lds = attention_fused_lds_bytes((int)DH, tk);
    static bool attr = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_fused_kernel<DH>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, ATTN_LDS_LIMIT) == hipSuccess;
    }();
    if (!attr) return fail(MLXHIP_ERR_FFI_FAILED, "attention: hipFuncSetAttribute failed");
    const dim3 grid((unsigned)ceil_div(tq, QB), (unsigned)batch);
    hipLaunchKernelGGL(attn_fused_kernel<DH>, grid, dim3(ATT_THREADS), lds, s, q, k, v, o, (int)tq, (int)tk, sq,
                       sk, sv, so, scale, causal);
    return launch_check("attn_fused_kernel");
}

}  // namespace

size_t attention_fused_lds_bytes(int dh, int64_t tk) {
    return std::max((size_t)QB * (size_t)(tk + 1), (size_t)ATT_WAVES * QB * dh) * sizeof(float);
}

bool attention_fused_supported(int64_t dh, int64_t tq, int64_t tk) {
    if (!(dh == 16 || dh == 32 || dh == 64 || dh == 128)) return false;
    if (tq <= 0 || tk <= 0 || tq > INT32_MAX || (tq + QB - 1) / QB > 65535) return false;
    return attention_fused_lds_bytes((int)dh, tk) <= (size_t)ATTN_LDS_LIMIT;
}

int attention_fused(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq,
                    int64_t tk, int64_t dh, int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale,
                    int causal, hipStream_t s) {
    if (batch <= 0 || batch > 65535) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: batch %lld", (long long)batch);
    if (!attention_fused_supported(dh, tq, tk))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: fused kernel unsupported for dh=%lld tq=%lld tk=%lld",
                    (long long)dh, (long long)tq, (long long)tk);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k);
    if (al % 16 || (sq | sk) % 4)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: Q and K need 16-byte aligned rows");
    switch (dh) {
        case 16: return launch<16>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
        case 32: return launch<32>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
        case 64: return launch<64>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
        default: return launch<128>(q, k, v, o, batch, tq, tk, sq, sk, sv, so, scale, causal, s);
    }
}

}  // namespace mlxhip
