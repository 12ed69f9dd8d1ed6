// attention_bwd.hip — gradient of fused causal attention for a batch of heads.
//
// Forward (the Attention op's arithmetic, cpu_attention in
// crates/mlx-core/src/cpu_kernels.rs:738-812, applied per head):
//   S = scale * Q K^T (keys j > query i excluded when causal),
//   P = softmax(S) over each query row,  O = P V,
// with Q, K, V, O, dO of shape [heads, T, dh]. The reference gives Attention
// no VJP (crates/mlx-autograd/src/vjp.rs:173-176); this is the standard one:
//   L_i = log sum_j exp(S_ij)           (row log-sum-exp)
//   D_i = sum_d dO_id O_id               (= sum_j P_ij dP_ij)
//   P_ij = exp(S_ij - L_i),  dP = dO V^T,  dS = P o (dP - D)
//   dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO.
// Nothing of size T x T is stored: two kernels stream over blocks of 64
// keys (queries) and recompute S and P in registers.
//
//   attn_bwd_dq_kernel, one workgroup per (head, block of 64 queries): a
//   first pass over the visible key blocks computes L (running max and sum
//   per row), the second recomputes P, dP and dS and accumulates dQ. Writes
//   dQ, L and D (for the second kernel).
//   attn_bwd_dkdv_kernel, one workgroup per (head, block of 64 keys): over
//   the query blocks that see them, recomputes P and dS from L and D and
//   accumulates dK and dV.
//
// Products are v_mfma_f32_32x32x2_f32 (exact f32 products, f32 sums). A
// workgroup's 4 waves each own a 32 x 32 tile of the 64 x 64 block: wave w
// takes query half qh = w & 1 and key half kh = w >> 1. For an MFMA lane l,
// c = l % 32 and h = l / 32; the A operand row is c and its k-slot h, the B
// operand column is c, and accumulator element v is row
// 8 (v / 4) + 4 h + v % 4, column c. The first products of a block put the
// lane's own row of one operand in registers (loaded once per workgroup) and
// read the other from LDS; they sum over d with slot (step s, half h) taking
// d = 32 h + s. The second products (dQ, dK, dV) sum over the tile's keys
// (queries) with slot (s, h) taking row 8 (s / 4) + 4 h + s % 4 of the
// first products' accumulator, which is that lane's own element s, so P
// and dS feed the next MFMAs straight from registers. The two waves that
// share a query (key) half hold partial dQ (dK, dV) over the two key (query)
// halves; they are added through LDS at the end.
#include <algorithm>

#include "../common.hpp"
#include "../kernels.hpp"

#pragma clang fp contract(off)

namespace mlxhip {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
// Native vector types throughout: HIP's float4 is a struct whose copies
// compile to memcpy, which kept register arrays of it in scratch memory.
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr int BT = 64;        // queries / keys per block
constexpr int DH = 64;        // head dimension
constexpr int PITCH = DH + 4; // LDS row pitch in floats: 16-byte rows, consecutive rows 4 banks apart
constexpr int THREADS = 4 * WAVE;
constexpr float LOG2E = 1.44269504088896340736f;

__device__ inline int crow(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

__device__ inline void mfma(float a, float b, f32x16& acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
}

__device__ inline f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int v = 0; v < 16; ++v) z[v] = 0.0f;
    return z;
}

// A lane's 32 consecutive floats of an LDS row (16-byte aligned) into
// registers, all reads issued before any use: the MFMAs that consume them
// then wait for the LDS latency once per block, not once per step.
__device__ inline void lds_row32(const float* p, float* r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 t = reinterpret_cast<const f32x4*>(p)[i];
        r[4 * i] = t[0], r[4 * i + 1] = t[1], r[4 * i + 2] = t[2], r[4 * i + 3] = t[3];
    }
}

// 2^x on the hardware exponential; x <= 0 here (a score minus its row's
// log-sum-exp), relative error about |x| 2^-24 plus one ulp.
__device__ inline float exp2_small(float x) { return __builtin_amdgcn_exp2f(x); }

// Offset of head `head`'s first row: head % hg of row group head / hg, the
// groups T rows of rs floats each (hg = 1, rs = DH: [heads][T][DH]).
__device__ inline int64_t head_offset(int64_t head, int T, int hg, int rs) {
    return (head / hg) * (int64_t)T * rs + (head % hg) * DH;
}

// Lane l's 32 values of row `row` of a head (rows rs floats apart): d = 32 h + s, s < 32.
__device__ inline void load_row_half(const float* __restrict__ head, int row, int rs, int h, float* r) {
    const f32x4* p = reinterpret_cast<const f32x4*>(head + (int64_t)row * rs + 32 * h);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 t = p[i];
        r[4 * i] = t[0], r[4 * i + 1] = t[1], r[4 * i + 2] = t[2], r[4 * i + 3] = t[3];
    }
}

// A 64 x DH block of rows row0 .. row0+63 of a head into registers (4 vectors
// per thread), then into LDS rows of PITCH floats.
__device__ inline void block_load(const float* __restrict__ head, int row0, int rs, int tid, f32x4 (&r)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = (i * THREADS + tid) * 4;  // element in the block
        r[i] = *reinterpret_cast<const f32x4*>(head + (int64_t)(row0 + e / DH) * rs + e % DH);
    }
}
__device__ inline void block_store(float* lds, int tid, const f32x4 (&r)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = (i * THREADS + tid) * 4;
        *reinterpret_cast<f32x4*>(lds + (e / DH) * PITCH + e % DH) = r[i];
    }
}

// Workgroup id -> (head, block). Under the causal mask a block's work grows
// with its index (dQ: key blocks 0..qb) or shrinks (dK/dV: query blocks
// kb..nb-1). Two workgroups run on each CU at once, and the dispatcher fills
// one slot on every CU with the first half of the ids before the second
// slot: ids i and i + half are paired as blocks b and nb - 1 - b of one
// head, so every CU gets the same work. `heavy_high`: block nb - 1 is the
// heaviest (dQ) rather than block 0 (dK/dV).
__device__ inline void block_of(int id, int heads, int nb, bool heavy_high, int* head, int* blk) {
    const int hp = nb / 2, half = heads * hp;
    int b;
    if (id < half) {                 // the heavier block of each pair
        *head = id / hp;
        b = nb - 1 - id % hp;
    } else if (id < 2 * half) {      // its partner
        const int j = id - half;
        *head = j / hp;
        b = j % hp;
    } else {                         // odd nb: the middle block of each head
        *head = id - 2 * half;
        b = hp;
    }
    *blk = heavy_high ? b : nb - 1 - b;
}

// ── dQ, L, D ───────────────────────────────────────────────────────────────
// S^T tile = K Q^T (rows keys, columns queries): the lane's column is query
// q = qb*64 + 32 qh + c, so L_q and D_q are per-lane scalars.
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dq_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                               const float* __restrict__ V, const float* __restrict__ O,
                                                               const float* __restrict__ dO, float* __restrict__ dQ,
                                                               float* __restrict__ lse_out, float* __restrict__ d_out,
                                                               int T, float scale, int causal, int hg, int rs) {
    // K and V blocks; at the end the kh = 1 partials of dQ ([qh][64 d][33]).
    __shared__ __align__(16) float smem[2 * BT * PITCH];
    __shared__ float xch[2][2][32][2];  // (m, l) per query half, key half, query
    float* Ks = smem;
    float* Vs = smem + BT * PITCH;
    const int nqb = T / BT;
    int head_i, qb;
    block_of((int)blockIdx.x, (int)(gridDim.x / nqb), nqb, true, &head_i, &qb);
    const int64_t head = head_i;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int qh = wave & 1, kh = wave >> 1, c = lane & 31, h = lane >> 5;
    const int64_t hoff = head_offset(head, T, hg, rs);
    const float *Qh = Q + hoff, *Kh = K + hoff, *Vh = V + hoff, *Oh = O + hoff, *dOh = dO + hoff;
    const int q = qb * BT + 32 * qh + c;

    float qr[32], dor[32];
    load_row_half(Qh, q, rs, h, qr);
    load_row_half(dOh, q, rs, h, dor);
    float Dq;
    {
        float orow[32];
        load_row_half(Oh, q, rs, h, orow);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) s += dor[i] * orow[i];
        Dq = s + __shfl_xor(s, 32, WAVE);
    }
    const int nkb = causal ? qb + 1 : nqb;
    f32x4 kc[4], vc[4];

    // Pass 1: L_q. Lanes c and c + 32 see different key rows of the same
    // query, and the two waves of a query half different key halves: their
    // (m, l) pairs are combined in a fixed order (lanes, then kh 0 before
    // kh 1), so both waves get the same L_q.
    // Blocks are staged without prefetch: two workgroups share each CU and
    // one computes while the other waits for its loads (registers for a
    // prefetch would leave room for only one).
    float m = -INFINITY, l = 0.0f;
    for (int kb = 0; kb < nkb; ++kb) {
        block_load(Kh, kb * BT, rs, tid, kc);
        __syncthreads();  // the previous block's readers are done
        block_store(Ks, tid, kc);
        __syncthreads();
        // Two independent accumulator chains (step s feeds chain s % 2),
        // summed in chain order: one chain of dependent MFMAs runs at about
        // half the matrix pipe's rate. Pass 2 sums S the same way.
        f32x16 s2[2] = {zero16(), zero16()};
        float kr[32];
        lds_row32(Ks + (32 * kh + c) * PITCH + 32 * h, kr);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 32; ++s) mfma(kr[s], qr[s], s2[s & 1]);
        const f32x16 sa = s2[0] + s2[1];
        float x[16], mt = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = kb * BT + 32 * kh + crow(v, h);
            x[v] = (causal && key > q) ? -INFINITY : sa[v] * scale;
            mt = fmaxf(mt, x[v]);
        }
        const float mn = fmaxf(m, mt);
        if (mn != -INFINITY) {
            float acc = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) acc += exp2_small((x[v] - mn) * LOG2E);
            l = l * exp2_small((m - mn) * LOG2E) + acc;
            m = mn;
        }
    }
    {
        const float m2 = __shfl_xor(m, 32, WAVE), l2 = __shfl_xor(l, 32, WAVE);
        const float mn = fmaxf(m, m2);
        l = (m == -INFINITY ? 0.0f : l * exp2_small((m - mn) * LOG2E)) +
            (m2 == -INFINITY ? 0.0f : l2 * exp2_small((m2 - mn) * LOG2E));
        m = mn;
    }
    if (h == 0) {
        xch[qh][kh][c][0] = m;
        xch[qh][kh][c][1] = l;
    }
    __syncthreads();
    {
        const float m0 = xch[qh][0][c][0], l0 = xch[qh][0][c][1];
        const float m1 = xch[qh][1][c][0], l1 = xch[qh][1][c][1];
        const float mn = fmaxf(m0, m1);
        l = (m0 == -INFINITY ? 0.0f : l0 * exp2_small((m0 - mn) * LOG2E)) +
            (m1 == -INFINITY ? 0.0f : l1 * exp2_small((m1 - mn) * LOG2E));
        m = mn;
    }
    const float Lq = m + logf(l);
    if (kh == 0 && h == 0) {
        lse_out[head * T + q] = Lq;
        d_out[head * T + q] = Dq;
    }

    // Pass 2: dQ^T (rows d, columns queries) += K^T dS^T over the wave's keys.
    f32x16 dq0 = zero16(), dq1 = zero16();
    for (int kb = 0; kb < nkb; ++kb) {
        block_load(Kh, kb * BT, rs, tid, kc);
        block_load(Vh, kb * BT, rs, tid, vc);
        __syncthreads();
        block_store(Ks, tid, kc);
        block_store(Vs, tid, vc);
        __syncthreads();
        f32x16 s2[2] = {zero16(), zero16()}, p2[2] = {zero16(), zero16()};
        // Two halves of 16 steps, each half's LDS reads issued before its MFMAs.
#pragma unroll
        for (int s0 = 0; s0 < 32; s0 += 16) {
            float kr[16], vr[16];
            const f32x4* kp = reinterpret_cast<const f32x4*>(Ks + (32 * kh + c) * PITCH + 32 * h + s0);
            const f32x4* vp = reinterpret_cast<const f32x4*>(Vs + (32 * kh + c) * PITCH + 32 * h + s0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 a = kp[i], b = vp[i];
                kr[4 * i] = a[0], kr[4 * i + 1] = a[1], kr[4 * i + 2] = a[2], kr[4 * i + 3] = a[3];
                vr[4 * i] = b[0], vr[4 * i + 1] = b[1], vr[4 * i + 2] = b[2], vr[4 * i + 3] = b[3];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                mfma(kr[i], qr[s0 + i], s2[i & 1]);     // S^T, as in pass 1
                mfma(vr[i], dor[s0 + i], p2[i & 1]);    // dP^T = V dO^T
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const f32x16 sa = s2[0] + s2[1];
        const f32x16 pa = p2[0] + p2[1];
        float ds[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = kb * BT + 32 * kh + crow(v, h);
            const float p = (causal && key > q) ? 0.0f : exp2_small((sa[v] * scale - Lq) * LOG2E);
            ds[v] = p * (pa[v] - Dq);
        }
        // Slot (s, h) is key 32 kh + crow(s, h): this lane's ds[s].
        float ka[16], kb2[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float* kk = Ks + (32 * kh + crow(s, h)) * PITCH + c;
            ka[s] = kk[0];
            kb2[s] = kk[32];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            mfma(ka[s], ds[s], dq0);
            mfma(kb2[s], ds[s], dq1);
        }
    }
    // Add the kh = 1 partials into the kh = 0 waves, then write dQ.
    __syncthreads();
    float* part = smem;  // [qh][64 d][32 queries], pitch 33
    if (kh == 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            part[(qh * 64 + crow(v, h)) * 33 + c] = dq0[v];
            part[(qh * 64 + 32 + crow(v, h)) * 33 + c] = dq1[v];
        }
    }
    __syncthreads();
    if (kh == 0) {
        float* out = dQ + hoff + (int64_t)q * rs;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 a, b;
            const int d0 = 8 * g + 4 * h;
            a.x = (dq0[4 * g + 0] + part[(qh * 64 + d0 + 0) * 33 + c]) * scale;
            a.y = (dq0[4 * g + 1] + part[(qh * 64 + d0 + 1) * 33 + c]) * scale;
            a.z = (dq0[4 * g + 2] + part[(qh * 64 + d0 + 2) * 33 + c]) * scale;
            a.w = (dq0[4 * g + 3] + part[(qh * 64 + d0 + 3) * 33 + c]) * scale;
            b.x = (dq1[4 * g + 0] + part[(qh * 64 + 32 + d0 + 0) * 33 + c]) * scale;
            b.y = (dq1[4 * g + 1] + part[(qh * 64 + 32 + d0 + 1) * 33 + c]) * scale;
            b.z = (dq1[4 * g + 2] + part[(qh * 64 + 32 + d0 + 2) * 33 + c]) * scale;
            b.w = (dq1[4 * g + 3] + part[(qh * 64 + 32 + d0 + 3) * 33 + c]) * scale;
            *reinterpret_cast<f32x4*>(out + d0) = a;
            *reinterpret_cast<f32x4*>(out + 32 + d0) = b;
        }
    }
}

// ── dK, dV ─────────────────────────────────────────────────────────────────
// S tile = Q K^T (rows queries, columns keys): the lane's column is key
// j = kb*64 + 32 kh + c; L and D of its 16 query rows come from LDS.
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dkdv_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                                 const float* __restrict__ V, const float* __restrict__ dO,
                                                                 const float* __restrict__ lse, const float* __restrict__ dd,
                                                                 float* __restrict__ dK, float* __restrict__ dV, int T,
                                                                 float scale, int causal, int hg, int rs) {
    // Q and dO blocks; at the end the qh = 1 partials ([kh][dK 64 + dV 64][33]).
    constexpr int SMEM = 2 * BT * PITCH > 2 * 128 * 33 ? 2 * BT * PITCH : 2 * 128 * 33;
    __shared__ __align__(16) float smem[SMEM];
    // L and D of the block's queries; slot BT takes the (unused) values of
    // the threads past the block, so every thread stores without a branch
    // (loads that only feed a store under a branch were sunk into it and
    // issued one at a time behind spilled addresses).
    __shared__ float Ls[BT + 1], Ds[BT + 1];
    float* Qs = smem;
    float* dOs = smem + BT * PITCH;
    const int nkb = T / BT;
    int head_i, kb;
    block_of((int)blockIdx.x, (int)(gridDim.x / nkb), nkb, false, &head_i, &kb);
    const int64_t head = head_i;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int qh = wave & 1, kh = wave >> 1, c = lane & 31, h = lane >> 5;
    const int64_t hoff = head_offset(head, T, hg, rs);
    const float *Qh = Q + hoff, *Kh = K + hoff, *Vh = V + hoff, *dOh = dO + hoff;
    const int j = kb * BT + 32 * kh + c;

    float kr[32], vr[32];
    load_row_half(Kh, j, rs, h, kr);
    load_row_half(Vh, j, rs, h, vr);
    f32x16 dk0 = zero16(), dk1 = zero16(), dv0 = zero16(), dv1 = zero16();
    // Blocks staged without prefetch (two workgroups per CU, as in the dQ kernel).
    f32x4 qc[4], oc[4];
    const int qb0 = causal ? kb : 0, nqb = T / BT;
    const int lrow = tid < BT ? tid : 0, lslot = tid < BT ? tid : BT;
    const float* lse_h = lse + head * T;  // the head's L and D (uniform bases)
    const float* dd_h = dd + head * T;
    for (int qb = qb0; qb < nqb; ++qb) {
        // L and D first: gfx9 waits for loads in issue order, so the Q / dO
        // loads behind them do not hold up their stores.
        const float lv = lse_h[qb * BT + lrow], dv = dd_h[qb * BT + lrow];
        block_load(Qh, qb * BT, rs, tid, qc);
        block_load(dOh, qb * BT, rs, tid, oc);
        __syncthreads();
        block_store(Qs, tid, qc);
        block_store(dOs, tid, oc);
        Ls[lslot] = lv;
        Ds[lslot] = dv;
        __syncthreads();
        f32x16 s2[2] = {zero16(), zero16()}, p2[2] = {zero16(), zero16()};
        // Two halves of 16 steps, each half's LDS reads issued before its MFMAs.
#pragma unroll
        for (int s0 = 0; s0 < 32; s0 += 16) {
            float qrow[16], orow[16];
            const f32x4* qp = reinterpret_cast<const f32x4*>(Qs + (32 * qh + c) * PITCH + 32 * h + s0);
            const f32x4* op = reinterpret_cast<const f32x4*>(dOs + (32 * qh + c) * PITCH + 32 * h + s0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 a = qp[i], b = op[i];
                qrow[4 * i] = a[0], qrow[4 * i + 1] = a[1], qrow[4 * i + 2] = a[2], qrow[4 * i + 3] = a[3];
                orow[4 * i] = b[0], orow[4 * i + 1] = b[1], orow[4 * i + 2] = b[2], orow[4 * i + 3] = b[3];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                mfma(qrow[i], kr[s0 + i], s2[i & 1]);  // S = Q K^T (chains as in the dQ kernel)
                mfma(orow[i], vr[s0 + i], p2[i & 1]);  // dP = dO V^T
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const f32x16 sa = s2[0] + s2[1];
        const f32x16 pa = p2[0] + p2[1];
        float p[16], ds[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int qi = 32 * qh + crow(v, h);
            const bool masked = causal && j > qb * BT + qi;
            p[v] = masked ? 0.0f : exp2_small((sa[v] * scale - Ls[qi]) * LOG2E);
            ds[v] = p[v] * (pa[v] - Ds[qi]);
        }
        // dV^T (rows d, columns keys) += dO^T P, dK^T += Q^T dS; slot (s, h)
        // is query 32 qh + crow(s, h): this lane's p[s] and ds[s].
        // Two halves of 8 steps, each half's LDS reads issued before its MFMAs.
#pragma unroll
        for (int s0 = 0; s0 < 16; s0 += 8) {
            float oa[8], ob[8], qa[8], qb2[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int qi = 32 * qh + crow(s0 + i, h);
                oa[i] = dOs[qi * PITCH + c];
                ob[i] = dOs[qi * PITCH + 32 + c];
                qa[i] = Qs[qi * PITCH + c];
                qb2[i] = Qs[qi * PITCH + 32 + c];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                mfma(oa[i], p[s0 + i], dv0);
                mfma(ob[i], p[s0 + i], dv1);
                mfma(qa[i], ds[s0 + i], dk0);
                mfma(qb2[i], ds[s0 + i], dk1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Add the qh = 1 partials into the qh = 0 waves, then write dK and dV.
    __syncthreads();
    float* part = smem;  // [kh][128 rows: dK d 0..63, dV d 0..63][32 keys], pitch 33
    if (qh == 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            part[(kh * 128 + crow(v, h)) * 33 + c] = dk0[v];
            part[(kh * 128 + 32 + crow(v, h)) * 33 + c] = dk1[v];
            part[(kh * 128 + 64 + crow(v, h)) * 33 + c] = dv0[v];
            part[(kh * 128 + 96 + crow(v, h)) * 33 + c] = dv1[v];
        }
    }
    __syncthreads();
    if (qh == 0) {
        float* ok = dK + hoff + (int64_t)j * rs;
        float* ov = dV + hoff + (int64_t)j * rs;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 8 * g + 4 * h;
            f32x4 a, b, e, f;
            a.x = (dk0[4 * g + 0] + part[(kh * 128 + d0 + 0) * 33 + c]) * scale;
            a.y = (dk0[4 * g + 1] + part[(kh * 128 + d0 + 1) * 33 + c]) * scale;
            a.z = (dk0[4 * g + 2] + part[(kh * 128 + d0 + 2) * 33 + c]) * scale;
            a.w = (dk0[4 * g + 3] + part[(kh * 128 + d0 + 3) * 33 + c]) * scale;
            b.x = (dk1[4 * g + 0] + part[(kh * 128 + 32 + d0 + 0) * 33 + c]) * scale;
            b.y = (dk1[4 * g + 1] + part[(kh * 128 + 32 + d0 + 1) * 33 + c]) * scale;
            b.z = (dk1[4 * g + 2] + part[(kh * 128 + 32 + d0 + 2) * 33 + c]) * scale;
            b.w = (dk1[4 * g + 3] + part[(kh * 128 + 32 + d0 + 3) * 33 + c]) * scale;
            e.x = dv0[4 * g + 0] + part[(kh * 128 + 64 + d0 + 0) * 33 + c];
            e.y = dv0[4 * g + 1] + part[(kh * 128 + 64 + d0 + 1) * 33 + c];
            e.z = dv0[4 * g + 2] + part[(kh * 128 + 64 + d0 + 2) * 33 + c];
            e.w = dv0[4 * g + 3] + part[(kh * 128 + 64 + d0 + 3) * 33 + c];
            f.x = dv1[4 * g + 0] + part[(kh * 128 + 96 + d0 + 0) * 33 + c];
            f.y = dv1[4 * g + 1] + part[(kh * 128 + 96 + d0 + 1) * 33 + c];
            f.z = dv1[4 * g + 2] + part[(kh * 128 + 96 + d0 + 2) * 33 + c];
            f.w = dv1[4 * g + 3] + part[(kh * 128 + 96 + d0 + 3) * 33 + c];
            *reinterpret_cast<f32x4*>(ok + d0) = a;
            *reinterpret_cast<f32x4*>(ok + 32 + d0) = b;
            *reinterpret_cast<f32x4*>(ov + d0) = e;
            *reinterpret_cast<f32x4*>(ov + 32 + d0) = f;
        }
    }
}

}  // namespace

bool attention_vjp_supported(int64_t dh, int64_t tq, int64_t tk) {
    return dh == DH && tq == tk && tq > 0 && tq % BT == 0 && tq <= (1 << 20);
}

int attention_vjp(const float* q, const float* k, const float* v, const float* o, const float* dout, float* dq,
                  float* dk, float* dv, int64_t batch, int64_t t, int64_t dh, float scale, int causal,
                  hipStream_t s, int64_t hg, int64_t rs) {
    if (batch <= 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention vjp: batch %lld", (long long)batch);
    if (rs == 0) rs = dh;
    if (hg < 1 || batch % hg || rs < hg * dh || rs % 4 || rs > INT32_MAX || hg > INT32_MAX ||
        (batch / hg) * t * rs >= ((int64_t)1 << 40))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention vjp: %lld heads per row of %lld floats (dh %lld, batch %lld)",
                    (long long)hg, (long long)rs, (long long)dh, (long long)batch);
    if (!attention_vjp_supported(dh, t, t))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT,
                    "attention vjp: needs dh = %d and a sequence length that is a multiple of %d (dh=%lld t=%lld)", DH,
                    BT, (long long)dh, (long long)t);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o) |
                         reinterpret_cast<uintptr_t>(dout) | reinterpret_cast<uintptr_t>(dq) |
                         reinterpret_cast<uintptr_t>(dk) | reinterpret_cast<uintptr_t>(dv);
    if (al % 16) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention vjp: operands must be 16-byte aligned");
    const int64_t blocks = batch * (t / BT);
    if (blocks > int64_t(UINT32_MAX) / THREADS)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention vjp: %lld heads exceed one launch", (long long)batch);
    // L and D of every query row: [batch][t] each, in the stream's workspace.
    void* ws = nullptr;
    MLXHIP_TRY(stream_workspace(s, WS_ATTN, (size_t)(2 * batch * t) * sizeof(float), &ws));
    float* lse = static_cast<float*>(ws);
    float* dd = lse + batch * t;
    hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3((unsigned)blocks), dim3(THREADS), 0, s, q, k, v, o, dout, dq, lse, dd,
                       (int)t, scale, causal, (int)hg, (int)rs);
    MLXHIP_TRY(launch_check("attn_bwd_dq_kernel"));
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel, dim3((unsigned)blocks), dim3(THREADS), 0, s, q, k, v, dout, lse, dd, dk,
                       dv, (int)t, scale, causal, (int)hg, (int)rs);
    return launch_check("attn_bwd_dkdv_kernel");
}

}  // namespace mlxhip
