// kernels.hpp — internal launch functions of the HIP kernels. Every function
// enqueues work on stream `s`, validates its sizes on the host first, and
// returns an mlxhip_status_t.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/mlxhip.h"

namespace mlxhip {

// ── rows.hip ──────────────────────────────────────────────────────────────
enum RowOp {
    ROW_SOFTMAX = 0,
    ROW_SCALED_MASKED_SOFTMAX = 1,
    ROW_LAYERNORM = 2,
    ROW_RMSNORM = 3,
    ROW_SOFTMAX_VJP = 4,    // a = dy, b = softmax output
    ROW_LAYERNORM_VJP = 5,  // a = dy, b = x
    ROW_RMSNORM_VJP = 6,    // a = dy, b = x
};
int row_op(int op, const float* a, const float* b, float* y, int64_t rows, int64_t cols, float p,
           int causal, hipStream_t s);
// Softmax (vjp=false) or SoftmaxVjp along a non-last axis of [outer, dim, inner].
int fibre_softmax(bool vjp, const float* a, const float* b, float* y, int64_t outer, int64_t dim,
                  int64_t inner, hipStream_t s);

// ── elementwise.hip ───────────────────────────────────────────────────────
int ew_chain(const mlxhip_ew_instr_t* prog, int n_instr, const float* const* inputs,
             int n_inputs, float* out, int64_t numel, hipStream_t s);
// ew_chain where input i may be periodic: periods[i] > 0 means it holds
// periods[i] values and element j reads in[j % periods[i]] (0 or numel: a
// full-size input). periods may be null.
int ew_chain_periodic(const mlxhip_ew_instr_t* prog, int n_instr, const float* const* inputs,
                      const int64_t* periods, int n_inputs, float* out, int64_t numel, hipStream_t s);
// ew_chain_periodic that also writes the output's three bf16 planes for the
// split-f32 GEMM (the split pass's arithmetic, x6_split), in storage order:
// plane p at planes + p * numel (16-byte aligned), *flag = gen when a value
// cannot be split. *written says whether it did: only the vector kernel
// writes planes (every pointer 16-byte aligned, numel % 4 == 0); otherwise
// the chain runs alone.
int ew_chain_planes(const mlxhip_ew_instr_t* prog, int n_instr, const float* const* inputs, const int64_t* periods,
                    int n_inputs, float* out, int64_t numel, uint16_t* planes, uint32_t* flag, uint32_t gen,
                    bool* written, hipStream_t s);
// General N-D permutation (rank <= 8): y[new] = x[old], out shape = shape[perm].
int permute(const float* x, float* y, const int64_t* shape, const int64_t* perm, int ndim,
            hipStream_t s);
int transpose2d(const float* x, float* y, int64_t rows, int64_t cols, hipStream_t s);
// NumPy right-aligned broadcast (rank <= 8).
int broadcast(const float* x, float* y, const int64_t* in_shape, int in_ndim,
              const int64_t* out_shape, int out_ndim, hipStream_t s);
// Sum/Mean/Max along an axis of [outer, dim, inner]: sequential fold per
// output element in the reference's order (bit-identical to the CPU).
// kind: 0 sum, 1 mean, 2 max.
int reduce_axis(int kind, const float* x, float* y, int64_t outer, int64_t dim, int64_t inner,
                hipStream_t s);
// Reduction of all n elements to y[0]. kind as above.
int reduce_all(int kind, const float* x, float* y, int64_t n, hipStream_t s);
int cast(const void* x, int src, void* y, int dst, int64_t n, hipStream_t s);
// f32 -> bf16/f16 (RNE) of a strided 2-D block [rows, cols] with row pitch
// ld_src into a packed [rows, cols] destination.
int embedding(const float* w, const float* idx, float* y, int64_t n_idx, int64_t num_emb,
              int64_t dim, hipStream_t s);
// Copy of [outer, length, inner] slices starting at `start` of a [outer, dim, inner] tensor.
int narrow(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, int64_t start,
           int64_t length, hipStream_t s);
// Copies src [outer, d, inner] into dst [outer, total, inner] at offset `at` along the axis.
int concat_part(const float* x, float* y, int64_t outer, int64_t d, int64_t inner, int64_t total,
                int64_t at, hipStream_t s);
int rope_interleaved(const float* x, float* y, int64_t tokens, int64_t head_dim,
                     int64_t rotary_dim, int64_t pos_offset, float theta, int64_t len,
                     hipStream_t s);
int rope_mlx(const float* x, float* y, int64_t n_rows, int64_t head_dim, int64_t offset,
             float base, int traditional, hipStream_t s);
int fill(float* y, float v, int64_t n, hipStream_t s);

// ── decode.hip (greedy decode step of a decoder-only model) ───────────────
constexpr int DEC_MAX_BATCH = 8;          // sequences per decode step
constexpr int DEC_LDS_LIMIT = 159 * 1024; // dynamic LDS (a CDNA4 CU has 160 KiB; 1 KiB kept for static LDS)
enum DecEpilogue {
    DEC_EPI_QKV = 1,     // q -> out, k / v -> KV cache at position t
    DEC_EPI_RESID = 2,   // out[b][n] += y (residual stream), and its planes
    DEC_EPI_SILU = 3,    // silu(y) -> planes (and out when set)
    DEC_EPI_ARGMAX = 4,  // logits history (optional) + per-workgroup argmax keys
};
// Y[b][n] = sum_k X[b][k] W[n][k] (+ bias[n]). W is bf16 in MFMA fragment
// order (dec_tiled_index) with its rows padded to a multiple of 16. X is read as
// its three bf16 planes xs[3][DEC_MAX_BATCH][ldxs] (hi, mid, lo; row b of a
// plane is sequence b; hi + mid + lo is the f32 value).
struct DecGemv {
    const uint16_t* w = nullptr;     // fragment-ordered [ceil(N/16)*16][K]
    const uint16_t* bias = nullptr;  // bf16 [N] or null
    const uint16_t* xs = nullptr;    // X planes
    int64_t ldxs = 0;
    float eps = 0.0f;                // RMS-norm eps
    int n = 0, k = 0, batch = 0;
    float* out = nullptr;            // SILU (optional)/RESID: [B, ldo]; QKV: q [B, ldo];
    int64_t ldo = 0;                 // ARGMAX: logits[b*ldo + t*n + n'] (may be null)
    uint16_t* outs = nullptr;        // SILU/RESID: planes of the output [3][DEC_MAX_BATCH][ldos]
    int64_t ldos = 0;
    float* kc = nullptr;             // QKV: K^T cache [B][H][hd][tmax]
    float* vc = nullptr;             // QKV: V cache   [B][H][tmax][hd]
    int dmodel = 0, heads = 0, head_dim = 0, tmax = 0;
    const int* tctr = nullptr;       // device step counter (position t)
    uint64_t* part = nullptr;        // ARGMAX: [groups][DEC_MAX_BATCH] per-workgroup maxima
    int part_capacity = 0;
};
int dec_prepare();
int dec_gemv(int epi, bool norm, const DecGemv& p, hipStream_t s);
int dec_gemv_groups(int n, int k);
// Position of W[n][k] of a [N][K] weight in the GEMV's fragment order: 16-row
// tiles, each a run of 32-k steps of 64 lanes x 8 bf16 (lane = n%16 +
// 16*((k%32)/8)), so one step's A fragments are 1 KB of consecutive memory.
size_t dec_tiled_index(int64_t n, int64_t k, int64_t K);
size_t dec_gemv_lds_bytes(int k, int ks, int r, bool argmax, bool norm);
size_t dec_attn_lds_bytes(int hd, int tmax);
// o of every (sequence, head) into the planes os[3][DEC_MAX_BATCH][heads*hd].
int dec_attention(const float* q, const float* kc, const float* vc, uint16_t* os, int batch, int heads, int hd,
                  int tmax, float scale, const int* tctr, hipStream_t s);
// x [batch][d] and its planes xs[3][DEC_MAX_BATCH][d] = embedding of the tokens at position t.
int dec_embed(const uint16_t* emb, const int* tokens, float* x, uint16_t* xs, int d, int vocab, int batch,
              const int* tctr, hipStream_t s);
// argmax over the LM head's partial maxima, next token (prompt or argmax),
// its embedding into x [batch][d] and its planes, t += 1.
int dec_finish(const uint64_t* part, int groups, int* tokens, int* argmax_out, const uint16_t* emb, float* x,
               uint16_t* xs, int d, int vocab, int batch, int prompt_len, int* tctr, hipStream_t s);
int dec_set_counter(int* p, int v, hipStream_t s);

// ── attention.hip (fused scaled, masked attention of a batch of heads) ────
// dh in {16, 32, 64, 128}; any tq, tk >= 1 (keys are streamed in tiles).
bool attention_fused_supported(int64_t dh, int64_t tq, int64_t tk);
// Q [batch][tq][dh], K/V [batch][tk][dh], O [batch][tq][dh], row-major with
// batch strides sq/sk/sv/so (elements); Q, K, V and O 16-byte aligned.
// With hg > 1, heads sit side by side in rows: head i is columns
// (i % hg) * dh .. +dh of row group i / hg (groups s* floats apart, rows
// rs floats apart; rs = 0 means dh), as in a [groups][t][hg * dh] tensor.
int attention_fused(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq,
                    int64_t tk, int64_t dh, int64_t sq, int64_t sk, int64_t sv, int64_t so, float scale,
                    int causal, hipStream_t s, int64_t hg = 1, int64_t rs = 0);

// ── attention_bwd.hip (gradient of fused attention, dQ / dK / dV) ──────────
// dh == 64, tq == tk a multiple of 64; operands [batch][t][dh], contiguous,
// 16-byte aligned. Scratch (row log-sum-exp and dO.O) comes from the
// stream's WS_ATTN workspace.
bool attention_vjp_supported(int64_t dh, int64_t tq, int64_t tk);
// hg > 1: heads side by side in rows of rs floats, as for attention_fused
// (every operand [batch / hg][t][rs]).
int attention_vjp(const float* q, const float* k, const float* v, const float* o, const float* dout, float* dq,
                  float* dk, float* dv, int64_t batch, int64_t t, int64_t dh, float scale, int causal,
                  hipStream_t s, int64_t hg = 1, int64_t rs = 0);

// ── gemm.hip ──────────────────────────────────────────────────────────────
// bf16 planes of f32 operands (the split-f32 GEMM) made during one graph
// evaluation, kept for its later products of the same stored matrices: a
// node's buffer is written once and not again while the evaluation runs.
// Blocks come from alloc(ctx, bytes) and must outlive the evaluation's
// kernels (the evaluation's Scratch).
struct PlaneCache {
    struct Entry {
        const void* src;
        int64_t ld, stride, rows, cols, batch;
        uint16_t* planes;  // three planes of batch * rows_p * cols_p, then the flag word
        uint32_t* flag;
        uint32_t gen;
    };
    std::vector<Entry> entries;
    void* (*alloc)(void* ctx, size_t bytes) = nullptr;
    void* ctx = nullptr;
};
int gemm(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
         int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
         int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s, PlaneCache* planes = nullptr,
         const float* bias = nullptr);
// Up to 4 f32 products of one shape and layout (C_i = op(A_i) op(B_i),
// rank 2), in one split-f32 launch when gemm_f32_groupable(m, n, k) (the
// products siblings of one graph, such as the Q/K/V projections of one
// input), else one gemm call each. Results within f32 accuracy of separate
// calls (the launch may tile and split them differently).
bool gemm_f32_groupable(int64_t m, int64_t n, int64_t k);
// Whether an f32 product of this shape runs on the split-f32 planes.
bool gemm_f32_reads_planes(int64_t m, int64_t n, int64_t k, int64_t batch);
// A plane block for an f32 operand that a producer splits itself: `src`
// stored contiguously as batch x [rows][cols] (rows and cols multiples of
// 32, so the planes need no padding and hold the operand in storage order),
// entered in `cache` under the key the split-f32 GEMM looks up, so products
// reading src skip its split. *planes stays null (nothing entered) when the
// shape needs padding or the cache cannot allocate. The producer must write
// all three planes (plane p at *planes + p * batch*rows*cols) and store
// *gen into *flag if a value cannot be split, before any product reads it.
int x6_plane_block(PlaneCache* cache, const void* src, int64_t rows, int64_t cols, int64_t batch, uint16_t** planes,
                   uint32_t** flag, uint32_t* gen);
int gemm_f32_grouped(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, int groups, const float* const* a,
                     int64_t lda, const float* const* b, int64_t ldb, float* const* c, int64_t ldc, hipStream_t s,
                     PlaneCache* planes = nullptr, const float* const* bias = nullptr);
// gemm16_small.hip: bf16 / f16 products in one launch of 64 x 64 tiles with
// register-staged, realigned operand loads (any 2-byte-aligned operand, no
// workspace); c_dtype F32 / BF16 / F16.
bool gemm16_small_fits(int64_t m, int64_t n, int64_t k, int64_t batch, int64_t lda, int64_t ldb, int ta, int tb);
int gemm16_small(int ab_dtype, int c_dtype, int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch,
                 const void* a, int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, void* c,
                 int64_t ldc, int64_t sc, hipStream_t s);

// Batched f32 products of attention over many heads (kernels/gemm_thin.hip):
// C = A B^T with K <= 64 (scores), or C [M][64] = op(A) B with B [K][64]
// (head-dimension outputs). gemm_thin_f32 runs whichever fits, on plain
// batch strides; gemm_thin_view on two-level ones: slice bt of an operand
// starts (bt / inner) * s + (bt % inner) * s2 elements past p, its rows ld
// apart (the heads of a [batch, seq, heads * dh] tensor without a permute).
struct ThinView {
    const float* p;
    int64_t ld, s, s2;
};
bool gemm_thin_view_fits(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, int inner,
                         const ThinView& a, const ThinView& b, const ThinView& c);
int gemm_thin_view(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, int inner, const ThinView& a,
                   const ThinView& b, const ThinView& c, hipStream_t s);
bool gemm_thin_f32_fits(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const void* a,
                        int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb, const void* c,
                        int64_t ldc, int64_t sc);
int gemm_thin_f32(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const float* a, int64_t lda,
                  int64_t sa, const float* b, int64_t ldb, int64_t sb, float* c, int64_t ldc, int64_t sc,
                  hipStream_t s);

// gemm_small.hip: f32 products small enough for one or two rounds of 32 x 32
// tiles with K <= 512, one launch, no workspace, any alignment; operand
// slices under 2 GiB.
bool gemm_small_f32_fits(int64_t m, int64_t n, int64_t k, int64_t batch, int64_t lda, int64_t ldb, int ta, int tb);
int gemm_small_f32(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, const float* a, int64_t lda,
                   int64_t sa, const float* b, int64_t ldb, int64_t sb, float* c, int64_t ldc, int64_t sc,
                   hipStream_t s);
// gemm with the same kernels and plan, its split-K partials and padded
// operand copies taken from a fixed device array of
// GEMM_NOALLOC_SCRATCH_BYTES instead of the memory pool: no allocation.
// Calls that overlap on one device share that array and race.
constexpr size_t GEMM_NOALLOC_SCRATCH_BYTES = size_t(64) << 20;
int gemm_noalloc(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                 int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
                 int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s);

}  // namespace mlxhip
