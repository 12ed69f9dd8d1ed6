/*
 * mlx_cpu_ref.c — CPU oracle (TEST INFRASTRUCTURE ONLY; see mlx_cpu_ref.h).
 *
 * Restates CpuRefBackend (crates/mlx-core/src/cpu_kernels.rs) op by op, with
 * the reference's loop orders, sequential f32 folds, divide-versus-multiply
 * choices and libm calls. Compiled with -ffp-contract=off so no a*b+c is
 * fused. Rust's `Iterator::sum::<f32>()` folds from -0.0 on current stable
 * (the reference pins `stable`, edition 2024), so `.sum()` restatements here
 * start from -0.0f; explicit `let mut s = 0.0f32` loops start from +0.0f.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   matmul, add/sub/mul/div/neg, transpose, broadcast, reshape, narrow,
 *   concatenate, sum/mean/max, embedding:
 *       the reference's known answers (cpu_kernels.rs:980-1079,
 *       tensor.rs:905-969, parity_gate.rs:71-83) plus brute force against
 *       numpy float64 / exact integer-valued inputs.
 *   softmax, layer_norm, rms_norm, scaled_masked_softmax, attention:
 *       closed forms of the reference's tests (parity_gate.rs:107-169,
 *       mlx-nn/src/lib.rs:81-91,173-183) and float64 numpy re-derivations
 *       within f32 rounding, plus invariants (rows sum to 1, mean 0 / var 1).
 *   exp, log, sqrt, silu, gelu: glibc libm called exactly as Rust std does;
 *       known answers SiLU(1)=0.7311, SiLU(-1)=-0.2689 (cpu_kernels.rs:1081-1091)
 *       and float64 numpy within 4 ulp.
 *   *_vjp: central finite differences of the forward oracle (the
 *       reference's own method, crates/mlx-autograd/src/lib.rs:157-175) and
 *       the LayerNorm invariant "grad rows sum to 0" (autograd/src/vjp.rs:236-261).
 *   rope (Rope and RoPE): the reference's known answer (cpu_kernels.rs:1093-1127)
 *       and closed forms on one-hot inputs: each pair rotates by the angle
 *       (offset + row) * base^(-2d/hd) into (cos, sin) / (-sin, cos) on the
 *       pair (2d, 2d+1) (traditional, and Rope) or (d, d+hd/2), every other
 *       output zero, dims past rotary_dim unchanged.
 *   gen_data: integer LCG restated; checked for determinism, range and a
 *       float64 re-derivation with Python integers.
 */
#include "mlx_cpu_ref.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static _Thread_local char g_err[512];

static int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

const char* oracle_last_error(void) { return g_err; }
void oracle_free(float* p) { free(p); }

/* ── helpers ─────────────────────────────────────────────────────────────── */

static size_t prod(const int64_t* s, size_t lo, size_t hi) {
    size_t p = 1;
    for (size_t i = lo; i < hi; ++i) p *= (size_t)s[i];
    return p;
}

static float* alloc_out(size_t n) {
    /* malloc(0) may return NULL; always hand back a valid pointer. */
    float* p = (float*)malloc(n ? n * sizeof(float) : sizeof(float));
    return p;
}

/* require_input (cpu_kernels.rs:108-112) */
#define REQUIRE(idx)                                                                    \
    do {                                                                                \
        if ((size_t)(idx) >= n_inputs)                                                  \
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "expected input at index %d", idx); \
    } while (0)

/* sigmoid (cpu_kernels.rs:104-106) */
static float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* Gelu forward, tanh approximation (cpu_kernels.rs:55-67). */
static float gelu(float x) {
    const float k = sqrtf(2.0f / (float)3.14159265358979323846);
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

/* ── gen_data (crates/mlx-parity/src/lib.rs:22-39) ───────────────────────── */

void oracle_gen_data(float* out, size_t n, uint64_t seed) {
    uint64_t state = seed;
    for (size_t i = 0; i < n; ++i) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        double v = (double)(state >> 33) / (double)(1ULL << 31) * 2.0 - 1.0;
        out[i] = (float)v;
    }
}

void oracle_gen_positive_data(float* out, size_t n, uint64_t seed) {
    oracle_gen_data(out, n, seed);
    for (size_t i = 0; i < n; ++i) out[i] = fabsf(out[i]) + 0.01f;
}

/* ── matmul (cpu_kernels.rs:197-230): i-j-p, sequential sum from 0.0 ─────── */

void oracle_matmul_rows(const float* a, const float* b, float* c, size_t m, size_t k,
                        size_t n, size_t row0, size_t nrows) {
    (void)m;
    for (size_t i = row0; i < row0 + nrows; ++i) {
        for (size_t j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p) sum += a[i * k + p] * b[p * n + j];
            c[i * n + j] = sum;
        }
    }
}

void oracle_matmul(const float* a, const float* b, float* c, size_t m, size_t k, size_t n) {
    oracle_matmul_rows(a, b, c, m, k, n, 0, m);
}

/* ── softmax (cpu_kernels.rs:276-315) ─────────────────────────────────────── */

static void softmax_fibres(float* data, size_t outer, size_t dim, size_t inner) {
    for (size_t o = 0; o < outer; ++o) {
        for (size_t i = 0; i < inner; ++i) {
            float max_val = -INFINITY;
            for (size_t d = 0; d < dim; ++d) {
                size_t idx = o * dim * inner + d * inner + i;
                if (data[idx] > max_val) max_val = data[idx];
            }
            float sum_exp = 0.0f;
            for (size_t d = 0; d < dim; ++d) {
                size_t idx = o * dim * inner + d * inner + i;
                data[idx] = expf(data[idx] - max_val);
                sum_exp += data[idx];
            }
            for (size_t d = 0; d < dim; ++d) {
                size_t idx = o * dim * inner + d * inner + i;
                data[idx] /= sum_exp;
            }
        }
    }
}

void oracle_softmax_lastdim(const float* x, float* y, size_t rows, size_t cols) {
    memcpy(y, x, rows * cols * sizeof(float));
    softmax_fibres(y, rows, cols, 1);
}

/* ── layer_norm (cpu_kernels.rs:338-363) ──────────────────────────────────── */

void oracle_layer_norm(const float* x, float* y, size_t rows, size_t d, float eps) {
    for (size_t o = 0; o < rows; ++o) {
        const float* s = x + o * d;
        float acc = -0.0f;
        for (size_t i = 0; i < d; ++i) acc += s[i];
        float mean = acc / (float)d;
        float vacc = -0.0f;
        for (size_t i = 0; i < d; ++i) vacc += (s[i] - mean) * (s[i] - mean);
        float var = vacc / (float)d;
        float sd = sqrtf(var + eps);
        for (size_t i = 0; i < d; ++i) y[o * d + i] = (s[i] - mean) / sd;
    }
}

/* ── rms_norm (cpu_kernels.rs:647-669) ────────────────────────────────────── */

void oracle_rms_norm(const float* x, float* y, size_t rows, size_t d, float eps) {
    for (size_t o = 0; o < rows; ++o) {
        const float* s = x + o * d;
        float acc = -0.0f;
        for (size_t i = 0; i < d; ++i) acc += s[i] * s[i];
        float rms = sqrtf(acc / (float)d + eps);
        for (size_t i = 0; i < d; ++i) y[o * d + i] = s[i] / rms;
    }
}

/* ── per-op implementations with the reference's checks ──────────────────── */

typedef struct {
    const mlxhip_op_t* op;
    const mlxhip_input_t* in;
    size_t n_inputs;
    const mlxhip_meta_t* meta;
    float** out;
    size_t* out_len;
} ctx_t;

static int binary(ctx_t* c, int kind) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t* a = &c->in[0];
    const mlxhip_input_t* b = &c->in[1];
    if (a->len != b->len) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "binary: length %zu vs %zu", a->len, b->len);
    float* r = alloc_out(a->len);
    for (size_t i = 0; i < a->len; ++i) {
        float x = a->data[i], y = b->data[i];
        switch (kind) {
            case MLXHIP_OP_ADD: r[i] = x + y; break;
            case MLXHIP_OP_MUL: r[i] = x * y; break;
            case MLXHIP_OP_SUB: r[i] = x - y; break;
            default: r[i] = x / y; break;
        }
    }
    *c->out = r;
    *c->out_len = a->len;
    return MLXHIP_OK;
}

static int unary(ctx_t* c, int kind) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    float* r = alloc_out(a->len);
    for (size_t i = 0; i < a->len; ++i) {
        float x = a->data[i];
        switch (kind) {
            case MLXHIP_OP_NEG: r[i] = -x; break;
            case MLXHIP_OP_EXP: r[i] = expf(x); break;
            case MLXHIP_OP_LOG: r[i] = logf(x); break;
            case MLXHIP_OP_SQRT: r[i] = sqrtf(x); break;
            case MLXHIP_OP_SILU: r[i] = x * sigmoid(x); break;
            case MLXHIP_OP_GELU: r[i] = gelu(x); break;
            default: r[i] = x; break; /* Reshape: data.to_vec() */
        }
    }
    *c->out = r;
    *c->out_len = a->len;
    return MLXHIP_OK;
}

/* reduce_sum / reduce_mean / reduce_max / reduce_along_axis (cpu_kernels.rs:130-195) */
static int reduce(ctx_t* c, int kind) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    if (!c->op->has_axis) {
        float v;
        if (kind == MLXHIP_OP_MAX) {
            v = -INFINITY;
            for (size_t i = 0; i < a->len; ++i) v = fmaxf(v, a->data[i]);
        } else {
            v = -0.0f;
            for (size_t i = 0; i < a->len; ++i) v += a->data[i];
            if (kind == MLXHIP_OP_MEAN) v = v / (float)a->len;
        }
        float* r = alloc_out(1);
        r[0] = v;
        *c->out = r;
        *c->out_len = 1;
        return MLXHIP_OK;
    }
    int ndim = (int)a->ndim;
    int axis = c->op->axis;
    int ax = axis < 0 ? ndim + axis : axis;
    if (ax < 0 || ax >= ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "axis %d out of range for ndim %d", axis, ndim);
    size_t outer = prod(a->shape, 0, (size_t)ax);
    size_t dim = (size_t)a->shape[ax];
    size_t inner = prod(a->shape, (size_t)ax + 1, a->ndim);
    float* r = alloc_out(outer * inner);
    float dimf = (float)a->shape[ax];
    for (size_t o = 0; o < outer; ++o) {
        for (size_t i = 0; i < inner; ++i) {
            float v = (kind == MLXHIP_OP_MAX) ? -INFINITY : -0.0f;
            for (size_t d = 0; d < dim; ++d) {
                float x = a->data[o * dim * inner + d * inner + i];
                if (kind == MLXHIP_OP_MAX) v = fmaxf(v, x);
                else v += x;
            }
            if (kind == MLXHIP_OP_MEAN) v = v / dimf;
            r[o * inner + i] = v;
        }
    }
    *c->out = r;
    *c->out_len = outer * inner;
    return MLXHIP_OK;
}

static int op_matmul(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t* a = &c->in[0];
    const mlxhip_input_t* b = &c->in[1];
    /* Rank 3 ([B,M,K] @ [B,K,N]): the batched form the reference specifies in
     * evals/tasks/003_matmul_batch_3d.json, computed as B independent rank-2
     * products with the loop of cpu_kernels.rs:216-228. */
    if (!((a->ndim == 2 && b->ndim == 2) || (a->ndim == 3 && b->ndim == 3)))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "matmul requires 2D tensors (or two 3D batched tensors)");
    size_t r = a->ndim - 2, batch = a->ndim == 3 ? (size_t)a->shape[0] : 1;
    if (a->ndim == 3 && (size_t)b->shape[0] != batch)
        return fail(MLXHIP_ERR_SHAPE_MISMATCH, "matmul: batch %zu vs %zu", batch, (size_t)b->shape[0]);
    size_t m = (size_t)a->shape[r], k = (size_t)a->shape[r + 1];
    size_t k2 = (size_t)b->shape[r], n = (size_t)b->shape[r + 1];
    if (k != k2) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "matmul: expected [%zu, %zu], got [%zu, %zu]", m, k, k2, n);
    float* out = alloc_out(batch * m * n);
    for (size_t i = 0; i < batch; ++i)
        oracle_matmul(a->data + i * m * k, b->data + i * k * n, out + i * m * n, m, k, n);
    *c->out = out;
    *c->out_len = batch * m * n;
    return MLXHIP_OK;
}

/* transpose (cpu_kernels.rs:232-274) */
static int op_transpose(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    size_t ndim = a->ndim;
    size_t perm[16];
    if (ndim > 16) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose: rank > 16");
    if (c->op->axes) {
        if (c->op->axes_len != ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose axes length must match ndim");
        for (size_t i = 0; i < ndim; ++i) perm[i] = (size_t)c->op->axes[i];
    } else {
        for (size_t i = 0; i < ndim; ++i) perm[i] = ndim - 1 - i;
    }
    size_t old_shape[16], new_shape[16], old_strides[16];
    for (size_t i = 0; i < ndim; ++i) old_shape[i] = (size_t)a->shape[i];
    for (size_t i = 0; i < ndim; ++i) {
        if (perm[i] >= ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose: axis out of range");
        new_shape[i] = old_shape[perm[i]];
    }
    for (size_t i = 0; i < ndim; ++i) old_strides[i] = 1;
    for (size_t i = ndim > 1 ? ndim - 1 : 0; i-- > 0;) old_strides[i] = old_strides[i + 1] * old_shape[i + 1];
    size_t total = a->len;
    float* r = alloc_out(total);
    for (size_t flat = 0; flat < total; ++flat) {
        size_t remaining = flat, old_flat = 0;
        for (size_t d = 0; d < ndim; ++d) {
            size_t sz = 1;
            for (size_t e = d + 1; e < ndim; ++e) sz *= new_shape[e];
            if (sz == 0) sz = 1; /* .product().max(1) */
            size_t coord = remaining / sz;
            remaining %= sz;
            old_flat += coord * old_strides[perm[d]];
        }
        r[flat] = a->data[old_flat];
    }
    *c->out = r;
    *c->out_len = total;
    return MLXHIP_OK;
}

static int op_softmax(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    int ndim = (int)a->ndim, axis = c->op->axis;
    int ax = axis < 0 ? ndim + axis : axis;
    if (ax < 0 || ax >= ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "axis %d out of range for ndim %d", axis, ndim);
    float* r = alloc_out(a->len);
    memcpy(r, a->data, a->len * sizeof(float));
    softmax_fibres(r, prod(a->shape, 0, (size_t)ax), (size_t)a->shape[ax], prod(a->shape, (size_t)ax + 1, a->ndim));
    *c->out = r;
    *c->out_len = a->len;
    return MLXHIP_OK;
}

/* embedding_lookup (cpu_kernels.rs:317-336) */
static int op_embedding(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t* w = &c->in[0];
    const mlxhip_input_t* idx = &c->in[1];
    if (w->ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Embedding weight must be 2D [num_embeddings, embedding_dim]");
    size_t ne = (size_t)w->shape[0], ed = (size_t)w->shape[1];
    size_t total = prod(c->meta->shape, 0, c->meta->ndim);
    float* r = alloc_out(total);
    memset(r, 0, total * sizeof(float));
    for (size_t i = 0; i < idx->len; ++i) {
        /* `idx_f as i32` saturates and maps NaN to 0 in Rust. */
        float f = idx->data[i];
        int32_t id;
        if (isnan(f)) id = 0;
        else if (f >= 2147483647.0f) id = 2147483647;
        else if (f <= -2147483648.0f) id = (int32_t)(-2147483647 - 1);
        else id = (int32_t)f;
        int32_t hi = (int32_t)ne - 1;
        int32_t row = id < 0 ? 0 : (id > hi ? hi : id);
        if (i * ed + ed > total) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "embedding: output too small");
        memcpy(r + i * ed, w->data + (size_t)row * ed, ed * sizeof(float));
    }
    *c->out = r;
    *c->out_len = total;
    return MLXHIP_OK;
}

static int op_norm(ctx_t* c, int rms) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    float* r = alloc_out(a->len);
    if (a->ndim == 0) {
        memcpy(r, a->data, a->len * sizeof(float));
    } else {
        size_t d = (size_t)a->shape[a->ndim - 1];
        size_t outer = d ? a->len / d : 0;
        if (rms) oracle_rms_norm(a->data, r, outer, d, c->op->eps);
        else oracle_layer_norm(a->data, r, outer, d, c->op->eps);
    }
    *c->out = r;
    *c->out_len = a->len;
    return MLXHIP_OK;
}

/* broadcast (cpu_kernels.rs:365-396) */
static int op_broadcast(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    size_t out_ndim = c->op->shape_len, in_ndim = a->ndim;
    if (in_ndim > out_ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "broadcast: rank grows only");
    size_t pad = out_ndim - in_ndim;
    size_t total = prod(c->op->shape, 0, out_ndim);
    float* r = alloc_out(total);
    for (size_t of = 0; of < total; ++of) {
        size_t remaining = of, in_flat = 0, in_stride = 1;
        for (size_t d = out_ndim; d-- > 0;) {
            size_t od = (size_t)c->op->shape[d];
            size_t coord = remaining % od;
            remaining /= od;
            if (d >= pad) {
                size_t idim = (size_t)a->shape[d - pad];
                size_t ic = idim == 1 ? 0 : coord;
                in_flat += ic * in_stride;
                in_stride *= idim;
            }
        }
        r[of] = a->data[in_flat];
    }
    *c->out = r;
    *c->out_len = total;
    return MLXHIP_OK;
}

static int same_shape(const mlxhip_input_t* x, const mlxhip_input_t* y) {
    if (x->ndim != y->ndim) return 0;
    for (size_t i = 0; i < x->ndim; ++i)
        if (x->shape[i] != y->shape[i]) return 0;
    return 1;
}

/* layer_norm_vjp (cpu_kernels.rs:403-454) and rms_norm_vjp (:462-510) */
static int op_norm_vjp(ctx_t* c, int rms) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t* dy = &c->in[0];
    const mlxhip_input_t* x = &c->in[1];
    if (!same_shape(dy, x) || dy->len != x->len) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "norm vjp: shape mismatch");
    float* r = alloc_out(x->len);
    *c->out = r;
    *c->out_len = x->len;
    if (x->ndim == 0) {
        memcpy(r, dy->data, dy->len * sizeof(float));
        return MLXHIP_OK;
    }
    size_t d = (size_t)x->shape[x->ndim - 1];
    if (d == 0 || x->len == 0) {
        memset(r, 0, x->len * sizeof(float));
        return MLXHIP_OK;
    }
    float df = (float)d;
    size_t outer = x->len / d;
    float* tmp = (float*)malloc(d * sizeof(float));
    float eps = c->op->eps;
    for (size_t o = 0; o < outer; ++o) {
        const float* xs = x->data + o * d;
        const float* gs = dy->data + o * d;
        if (!rms) {
            float acc = -0.0f;
            for (size_t i = 0; i < d; ++i) acc += xs[i];
            float mean = acc / df;
            float vacc = -0.0f;
            for (size_t i = 0; i < d; ++i) vacc += (xs[i] - mean) * (xs[i] - mean);
            float var = vacc / df;
            float sd = sqrtf(var + eps);
            float inv_std = 1.0f / sd;
            for (size_t i = 0; i < d; ++i) tmp[i] = (xs[i] - mean) * inv_std;
            float sdy = -0.0f;
            for (size_t i = 0; i < d; ++i) sdy += gs[i];
            float mean_dy = sdy / df;
            float sdx = -0.0f;
            for (size_t i = 0; i < d; ++i) sdx += gs[i] * tmp[i];
            float mean_dy_xhat = sdx / df;
            for (size_t i = 0; i < d; ++i) r[o * d + i] = inv_std * (gs[i] - mean_dy - tmp[i] * mean_dy_xhat);
        } else {
            float acc = -0.0f;
            for (size_t i = 0; i < d; ++i) acc += xs[i] * xs[i];
            float rmsv = sqrtf(acc / df + eps);
            float inv_rms = 1.0f / rmsv;
            for (size_t i = 0; i < d; ++i) tmp[i] = xs[i] * inv_rms;
            float sdy = -0.0f;
            for (size_t i = 0; i < d; ++i) sdy += gs[i] * tmp[i];
            float mean_dy_y = sdy / df;
            for (size_t i = 0; i < d; ++i) r[o * d + i] = inv_rms * (gs[i] - tmp[i] * mean_dy_y);
        }
    }
    free(tmp);
    return MLXHIP_OK;
}

/* softmax_vjp (cpu_kernels.rs:515-553) */
static int op_softmax_vjp(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t* dy = &c->in[0];
    const mlxhip_input_t* s = &c->in[1];
    if (dy->len != s->len) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "softmax vjp: length mismatch");
    int ndim = (int)s->ndim, axis = c->op->axis;
    int ax = axis < 0 ? ndim + axis : axis;
    if (ax < 0 || ax >= ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "axis %d out of range for ndim %d", axis, ndim);
    size_t outer = prod(s->shape, 0, (size_t)ax), dim = (size_t)s->shape[ax];
    size_t inner = prod(s->shape, (size_t)ax + 1, s->ndim);
    float* r = alloc_out(s->len);
    memset(r, 0, s->len * sizeof(float));
    for (size_t o = 0; o < outer; ++o) {
        for (size_t i = 0; i < inner; ++i) {
            float dot = 0.0f;
            for (size_t d = 0; d < dim; ++d) {
                size_t idx = o * dim * inner + d * inner + i;
                dot += dy->data[idx] * s->data[idx];
            }
            for (size_t d = 0; d < dim; ++d) {
                size_t idx = o * dim * inner + d * inner + i;
                r[idx] = s->data[idx] * (dy->data[idx] - dot);
            }
        }
    }
    *c->out = r;
    *c->out_len = s->len;
    return MLXHIP_OK;
}

/* silu_vjp (cpu_kernels.rs:558-576) and gelu_vjp (:582-606) */
static int op_act_vjp(ctx_t* c, int gelu_kind) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t* dy = &c->in[0];
    const mlxhip_input_t* x = &c->in[1];
    if (dy->len != x->len) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "activation vjp: length mismatch");
    float* r = alloc_out(x->len);
    const float a = sqrtf(2.0f / (float)3.14159265358979323846);
    const float b = 0.044715f;
    for (size_t i = 0; i < x->len; ++i) {
        float g = dy->data[i], xi = x->data[i];
        if (!gelu_kind) {
            float sig = sigmoid(xi);
            r[i] = g * sig * (1.0f + xi * (1.0f - sig));
        } else {
            float inner = a * (xi + b * xi * xi * xi);
            float t = tanhf(inner);
            float sech2 = 1.0f - t * t;
            float dg = 0.5f * (1.0f + t) + 0.5f * xi * sech2 * a * (1.0f + 3.0f * b * xi * xi);
            r[i] = g * dg;
        }
    }
    *c->out = r;
    *c->out_len = x->len;
    return MLXHIP_OK;
}

/* cpu_rope (cpu_kernels.rs:608-645), OpKind::Rope */
static int op_rope(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* x = &c->in[0];
    if (c->meta->ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Rope input must be 2-D [tokens, head_dim]");
    size_t tokens = (size_t)c->meta->shape[0], hd = (size_t)c->meta->shape[1];
    size_t rd = (size_t)c->op->rotary_dim;
    if (rd > hd || (rd % 2) != 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "rotary_dim must be even and <= head_dim");
    if (x->len < tokens * hd) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Rope: input shorter than meta");
    float* r = alloc_out(x->len);
    memcpy(r, x->data, x->len * sizeof(float));
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t i = 0; i < rd / 2; ++i) {
            float inv_freq = powf(c->op->theta, -2.0f * (float)i / (float)rd);
            float angle = (float)(c->op->pos_offset + t) * inv_freq;
            float s = sinf(angle), co = cosf(angle);
            size_t base = t * hd + i * 2;
            float x0 = x->data[base], x1 = x->data[base + 1];
            r[base] = x0 * co - x1 * s;
            r[base + 1] = x0 * s + x1 * co;
        }
    }
    *c->out = r;
    *c->out_len = x->len;
    return MLXHIP_OK;
}

/* rope (cpu_kernels.rs:896-956), OpKind::RoPE */
static int op_rope_mlx(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    if (a->ndim < 1) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "RoPE requires at least 1 dimension");
    size_t hd = (size_t)a->shape[a->ndim - 1];
    if (hd % 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "RoPE head_dim must be even, got %zu", hd);
    size_t half = hd / 2, total = a->len, nh = hd ? total / hd : 0;
    float* r = alloc_out(total);
    memset(r, 0, total * sizeof(float));
    for (size_t i = 0; i < nh; ++i) {
        float pos = (float)(c->op->offset + i);
        for (size_t d = 0; d < half; ++d) {
            float th = pos * powf(c->op->base, -(2.0f * (float)d / (float)hd));
            float ct = cosf(th), st = sinf(th);
            size_t i0, i1;
            if (c->op->traditional) { i0 = i * hd + 2 * d; i1 = i0 + 1; }
            else { i0 = i * hd + d; i1 = i * hd + d + half; }
            float x0 = a->data[i0], x1 = a->data[i1];
            r[i0] = x0 * ct - x1 * st;
            r[i1] = x0 * st + x1 * ct;
        }
    }
    *c->out = r;
    *c->out_len = total;
    return MLXHIP_OK;
}

/* scaled_masked_softmax (cpu_kernels.rs:671-712) on a [tq, tk] row-major buffer in place. */
static void scaled_masked_rows(const float* src, float* data, size_t tq, size_t tk, float scale, int causal) {
    for (size_t i = 0; i < tq; ++i) {
        for (size_t j = 0; j < tk; ++j) {
            size_t idx = i * tk + j;
            float v = src[idx] * scale;
            if (causal && j > i) v = -1e9f;
            data[idx] = v;
        }
        float* row = data + i * tk;
        float mx = -INFINITY;
        for (size_t j = 0; j < tk; ++j)
            if (row[j] > mx) mx = row[j];
        float se = 0.0f;
        for (size_t j = 0; j < tk; ++j) {
            row[j] = expf(row[j] - mx);
            se += row[j];
        }
        for (size_t j = 0; j < tk; ++j) row[j] /= se;
    }
}

static int op_scaled_masked_softmax(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    if (a->ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ScaledMaskedSoftmax requires 2D input [Tq, Tk]");
    size_t tq = (size_t)a->shape[0], tk = (size_t)a->shape[1];
    float* r = alloc_out(tq * tk);
    scaled_masked_rows(a->data, r, tq, tk, c->op->scale, c->op->causal);
    *c->out = r;
    *c->out_len = tq * tk;
    return MLXHIP_OK;
}

/* cpu_attention (cpu_kernels.rs:738-812) */
static int op_attention(ctx_t* c) {
    if (c->n_inputs != 3) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Attention requires exactly 3 inputs [Q, K, V]");
    const mlxhip_input_t *q = &c->in[0], *k = &c->in[1], *v = &c->in[2];
    if (q->ndim != 2 || k->ndim != 2 || v->ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Attention inputs must be 2D");
    size_t tq = (size_t)q->shape[0], dh = (size_t)q->shape[1];
    size_t tk = (size_t)k->shape[0], dhk = (size_t)k->shape[1];
    size_t tkv = (size_t)v->shape[0], dhv = (size_t)v->shape[1];
    if (dh != dhk) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "attention: q/k head dim");
    if (tk != tkv || dh != dhv) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "attention: k/v shape");
    float* kt = alloc_out(tk * dh);
    for (size_t r = 0; r < tk; ++r)
        for (size_t cc = 0; cc < dh; ++cc) kt[cc * tk + r] = k->data[r * dh + cc];
    float* scores = alloc_out(tq * tk);
    oracle_matmul(q->data, kt, scores, tq, dh, tk);
    float* probs = alloc_out(tq * tk);
    scaled_masked_rows(scores, probs, tq, tk, c->op->scale, c->op->causal);
    float* y = alloc_out(tq * dh);
    oracle_matmul(probs, v->data, y, tq, tk, dh);
    free(kt);
    free(scores);
    free(probs);
    *c->out = y;
    *c->out_len = tq * dh;
    return MLXHIP_OK;
}

/* narrow (cpu_kernels.rs:814-845) */
static int op_narrow(ctx_t* c) {
    size_t n_inputs = c->n_inputs;
    REQUIRE(0);
    const mlxhip_input_t* a = &c->in[0];
    int ndim = (int)a->ndim, axis = c->op->axis;
    int ax = axis < 0 ? ndim + axis : axis;
    if (ax < 0 || ax >= ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "narrow: axis %d out of range for ndim %d", axis, ndim);
    int64_t ds = a->shape[ax], start = c->op->start, length = c->op->length;
    if (start < 0 || start + length > ds) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "narrow: start %lld + length %lld exceeds dim size %lld", (long long)start, (long long)length, (long long)ds);
    size_t outer = prod(a->shape, 0, (size_t)ax), dim = (size_t)ds, inner = prod(a->shape, (size_t)ax + 1, a->ndim);
    size_t n = outer * (size_t)length * inner;
    float* r = alloc_out(n);
    size_t w = 0;
    for (size_t o = 0; o < outer; ++o)
        for (size_t d = (size_t)start; d < (size_t)(start + length); ++d) {
            memcpy(r + w, a->data + (o * dim + d) * inner, inner * sizeof(float));
            w += inner;
        }
    *c->out = r;
    *c->out_len = n;
    return MLXHIP_OK;
}

/* concatenate (cpu_kernels.rs:847-894) */
static int op_concatenate(ctx_t* c) {
    if (c->n_inputs == 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Concatenate requires at least one input");
    const mlxhip_input_t* f = &c->in[0];
    int ndim = (int)f->ndim, axis = c->op->axis;
    int ax = axis < 0 ? ndim + axis : axis;
    if (ax < 0 || ax >= ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "concatenate: axis %d out of range for ndim %d", axis, ndim);
    for (size_t i = 1; i < c->n_inputs; ++i) {
        const mlxhip_input_t* p = &c->in[i];
        if (p->ndim != f->ndim) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Concatenate: all inputs must have same ndim");
        for (size_t d = 0; d < f->ndim; ++d)
            if ((int)d != ax && f->shape[d] != p->shape[d]) return fail(MLXHIP_ERR_SHAPE_MISMATCH, "concatenate: shape mismatch");
    }
    size_t outer = prod(f->shape, 0, (size_t)ax), inner = prod(f->shape, (size_t)ax + 1, f->ndim);
    size_t total_dim = 0;
    for (size_t i = 0; i < c->n_inputs; ++i) total_dim += (size_t)c->in[i].shape[ax];
    size_t n = outer * total_dim * inner;
    float* r = alloc_out(n);
    size_t w = 0;
    for (size_t o = 0; o < outer; ++o)
        for (size_t i = 0; i < c->n_inputs; ++i) {
            size_t dim = (size_t)c->in[i].shape[ax];
            memcpy(r + w, c->in[i].data + o * dim * inner, dim * inner * sizeof(float));
            w += dim * inner;
        }
    *c->out = r;
    *c->out_len = n;
    return MLXHIP_OK;
}

/* CpuRefBackend::eval_node (cpu_kernels.rs:13-102) */
int oracle_eval_node(const mlxhip_op_t* op, const mlxhip_input_t* inputs, size_t n_inputs,
                     const mlxhip_meta_t* out_meta, float** out, size_t* out_len) {
    if (!op || !out_meta || !out || !out_len || (n_inputs && !inputs)) return fail(MLXHIP_ERR_NULL_PTR, "null argument");
    *out = NULL;
    *out_len = 0;
    ctx_t c = {op, inputs, n_inputs, out_meta, out, out_len};
    switch (op->kind) {
        case MLXHIP_OP_CONSTANT:
        case MLXHIP_OP_PARAMETER:
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Constant/Parameter nodes should be pre-materialized");
        case MLXHIP_OP_ADD:
        case MLXHIP_OP_MUL:
        case MLXHIP_OP_SUB:
        case MLXHIP_OP_DIV: return binary(&c, op->kind);
        case MLXHIP_OP_NEG:
        case MLXHIP_OP_EXP:
        case MLXHIP_OP_LOG:
        case MLXHIP_OP_SQRT:
        case MLXHIP_OP_SILU:
        case MLXHIP_OP_GELU:
        case MLXHIP_OP_RESHAPE: return unary(&c, op->kind);
        case MLXHIP_OP_SUM:
        case MLXHIP_OP_MEAN:
        case MLXHIP_OP_MAX: return reduce(&c, op->kind);
        case MLXHIP_OP_MATMUL: return op_matmul(&c);
        case MLXHIP_OP_EMBEDDING: return op_embedding(&c);
        case MLXHIP_OP_TRANSPOSE: return op_transpose(&c);
        case MLXHIP_OP_SOFTMAX: return op_softmax(&c);
        case MLXHIP_OP_LAYER_NORM: return op_norm(&c, 0);
        case MLXHIP_OP_RMS_NORM: return op_norm(&c, 1);
        case MLXHIP_OP_BROADCAST: return op_broadcast(&c);
        case MLXHIP_OP_SCALED_MASKED_SOFTMAX: return op_scaled_masked_softmax(&c);
        case MLXHIP_OP_ATTENTION: return op_attention(&c);
        case MLXHIP_OP_ROPE: return op_rope(&c);
        case MLXHIP_OP_LAYER_NORM_VJP: return op_norm_vjp(&c, 0);
        case MLXHIP_OP_RMS_NORM_VJP: return op_norm_vjp(&c, 1);
        case MLXHIP_OP_SOFTMAX_VJP: return op_softmax_vjp(&c);
        case MLXHIP_OP_SILU_VJP: return op_act_vjp(&c, 0);
        case MLXHIP_OP_GELU_VJP: return op_act_vjp(&c, 1);
        case MLXHIP_OP_ROPE_MLX: return op_rope_mlx(&c);
        case MLXHIP_OP_NARROW: return op_narrow(&c);
        case MLXHIP_OP_CONCATENATE: return op_concatenate(&c);
        default: return fail(MLXHIP_ERR_INVALID_ARGUMENT, "unknown op kind %d", op->kind);
    }
}
