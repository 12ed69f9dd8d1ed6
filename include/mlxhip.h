/*
 * mlxhip.h — C ABI of mlx-hip, an MI355X (gfx950) compute backend for the
 * oxidizedMLX tensor runtime.
 *
 * ABI version: 1
 *
 * Conventions follow the reference's own C ABI (crates/mlx-sys/csrc/mlxrs.h:1-12):
 *   - opaque handles, created and freed exactly once; free(NULL) is a no-op;
 *   - functions returning a handle return NULL on failure;
 *   - functions returning int return MLXHIP_OK (0) on success, otherwise one
 *     of mlxhip_status_t, which maps 1:1 onto the reference's MlxError
 *     variants (crates/mlx-core/src/lib.rs:31-50);
 *   - the message of the last failure on the calling thread is available
 *     from mlxhip_last_error().
 * Every entry point is thread-safe. Pointers named "device" are HIP device
 * addresses (from mlxhip_buffer_ptr or any other HIP allocation on the same
 * device); everything else is host memory. No torch or HIP types appear in
 * any signature: streams are passed as `void*` holding a hipStream_t
 * (NULL = the device's null stream).
 */
#ifndef MLXHIP_H
#define MLXHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLXHIP_ABI_VERSION 1

/* ── Status codes (MlxError, crates/mlx-core/src/lib.rs:31-50) ───────────── */
typedef enum {
    MLXHIP_OK = 0,
    MLXHIP_ERR_NULL_PTR = 1,            /* MlxError::NullPtr */
    MLXHIP_ERR_FFI_FAILED = 2,          /* MlxError::FfiFailed (HIP runtime error) */
    MLXHIP_ERR_SHAPE_MISMATCH = 3,      /* MlxError::ShapeMismatch */
    MLXHIP_ERR_INVALID_ARGUMENT = 4,    /* MlxError::InvalidArgument */
    MLXHIP_ERR_BACKEND_UNAVAILABLE = 5, /* MlxError::BackendUnavailable (no GPU) */
    MLXHIP_ERR_IO = 6                   /* MlxError::IoError */
} mlxhip_status_t;

/* ── Element types (DType, crates/mlx-core/src/types.rs:4-11; same codes as
 *    mlx_dtype_t in crates/mlx-sys/csrc/mlxrs.h:40-46) ───────────────────── */
typedef enum {
    MLXHIP_DTYPE_F32 = 0,
    MLXHIP_DTYPE_F16 = 1,
    MLXHIP_DTYPE_BF16 = 2,
    MLXHIP_DTYPE_I32 = 3,
    MLXHIP_DTYPE_I64 = 4
} mlxhip_dtype_t;

/* ── Op kinds: OpKind (crates/mlx-core/src/graph.rs:33-168), same order ──── */
typedef enum {
    MLXHIP_OP_CONSTANT = 0,
    MLXHIP_OP_PARAMETER = 1,
    MLXHIP_OP_ADD = 2,
    MLXHIP_OP_SUB = 3,
    MLXHIP_OP_MUL = 4,
    MLXHIP_OP_DIV = 5,
    MLXHIP_OP_NEG = 6,
    MLXHIP_OP_EXP = 7,
    MLXHIP_OP_LOG = 8,
    MLXHIP_OP_SUM = 9,                    /* axis, has_axis */
    MLXHIP_OP_MEAN = 10,                  /* axis, has_axis */
    MLXHIP_OP_MAX = 11,                   /* axis, has_axis */
    MLXHIP_OP_MATMUL = 12,
    MLXHIP_OP_RESHAPE = 13,               /* shape = new_shape */
    MLXHIP_OP_TRANSPOSE = 14,             /* axes (NULL = reverse) */
    MLXHIP_OP_SOFTMAX = 15,               /* axis */
    MLXHIP_OP_SILU = 16,
    MLXHIP_OP_GELU = 17,
    MLXHIP_OP_LAYER_NORM = 18,            /* eps */
    MLXHIP_OP_RMS_NORM = 19,              /* eps */
    MLXHIP_OP_ROPE = 20,                  /* rotary_dim, pos_offset, theta */
    MLXHIP_OP_BROADCAST = 21,             /* shape = target_shape */
    MLXHIP_OP_EMBEDDING = 22,
    MLXHIP_OP_SCALED_MASKED_SOFTMAX = 23, /* scale, causal */
    MLXHIP_OP_ATTENTION = 24,             /* scale, causal */
    MLXHIP_OP_LAYER_NORM_VJP = 25,        /* eps */
    MLXHIP_OP_RMS_NORM_VJP = 26,          /* eps */
    MLXHIP_OP_SOFTMAX_VJP = 27,           /* axis */
    MLXHIP_OP_SILU_VJP = 28,
    MLXHIP_OP_GELU_VJP = 29,
    MLXHIP_OP_SQRT = 30,
    MLXHIP_OP_ROPE_MLX = 31,              /* OpKind::RoPE: base, offset, traditional */
    MLXHIP_OP_NARROW = 32,                /* axis, start, length */
    MLXHIP_OP_CONCATENATE = 33,           /* axis */
    /* No reference counterpart (extensions for training through fused
     * attention; the reference's Attention is 2-D and has no VJP,
     * crates/mlx-autograd/src/vjp.rs:173-176):
     * HeadAttention: inputs Q, K, V [heads, t, dh], output [heads, t, dh]:
     * per head the Attention op's arithmetic (cpu_attention,
     * crates/mlx-core/src/cpu_kernels.rs:738-812) through mlxhip_attention.
     * With has_axis, axis = H: inputs and output [groups, t, H*dh], H heads
     * side by side in each row (a [batch*t, d_model] projection viewed as
     * [batch, t, d_model]); head h of group b is columns h*dh .. h*dh+dh-1.
     * Differentiable: its VJP is one HeadAttentionVjp node.
     * HeadAttentionVjp: inputs Q, K, V, O (the forward output), dO, the same
     * axis; output [3, <input shape>] = dQ, dK, dV (mlxhip_attention_vjp). */
    MLXHIP_OP_HEAD_ATTENTION = 34,        /* scale, causal, axis (heads per row, if has_axis) */
    MLXHIP_OP_HEAD_ATTENTION_VJP = 35,    /* scale, causal, axis (heads per row, if has_axis) */
    MLXHIP_OP_COUNT_ = 36
} mlxhip_op_kind_t;

/* One OpKind value with its parameters. Fields an op does not use are
 * ignored. Mirrors the enum payloads of graph.rs:33-168. */
typedef struct {
    int32_t kind;           /* mlxhip_op_kind_t */
    int32_t axis;           /* Sum/Mean/Max (if has_axis), Softmax, SoftmaxVjp, Narrow, Concatenate */
    int32_t has_axis;       /* Sum/Mean/Max: 0 means `axis: None` */
    int32_t causal;         /* ScaledMaskedSoftmax, Attention (0/1) */
    float eps;              /* LayerNorm, RmsNorm and their VJPs */
    float scale;            /* ScaledMaskedSoftmax, Attention */
    float theta;            /* Rope */
    float base;             /* RoPE */
    const int64_t* shape;   /* Reshape new_shape, Broadcast target_shape */
    size_t shape_len;
    const int64_t* axes;    /* Transpose permutation; NULL means `axes: None` */
    size_t axes_len;
    int64_t start;          /* Narrow */
    int64_t length;         /* Narrow */
    uint64_t rotary_dim;    /* Rope */
    uint64_t pos_offset;    /* Rope */
    uint64_t offset;        /* RoPE */
    int32_t traditional;    /* RoPE */
    int32_t reserved_;
} mlxhip_op_t;

/* NodeInput (crates/mlx-core/src/backend.rs:16-20): row-major contiguous f32
 * data of `len` elements with its logical shape and dtype. */
typedef struct {
    const float* data;
    size_t len;
    const int64_t* shape;
    size_t ndim;
    int32_t dtype;          /* mlxhip_dtype_t (logical tag; data is always f32) */
} mlxhip_input_t;

/* TensorMeta (crates/mlx-core/src/graph.rs:18-21). */
typedef struct {
    const int64_t* shape;
    size_t ndim;
    int32_t dtype;          /* mlxhip_dtype_t */
} mlxhip_meta_t;

/* ── Library, device and error state ─────────────────────────────────────── */

/* Returns MLXHIP_ABI_VERSION of the loaded library. */
int mlxhip_abi_version(void);

/* Message of the last failure on this thread ("" if none). The pointer stays
 * valid until the next failing call on the same thread. */
const char* mlxhip_last_error(void);

/* Status code (mlxhip_status_t) of the last failure on this thread; lets
 * callers of the handle/id-returning functions recover the MlxError variant. */
int mlxhip_last_status(void);

/* The payload of MlxError::ShapeMismatch{expected, got}
 * (crates/mlx-core/src/lib.rs:40-41) for the last failure on this thread,
 * when that failure was MLXHIP_ERR_SHAPE_MISMATCH: copies up to `cap` dims of
 * each shape into `expected` / `got` (either may be NULL) and stores their
 * full lengths in *expected_ndim / *got_ndim. Returns MLXHIP_OK, or
 * MLXHIP_ERR_INVALID_ARGUMENT (without recording a new error) when the last
 * failure was not a shape mismatch. The shapes are the reference's for the
 * same failure: e.g. matmul K mismatch expected [M, K], got [K2, N]
 * (cpu_kernels.rs:212-217); binary ops expected = lhs shape, got = rhs shape
 * (:117-121); VJPs expected = the forward input's shape, got = dy's. */
int mlxhip_last_shape_mismatch(int64_t* expected, size_t* expected_ndim,
                               int64_t* got, size_t* got_ndim, size_t cap);

/* Allocation-failure hook for error-path tests (no counterpart in the
 * reference, whose tests force failures through bad shapes and parameters
 * only: crates/mlx-core/tests/attention_golden.rs:259-302). After `after`
 * more successful device allocations, every device allocation the library
 * makes (stream buffers and scratch, GEMM workspaces, mlxhip_buffer_alloc,
 * decoders) fails with MLXHIP_ERR_FFI_FAILED until the hook is reset with
 * after < 0. Cached blocks count as allocations. The environment variable
 * MLXHIP_FAIL_ALLOC_AFTER=n sets it at the first allocation. Returns MLXHIP_OK. */
int mlxhip_debug_fail_allocations(int64_t after);

/* Number of visible HIP devices (0 when no GPU; never fails). */
int mlxhip_device_count(void);

/* Selects the device used by later calls on this thread and initialises it
 * (replaces Metal context creation, crates/mlx-metal/src/context.rs:25).
 * Returns MLXHIP_ERR_BACKEND_UNAVAILABLE when no GPU is present. */
int mlxhip_init(int device);

/* Blocks until all work on `stream` (NULL = every stream of the device) ends. */
int mlxhip_synchronize(void* stream);

/* ── Backend::eval_node, host-vector contract ────────────────────────────── */

/* Backend::eval_node (crates/mlx-core/src/backend.rs:27-35): evaluates one
 * op on materialised host inputs and writes numel(out_meta) f32 values to
 * out_host. `out_len` must equal that count (else MLXHIP_ERR_SHAPE_MISMATCH).
 * Constant/Parameter return MLXHIP_ERR_INVALID_ARGUMENT as in
 * crates/mlx-core/src/cpu_kernels.rs:21-23; ops without a HIP kernel return
 * MLXHIP_ERR_INVALID_ARGUMENT ("unsupported op") as in
 * crates/mlx-metal/src/backend.rs:511-514. Inputs are copied to HBM, the
 * kernel runs there, and the result is copied back before returning. */
int mlxhip_eval_node(const mlxhip_op_t* op,
                     const mlxhip_input_t* inputs, size_t n_inputs,
                     const mlxhip_meta_t* out_meta,
                     float* out_host, size_t out_len);

/* ── Device-resident buffers (the "Unified Buffer" the reference planned,
 *    docs/ARCHITECTURE_TDD.md:89-99; replaces UnifiedBuffer,
 *    crates/mlx-metal/src/unified.rs:136-239) ────────────────────────────── */

typedef struct mlxhip_buffer_t mlxhip_buffer_t;

/* Allocates `bytes` of HBM on the current device. bytes == 0 yields a valid
 * empty buffer (crates/mlx-metal/src/unified.rs:318-324). */
mlxhip_buffer_t* mlxhip_buffer_alloc(size_t bytes);
void mlxhip_buffer_free(mlxhip_buffer_t* buf);
void* mlxhip_buffer_ptr(const mlxhip_buffer_t* buf);    /* device address */
size_t mlxhip_buffer_size(const mlxhip_buffer_t* buf);  /* bytes */
/* Synchronous host <-> device copies of `bytes` at byte `offset`. */
int mlxhip_buffer_upload(mlxhip_buffer_t* buf, size_t offset, const void* host, size_t bytes);
int mlxhip_buffer_download(const mlxhip_buffer_t* buf, size_t offset, void* host, size_t bytes);

/* Backend::eval_node with device-resident operands: as mlxhip_eval_node but
 * every input's `data` is a device address and the result is written to the
 * device address `out` (numel(out_meta) f32 values). Runs on `stream`,
 * asynchronously; no host copies. */
int mlxhip_eval_node_dev(const mlxhip_op_t* op,
                         const mlxhip_input_t* inputs, size_t n_inputs,
                         const mlxhip_meta_t* out_meta,
                         float* out, void* stream);

/* ── Stream: lazy graph + scheduler with HBM-resident buffers ────────────────
 * Restates Stream (crates/mlx-core/src/backend.rs:37-185) and Graph
 * (crates/mlx-core/src/graph.rs:170-305) with this backend bound: CSE of
 * non-source ops, memoisation, eval_count/cache_len, and buffers that stay in
 * HBM until the stream is freed. Only get_buffer copies to the host. */

typedef struct mlxhip_stream_t mlxhip_stream_t;

mlxhip_stream_t* mlxhip_stream_new(void);
void mlxhip_stream_free(mlxhip_stream_t* s);
/* Stream::add_constant (backend.rs:59-71). Returns the node id (never 0), or
 * 0 on failure. */
uint64_t mlxhip_stream_add_constant(mlxhip_stream_t* s, const float* data, size_t len,
                                    const mlxhip_meta_t* meta);
/* Stream::add_op (backend.rs:74-82). Returns the node id, or 0 on failure. */
uint64_t mlxhip_stream_add_op(mlxhip_stream_t* s, const mlxhip_op_t* op,
                              const uint64_t* inputs, size_t n_inputs,
                              const mlxhip_meta_t* meta);
/* Stream::eval (backend.rs:85-159). */
int mlxhip_stream_eval(mlxhip_stream_t* s, uint64_t node);
/* Stream::get_buffer (backend.rs:162-164): copies the node's f32 data to
 * `out` (len must equal its numel). MLXHIP_ERR_INVALID_ARGUMENT if the node
 * is not materialised. */
int mlxhip_stream_get_buffer(mlxhip_stream_t* s, uint64_t node, float* out, size_t len);
/* Stream::eval_count (backend.rs:177-179): number of backend node
 * evaluations (a fused group counts each node it covers). */
uint64_t mlxhip_stream_eval_count(const mlxhip_stream_t* s);
/* Stream::cache_len (backend.rs:182-184). */
size_t mlxhip_stream_cache_len(const mlxhip_stream_t* s);
/* Number of kernel launches issued by eval so far (fusion makes this smaller
 * than eval_count). No reference counterpart; telemetry in the spirit of
 * BufferTelemetry, crates/mlx-metal/src/instrument.rs:2-29. */
uint64_t mlxhip_stream_launch_count(const mlxhip_stream_t* s);
/* Enables (1, default) or disables (0) look-ahead fusion of single-consumer
 * elementwise chains and of Transpose into MatMul operand layouts. */
int mlxhip_stream_set_fusion(mlxhip_stream_t* s, int enabled);
/* Asynchronous evaluation (0 = off, the default): eval and eval_many return
 * once the stream's kernels are enqueued instead of after they finish, so
 * the caller can build its next graph while the GPU works. Results are the
 * same bit for bit. get_buffer, mlxhip_stream_synchronize and stream_free
 * wait for the work; an error a kernel meets after its launch is reported
 * there. No reference counterpart: the reference's Stream::eval returns
 * computed values (backend.rs:85-159); a caller that only reads results
 * through get_buffer sees the same values. Turning it off synchronizes. */
int mlxhip_stream_set_async(mlxhip_stream_t* s, int enabled);
/* Waits for every kernel of the stream (see mlxhip_stream_set_async). */
int mlxhip_stream_synchronize(mlxhip_stream_t* s);
/* Forgets every node of the stream, as if it were new (node ids are not
 * reused; using an old one is MLXHIP_ERR_INVALID_ARGUMENT). Their HBM
 * returns to the library: with asynchronous evaluation the stream's later
 * work may reuse it at once, in queue order, without waiting for the
 * kernels already queued; caller memory that view constants read
 * (mlxhip_stream_add_constant_view) may still be read by those kernels until
 * the stream is next synchronized. No reference counterpart (a reference Stream keeps
 * every node until it is dropped, backend.rs:37-185); for a loop that builds
 * a new graph every step on one stream. */
int mlxhip_stream_clear(mlxhip_stream_t* s);
/* Stream::eval over several outputs at once (Graph::topo_sort takes a slice
 * of outputs, crates/mlx-core/src/graph.rs:268-294): one topological order
 * and one fusion plan for all of them, one synchronisation at the end. Every
 * requested node is materialised. */
int mlxhip_stream_eval_many(mlxhip_stream_t* s, const uint64_t* nodes, size_t n);
/* As mlxhip_stream_add_constant with `data` a device address: the values are
 * copied device-to-device on the stream's queue, so `data` must stay
 * unchanged until the next mlxhip_stream_eval* call on `s` returns (with
 * asynchronous evaluation: until the stream is next synchronized). No
 * reference counterpart (the reference's constants always come from host
 * vectors, backend.rs:59-71); for callers whose inputs already live in HBM. */
uint64_t mlxhip_stream_add_constant_dev(mlxhip_stream_t* s, const float* data, size_t len,
                                        const mlxhip_meta_t* meta);
/* As mlxhip_stream_add_constant_dev without the copy: the node reads `data`
 * (256-byte-aligned device memory of the caller) in place; the stream never
 * writes or frees it. `data` must stay valid and unchanged for as long as a
 * queued kernel may read it: while the node exists and, with asynchronous
 * evaluation, until the stream is next synchronized (mlxhip_stream_synchronize,
 * mlxhip_stream_get_buffer, turning asynchronous evaluation off, or freeing
 * the stream), even after mlxhip_stream_clear, which does not wait for
 * queued kernels. With synchronous evaluation, clearing or freeing the
 * stream ends it. No reference counterpart; for inputs that already live in
 * HBM, such as a model's weights read by every step. */
uint64_t mlxhip_stream_add_constant_view(mlxhip_stream_t* s, const float* data, size_t len,
                                         const mlxhip_meta_t* meta);
/* value_and_grad / backward (crates/mlx-autograd/src/lib.rs:30-107) with the
 * VJP table of crates/mlx-autograd/src/vjp.rs:8-178: `loss` must have one
 * element (else MLXHIP_ERR_INVALID_ARGUMENT "grad requires scalar loss"); it
 * is evaluated, seeded with ones, and VJP nodes are added to the graph in
 * reverse topological order. grads[i] receives the node id of
 * d(loss)/d(wrt[i]), unevaluated (evaluate with mlxhip_stream_eval_many).
 * Several wrt nodes per call (the reference takes one, lib.rs:104-106);
 * "gradient not found" (MLXHIP_ERR_INVALID_ARGUMENT) when a wrt node does
 * not affect the loss; "VJP not implemented" for ops without a VJP on the
 * path. Rank-3 MatMul differentiates with Transpose [0,2,1]. */
int mlxhip_stream_grad(mlxhip_stream_t* s, uint64_t loss, const uint64_t* wrt, size_t n_wrt,
                       uint64_t* grads);

/* ── Direct kernel entry points (device pointers, asynchronous on `stream`) ─ */

/* Batched GEMM, row-major: for each b < batch,
 *   C_b[M,N] = op(A_b) · op(B_b), f32 accumulate,
 * op(A) = A [M,K] (trans_a = 0, row pitch lda) or A^T with A stored [K,M]
 * (trans_a = 1); op(B) = B [K,N] (trans_b = 0, row pitch ldb) or B^T with B
 * stored [N,K] (trans_b = 1). A_b = a + b*stride_a elements (likewise B, C).
 * ab_dtype: F32, BF16 or F16 (16-bit MFMA); both operands share it. F32
 * products with m, n, k >= 256 and m*n*k*batch >= 2^31 run as six bf16
 * products of an exact three-plane split of each operand (f32 accuracy;
 * inf/NaN inputs take an exact f32 path), smaller ones on the f32 MFMA.
 * c_dtype: F32, or BF16/F16 (round-to-nearest-even of the f32 accumulator).
 * Replaces matmul (crates/mlx-core/src/cpu_kernels.rs:197-230) and the Metal
 * tiled_gemm_f32 (crates/mlx-metal/src/kernels/gemm.metal:32-77), adding the
 * batched and transposed-operand forms that autograd's MatMul VJP
 * (crates/mlx-autograd/src/vjp.rs:71-80) and Linear (crates/mlx-nn/src/linear.rs:34-43)
 * express through Transpose nodes. */
int mlxhip_gemm(int32_t ab_dtype, int32_t c_dtype, int32_t trans_a, int32_t trans_b,
                int64_t m, int64_t n, int64_t k, int64_t batch,
                const void* a, int64_t lda, int64_t stride_a,
                const void* b, int64_t ldb, int64_t stride_b,
                void* c, int64_t ldc, int64_t stride_c,
                void* stream);

/* mlxhip_gemm for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same arguments, kernels, split-K plan and
 * results (bit for bit) as mlxhip_gemm, except as noted below, but its workspace (split-K partials,
 * zero-padded copies of unaligned operands, the bf16 planes of large f32
 * products) comes from one fixed device array
 * of mlxhip_gemm_noalloc_scratch_bytes() bytes (64 MiB) per device, held
 * until the process ends; it calls no hipMalloc/hipFree and no allocating
 * library routine. A large f32 product whose bf16 planes (1.5x the f32 bytes
 * of both operands, padded to multiples of 32) and split-K partials do not
 * fit that array runs on the direct f32 MFMA kernel instead, which needs
 * none (e.g. 4096^3 f32: 192 MiB of planes); its result is then within the
 * f32 bound but not bit-identical to mlxhip_gemm's. Any other product whose
 * workspace exceeds the array returns MLXHIP_ERR_INVALID_ARGUMENT (C is then
 * unchanged). Every call on one device
 * shares that device's array: calls that overlap on one device (several
 * streams or threads at once) race, so the caller serialises them. A call on
 * a different stream than the previous call on that device, made while the
 * previous call's kernels have not finished, returns
 * MLXHIP_ERR_INVALID_ARGUMENT instead of racing (C unchanged); this check
 * is skipped for calls made under stream capture. */
int mlxhip_gemm_noalloc(int32_t ab_dtype, int32_t c_dtype, int32_t trans_a, int32_t trans_b,
                        int64_t m, int64_t n, int64_t k, int64_t batch,
                        const void* a, int64_t lda, int64_t stride_a,
                        const void* b, int64_t ldb, int64_t stride_b,
                        void* c, int64_t ldc, int64_t stride_c,
                        void* stream);
/* Bytes of the fixed device scratch mlxhip_gemm_noalloc draws from. */
size_t mlxhip_gemm_noalloc_scratch_bytes(void);

/* Row-wise softmax over the last axis of a [rows, cols] f32 matrix
 * (softmax, crates/mlx-core/src/cpu_kernels.rs:276-315, axis = -1). */
int mlxhip_softmax_rows(const float* x, float* y, int64_t rows, int64_t cols, void* stream);
/* Row softmax of x*scale with the causal fill -1e9 for col > row
 * (scaled_masked_softmax, cpu_kernels.rs:671-712); causal is 0/1. */
int mlxhip_scaled_masked_softmax_rows(const float* x, float* y, int64_t rows, int64_t cols,
                                      float scale, int32_t causal, void* stream);
/* LayerNorm without affine over the last axis (layer_norm, cpu_kernels.rs:338-363). */
int mlxhip_layernorm_rows(const float* x, float* y, int64_t rows, int64_t cols,
                          float eps, void* stream);
/* RMSNorm without weight over the last axis (rms_norm, cpu_kernels.rs:647-669). */
int mlxhip_rmsnorm_rows(const float* x, float* y, int64_t rows, int64_t cols,
                        float eps, void* stream);
/* SoftmaxVjp, last axis: dx = s*(dy - sum(dy*s)) (softmax_vjp, cpu_kernels.rs:515-553). */
int mlxhip_softmax_vjp_rows(const float* dy, const float* s, float* dx,
                            int64_t rows, int64_t cols, void* stream);
/* LayerNormVjp (layer_norm_vjp, cpu_kernels.rs:403-454). */
int mlxhip_layernorm_vjp_rows(const float* dy, const float* x, float* dx,
                              int64_t rows, int64_t cols, float eps, void* stream);
/* RmsNormVjp (rms_norm_vjp, cpu_kernels.rs:462-510). */
int mlxhip_rmsnorm_vjp_rows(const float* dy, const float* x, float* dx,
                            int64_t rows, int64_t cols, float eps, void* stream);

/* Fused elementwise chain. acc starts as inputs[0][i]; each instruction
 * updates it in order; out[i] = acc. Every input is read once and out is
 * written once, whatever the chain length. Each instruction's arithmetic is
 * the f32 operation of the matching OpKind (cpu_kernels.rs:24-35,51-67,
 * 85-88,104-106, 558-606), rounded to f32 after every step exactly as the
 * unfused graph would (no contraction into FMA). */
typedef enum {
    MLXHIP_EW_ADD = 0,    /* acc = acc + in[operand] */
    MLXHIP_EW_SUB = 1,    /* acc = acc - in[operand] */
    MLXHIP_EW_RSUB = 2,   /* acc = in[operand] - acc */
    MLXHIP_EW_MUL = 3,    /* acc = acc * in[operand] */
    MLXHIP_EW_DIV = 4,    /* acc = acc / in[operand] */
    MLXHIP_EW_RDIV = 5,   /* acc = in[operand] / acc */
    MLXHIP_EW_NEG = 6,    /* acc = -acc */
    MLXHIP_EW_EXP = 7,
    MLXHIP_EW_LOG = 8,
    MLXHIP_EW_SQRT = 9,
    MLXHIP_EW_SILU = 10,
    MLXHIP_EW_GELU = 11,
    MLXHIP_EW_SILU_VJP = 12, /* acc = in[operand] * silu'(acc)  (dy = in[operand]) */
    MLXHIP_EW_GELU_VJP = 13, /* acc = in[operand] * gelu'(acc) */
    MLXHIP_EW_COUNT_ = 14
} mlxhip_ew_op_t;

typedef struct {
    int32_t op;       /* mlxhip_ew_op_t */
    int32_t operand;  /* input index for binary ops; ignored by unary ops */
} mlxhip_ew_instr_t;

#define MLXHIP_EW_MAX_INSTR 16
#define MLXHIP_EW_MAX_INPUTS 8

int mlxhip_ew_chain(const mlxhip_ew_instr_t* prog, size_t n_instr,
                    const float* const* inputs, size_t n_inputs,
                    float* out, int64_t numel, void* stream);

/* Fused scaled, masked attention of `batch` heads (cpu_attention,
 * crates/mlx-core/src/cpu_kernels.rs:738-812, per head): for each b,
 *   O_b = softmax(Q_b K_b^T * scale, with -1e9 where causal && key > query) V_b,
 * Q_b and O_b [tq, dh], K_b and V_b [tk, dh], f32, contiguous and packed one
 * head after another (head b starts at b*tq*dh / b*tk*dh); Q, K, V and O
 * 16-byte aligned. Keys are streamed in tiles with a running softmax, so tk is
 * not bounded by on-chip memory; dh must be 16, 32, 64 or 128, otherwise
 * MLXHIP_ERR_INVALID_ARGUMENT. The f32 products run on the bf16 matrix
 * cores as exact three-term splits (f32-level accuracy); a non-finite Q, K
 * or V element makes its rows NaN where the reference may give +-inf. The
 * Attention op
 * of mlxhip_eval_node* uses this kernel when the shape allows and the
 * GEMM + softmax + GEMM sequence otherwise. Replaces the per-head Narrow +
 * Attention of MultiHeadAttention (crates/mlx-nn/src/attention.rs:47-111)
 * with one launch (several for a batch whose workgroups exceed one
 * dispatch's 32-bit work-item count). */
int mlxhip_attention(const float* q, const float* k, const float* v, float* o,
                     int64_t batch, int64_t tq, int64_t tk, int64_t dh,
                     float scale, int32_t causal, void* stream);

/* Gradient of mlxhip_attention for `batch` packed heads of t queries and t
 * keys (dh = 64, t a multiple of 64): given Q, K, V, the forward output O
 * and its cotangent dO ([batch][t][dh] f32 each), writes dQ, dK and dV of the
 * same shape. No reference counterpart: the reference's Attention op has no
 * VJP (crates/mlx-autograd/src/vjp.rs:173-176); this is the standard one
 * (P = softmax(scale Q K^T) under the causal mask, dS = P o (dO V^T - rowsum(dO o O)),
 * dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO), streamed over blocks of
 * 64 keys / queries with f32 matrix-core products; nothing of size t x t is
 * stored. Operands 16-byte aligned; any other shape MLXHIP_ERR_INVALID_ARGUMENT.
 * Row statistics go to a per-stream workspace. */
int mlxhip_attention_vjp(const float* q, const float* k, const float* v, const float* o,
                         const float* dout, float* dq, float* dk, float* dv, int64_t batch,
                         int64_t t, int64_t dh, float scale, int32_t causal, void* stream);

/* 2-D transpose y[cols, rows] = x[rows, cols]^T of 4-byte elements
 * (transpose, cpu_kernels.rs:232-274, axes = None on rank 2). Bit-exact. */
int mlxhip_transpose2d(const float* x, float* y, int64_t rows, int64_t cols, void* stream);

/* Element type conversion of n elements: f32 -> bf16/f16 round to nearest
 * even, bf16/f16 -> f32 exact, same-type copy. */
int mlxhip_cast(const void* x, int32_t src_dtype, void* y, int32_t dst_dtype,
                int64_t n, void* stream);

/* ── Greedy decoding of a decoder-only language model ───────────────────────
 * The token loop of crates/mlx-conformance/tests/ttft_behavior.rs:101-216
 * (project the new token, append K/V to the cache, attend over the cache)
 * for a model built from mlx-nn layers: Embedding (crates/mlx-nn/src/embed.rs),
 * n_layers pre-norm blocks h = x + attn(rms_norm(x)), y = h + W2 silu(W1
 * rms_norm(h) + b1) + b2 with Linear (linear.rs:34-43: y = x W^T + b) Q/K/V/O
 * projections and n_heads heads of d_model/n_heads, a final RmsNorm and an
 * LM-head Linear without bias, then argmax (host-side in the reference).
 * Parameters are held in HBM as bf16 (round to nearest even of the given f32
 * values); activations, the KV cache and accumulation are f32. The reference
 * keeps the KV cache in host vectors and re-uploads it every step; here the
 * cache, the token history and the argmax stay on the device and one step is
 * replayed as a HIP graph. Prompt tokens are consumed one position per step.
 * Requirements: max_batch <= 8, d_model and hidden multiples of 32,
 * head_dim (d_model / n_heads) one of 8, 16, 32, 64, 128, 256. The captured
 * graph of a (batch, prompt_len[, positions with logits]) shape is kept for
 * later calls of the same shape. */
typedef struct {
    int32_t n_layers;
    int32_t d_model;
    int32_t n_heads;
    int32_t hidden;      /* MLP width */
    int32_t vocab;
    int32_t max_batch;   /* sequences per call, <= 8 */
    int32_t max_seq;     /* KV-cache positions: prompt_len + n_new - 1 <= max_seq */
    float eps;           /* RmsNorm eps */
} mlxhip_decoder_config_t;

typedef enum {
    MLXHIP_DEC_EMBEDDING = 0, /* [vocab, d_model] (layer ignored) */
    MLXHIP_DEC_LM_HEAD = 1,   /* [vocab, d_model] (layer ignored) */
    MLXHIP_DEC_WQ = 2,        /* [d_model, d_model], Linear weight [out, in] */
    MLXHIP_DEC_BQ = 3,        /* [d_model] */
    MLXHIP_DEC_WK = 4,
    MLXHIP_DEC_BK = 5,
    MLXHIP_DEC_WV = 6,
    MLXHIP_DEC_BV = 7,
    MLXHIP_DEC_WO = 8,
    MLXHIP_DEC_BO = 9,
    MLXHIP_DEC_W1 = 10,       /* [hidden, d_model] */
    MLXHIP_DEC_B1 = 11,       /* [hidden] */
    MLXHIP_DEC_W2 = 12,       /* [d_model, hidden] */
    MLXHIP_DEC_B2 = 13        /* [d_model] */
} mlxhip_decoder_param_t;

/* generate() flag: launch the step's kernels one by one instead of replaying
 * a captured HIP graph (same results bit for bit). */
#define MLXHIP_DEC_EAGER 1

typedef struct mlxhip_decoder_t mlxhip_decoder_t;

/* Allocates the model's parameters, KV cache and step state in HBM of the
 * current device. NULL on failure (invalid config: MLXHIP_ERR_INVALID_ARGUMENT,
 * checked before the device; no GPU: MLXHIP_ERR_BACKEND_UNAVAILABLE). */
mlxhip_decoder_t* mlxhip_decoder_new(const mlxhip_decoder_config_t* cfg);
void mlxhip_decoder_free(mlxhip_decoder_t* dec);
/* Loads one parameter from `len` row-major f32 host values (rounded to bf16).
 * `layer` selects the block for the per-layer parameters. */
int mlxhip_decoder_set_param(mlxhip_decoder_t* dec, int32_t layer, int32_t which,
                             const float* values, size_t len);
/* Greedy generation for `batch` sequences: prompt [batch, prompt_len] token
 * ids (clamped to [0, vocab-1] as embedding_lookup does,
 * crates/mlx-core/src/cpu_kernels.rs:317-336); tokens_out [batch, n_new]
 * receives the argmax tokens after positions prompt_len-1 .. prompt_len+n_new-2
 * (equal logits resolve to the lowest id). Optional outputs (NULL to skip),
 * with S = prompt_len + n_new - 1 positions: argmax_out [batch, S], the argmax
 * after every position; logits_out [batch, S, vocab]. Synchronous. */
int mlxhip_decoder_generate(mlxhip_decoder_t* dec, const int32_t* prompt, int32_t batch,
                            int32_t prompt_len, int32_t n_new, int32_t* tokens_out,
                            int32_t* argmax_out, float* logits_out, int32_t flags);
/* Device time (HIP events on the decoder's stream) of the last generate's
 * S positions, and S. */
int mlxhip_decoder_last_timing(const mlxhip_decoder_t* dec, float* ms, int32_t* steps);
/* Bytes of bf16 parameters held in HBM (0 for NULL). */
size_t mlxhip_decoder_weight_bytes(const mlxhip_decoder_t* dec);

/* ── Timing (HIP events, for benchmarks) ─────────────────────────────────── */

typedef struct mlxhip_event_t mlxhip_event_t;
mlxhip_event_t* mlxhip_event_create(void);
void mlxhip_event_destroy(mlxhip_event_t* e);
int mlxhip_event_record(mlxhip_event_t* e, void* stream);
/* Milliseconds between two recorded events (waits for `end`). */
int mlxhip_event_elapsed_ms(const mlxhip_event_t* start, const mlxhip_event_t* end, float* ms);

/* Creates / destroys a HIP stream at the default priority. */
void* mlxhip_stream_create_hip(void);
void mlxhip_stream_destroy_hip(void* stream);

/* ── Recorded launch sequences (HIP graphs) ──────────────────────────────
 * For callers whose loops are launch-bound (many small kernels): the direct
 * kernel entry points called on `stream` between mlxhip_graph_begin and
 * mlxhip_graph_end, by the calling thread, are recorded instead of run;
 * mlxhip_graph_launch replays the whole sequence with the same arguments.
 * `stream` must be a created stream (not NULL). The Stream and decoder
 * objects and mlxhip_eval_node synchronise internally and cannot be
 * recorded. No reference counterpart (the reference evaluates each node
 * when asked, crates/mlx-core/src/backend.rs:85-159). */
typedef struct mlxhip_graph_t mlxhip_graph_t;
int mlxhip_graph_begin(void* stream);
/* NULL on failure (e.g. a recorded call failed or synchronised). */
mlxhip_graph_t* mlxhip_graph_end(void* stream);
int mlxhip_graph_launch(mlxhip_graph_t* graph, void* stream);
void mlxhip_graph_free(mlxhip_graph_t* graph);

#ifdef __cplusplus
}
#endif

#endif /* MLXHIP_H */
