// backend.hpp — HipBackend: the reference's Backend::eval_node
// (crates/mlx-core/src/backend.rs:27-35) over HBM-resident operands, plus the
// device-memory pool the host-vector contract and the Stream use.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/mlxhip.h"
#include "kernels.hpp"

namespace mlxhip {

// Caching pool of device allocations on the current device. release() may
// only be called once no queued GPU work still uses the block (the callers
// synchronise their stream first).
void* pool_alloc(size_t bytes);
void pool_release(void* p);
// The size pool_alloc rounds a request of `bytes` to, and the size of a block
// it handed out (0 for a pointer it does not own).
size_t pool_round(size_t bytes);
size_t pool_block_size(void* p);

// Temporary device buffers of one node evaluation, handed back to the pool
// by the owner after its stream has been synchronised.
struct Scratch {
    std::vector<void*> blocks;
    // Split-f32 planes of the f32 products: by default kept in blocks of this
    // scratch (as long as it lives); a Stream points `planes` at its own
    // cache, which lives until the stream is cleared.
    PlaneCache own_planes;
    PlaneCache* planes = &own_planes;
    Scratch() {
        own_planes.alloc = [](void* ctx, size_t bytes) { return static_cast<Scratch*>(ctx)->get_bytes(bytes); };
        own_planes.ctx = this;
    }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    float* get(size_t n_floats);
    void* get_bytes(size_t bytes);
    void release_all();
    ~Scratch() { release_all(); }
};

inline int64_t numel_of(const int64_t* shape, size_t ndim) {
    int64_t n = 1;
    for (size_t i = 0; i < ndim; ++i) n *= shape[i];
    return n;
}

// Backend::eval_node on device memory: inputs[i].data are device addresses,
// `out` receives numel(out_meta) floats. Asynchronous on `s`; temporaries go
// to `scratch`. `trans_hint` (optional) lets the Stream pass MatMul operands
// whose Transpose node was folded: trans_hint[i] = 1 means inputs[i] holds
// the untransposed source, so the GEMM reads it transposed.
int eval_node_device(const mlxhip_op_t& op, const mlxhip_input_t* inputs, size_t n_inputs,
                     const mlxhip_meta_t& out_meta, float* out, hipStream_t s, Scratch& scratch,
                     const int* trans_hint = nullptr);

// `groups` (2..4) rank-2 MatMuls of one shape and operand layout, evaluated
// together (sibling products of the Stream's graph): group i's operands are
// inputs[2i], inputs[2i + 1] with the folded-Transpose hints hints[2i],
// hints[2i + 1] (the same for every group), its result goes to outs[i].
int eval_matmul_group(int groups, const mlxhip_input_t* inputs, const int* hints, float* const* outs,
                      hipStream_t s, Scratch& scratch, const float* const* biases = nullptr);

// A rank-2 f32 MatMul followed by the Add of a bias row broadcast over its
// rows (out = A B + bias, bias[j] added to column j; the Stream's linear
// layers): the bias is added as C is stored, the same f32 addition a
// separate Add performs. eval_matmul_group's `biases` (one per group, or
// nullptr) do the same for grouped products.
int eval_matmul_bias(const mlxhip_input_t* inputs, const mlxhip_meta_t& out_meta, float* out, hipStream_t s,
                     Scratch& scratch, const int* trans_hint, const float* bias);

// Per-thread HIP stream used by the synchronous host-vector entry points.
hipStream_t thread_stream();

}  // namespace mlxhip
