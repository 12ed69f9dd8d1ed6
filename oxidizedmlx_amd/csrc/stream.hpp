// stream.hpp — graph state of the HBM-resident Stream (stream.cpp) shared
// with reverse-mode autograd (autograd.cpp).
#pragma once

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "backend.hpp"
#include "common.hpp"

namespace mlxhip {

struct OpVal {
    mlxhip_op_t op{};
    std::vector<int64_t> shape, axes;
    bool has_shape = false, has_axes = false;

    static OpVal from(const mlxhip_op_t& o) {
        OpVal v;
        v.op = o;
        if (o.shape) {
            v.shape.assign(o.shape, o.shape + o.shape_len);
            v.has_shape = true;
        }
        if (o.axes) {
            v.axes.assign(o.axes, o.axes + o.axes_len);
            v.has_axes = true;
        }
        return v;
    }
    mlxhip_op_t c() const {
        mlxhip_op_t o = op;
        o.shape = has_shape ? shape.data() : nullptr;
        o.shape_len = shape.size();
        o.axes = has_axes ? axes.data() : nullptr;
        o.axes_len = axes.size();
        return o;
    }
};

struct MetaVal {
    std::vector<int64_t> shape;
    int dtype = MLXHIP_DTYPE_F32;
    int64_t numel() const { return numel_of(shape.data(), shape.size()); }
    mlxhip_meta_t c() const { return mlxhip_meta_t{shape.data(), shape.size(), dtype}; }
};

struct Node {
    uint64_t id;
    OpVal op;
    std::vector<uint64_t> inputs;
    MetaVal meta;
};

struct DevBuf {
    float* ptr = nullptr;
    size_t len = 0;
    bool owned = true;  // false: aliases another node's buffer (Reshape)
};

inline void append_bits(std::string& k, const void* p, size_t n) { k.append(static_cast<const char*>(p), n); }


}  // namespace mlxhip

struct mlxhip_stream_t {
    std::mutex mu;  // guards everything below; eval runs under it
    std::unordered_map<uint64_t, mlxhip::Node> nodes;
    std::unordered_map<std::string, uint64_t> cse;
    std::unordered_map<uint64_t, uint32_t> consumers;
    std::unordered_map<uint64_t, mlxhip::DevBuf> buffers;
    uint64_t next_id = 1;
    std::atomic<uint64_t> eval_calls{0};
    std::atomic<uint64_t> launches{0};
    // Nodes read or written in place and never materialised (attention head
    // views): counted in eval_calls once, however many evaluations plan them.
    std::unordered_set<uint64_t> counted_views;
    bool fusion = true;
    // Asynchronous evaluation (mlxhip_stream_set_async): eval returns once
    // its kernels are enqueued. Blocks released while queued kernels may
    // still use them wait in `pending` (size, block) until the stream drains
    // (get_buffer, synchronize, free); meanwhile later work of this stream may
    // take them at once (stream_alloc), since the stream runs in order.
    bool async_eval = false;
    std::vector<std::pair<size_t, void*>> pending;
    hipStream_t hs = nullptr;
    int device = 0;
    // A second queue for leaf reductions (created on first use): an axis
    // reduction that no node consumes is a long chain of dependent adds on a
    // few CUs (the bias gradients of a block), and runs beside the rest of
    // the evaluation instead of between its kernels. It starts after
    // everything queued on hs before it (fork event), and hs waits for it
    // at the end of the evaluation (join event), so to every later user the
    // two queues are one. Default priority, like hs.
    hipStream_t side = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    bool side_pending = false;
    // bf16 planes of the f32 operands of this stream's split-f32 products,
    // kept until clear() so products in later evaluations reuse them (the
    // forward's weights and activations in the gradient's evaluation). A
    // node's buffer is never written again while the node exists (view
    // constants by the contract of add_constant_view), and a block released
    // before clear() drops the planes made from it (release_later).
    mlxhip::PlaneCache planes;
    std::vector<void*> plane_blocks;

    mlxhip_stream_t() {
        planes.alloc = [](void* ctx, size_t bytes) {
            auto* self = static_cast<mlxhip_stream_t*>(ctx);
            void* p = self->stream_alloc(bytes);
            if (p) self->plane_blocks.push_back(p);
            return p;
        };
        planes.ctx = this;
    }
    mlxhip_stream_t(const mlxhip_stream_t&) = delete;
    mlxhip_stream_t& operator=(const mlxhip_stream_t&) = delete;

    ~mlxhip_stream_t() {
        // The queues' cached workspaces (split-K partials, padded operand
        // copies, reduction partials, attention-gradient row statistics) are
        // keyed by (device, queue): return them to the pool with this
        // stream's device current, once the queues are idle, before the
        // handles die (a later queue may reuse the handle value).
        int cur = 0;
        const bool have_cur = hipGetDevice(&cur) == hipSuccess;
        if (have_cur && cur != device) (void)hipSetDevice(device);
        if (side && hipStreamSynchronize(side) == hipSuccess) mlxhip::release_stream_workspaces(side);
        if (hs && hipStreamSynchronize(hs) == hipSuccess) mlxhip::release_stream_workspaces(hs);
        if (have_cur && cur != device) (void)hipSetDevice(cur);
        (void)hipGetLastError();
        for (auto& b : pending) mlxhip::pool_release(b.second);
        for (auto& kv : buffers)
            if (kv.second.owned) mlxhip::pool_release(kv.second.ptr);
        for (void* p : plane_blocks) mlxhip::pool_release(p);
        if (fork_ev) (void)hipEventDestroy(fork_ev);
        if (join_ev) (void)hipEventDestroy(join_ev);
        if (side) (void)hipStreamDestroy(side);
        if (hs) (void)hipStreamDestroy(hs);
    }

    // The side queue, ready to start after all work queued so far on hs.
    int fork_side(hipStream_t* out) {
        if (!side) {
            MLXHIP_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
            MLXHIP_HIP(hipEventCreateWithFlags(&fork_ev, hipEventDisableTiming));
            MLXHIP_HIP(hipEventCreateWithFlags(&join_ev, hipEventDisableTiming));
        }
        MLXHIP_HIP(hipEventRecord(fork_ev, hs));
        MLXHIP_HIP(hipStreamWaitEvent(side, fork_ev, 0));
        side_pending = true;
        *out = side;
        return MLXHIP_OK;
    }

    // hs waits for the side queue's work (end of an evaluation).
    int join_side() {
        if (!side_pending) return MLXHIP_OK;
        side_pending = false;
        MLXHIP_HIP(hipEventRecord(join_ev, side));
        MLXHIP_HIP(hipStreamWaitEvent(hs, join_ev, 0));
        return MLXHIP_OK;
    }

    // Waits for every kernel of this stream, then returns the blocks of
    // earlier asynchronous evaluations to the pool.
    int drain() {
        const hipError_t e = hipStreamSynchronize(hs);
        for (auto& b : pending) mlxhip::pool_release(b.second);
        pending.clear();
        return e == hipSuccess ? MLXHIP_OK : mlxhip::hip_fail(e, "hipStreamSynchronize");
    }

    // A block a kernel of this stream may still use goes back to the pool
    // now (synchronous evaluation: the stream is drained before eval
    // returns) or when the stream drains.
    void release_later(void* p) {
        const size_t sz = mlxhip::pool_block_size(p);
        if (!planes.entries.empty()) {
            const char* lo = static_cast<const char*>(p);
            auto& e = planes.entries;
            for (size_t i = 0; i < e.size();) {
                const char* src = static_cast<const char*>(e[i].src);
                if (src >= lo && src < lo + sz) {
                    e[i] = e.back();
                    e.pop_back();
                } else {
                    ++i;
                }
            }
        }
        if (async_eval) pending.emplace_back(sz, p);
        else mlxhip::pool_release(p);
    }

    // A block for memory that only this stream's queue writes and reads: a
    // pending block of fitting size (the smallest in [size, 1.5 size], as the
    // pool chooses) if there is one, else one from the pool.
    void* stream_alloc(size_t bytes) {
        const size_t sz = mlxhip::pool_round(bytes);
        size_t best = 0;
        bool found = false;
        for (size_t i = 0; i < pending.size(); ++i) {
            const size_t b = pending[i].first;
            if (b >= sz && b <= sz + sz / 2 && (!found || b < pending[best].first)) {
                best = i;
                found = true;
            }
        }
        if (found) {
            void* p = pending[best].second;
            pending[best] = pending.back();
            pending.pop_back();
            return p;
        }
        return mlxhip::pool_alloc(bytes);
    }

    // Forgets every node (mlxhip_stream_clear); their blocks go back through
    // release_later. Node ids are never reused.
    int clear() {
        if (!async_eval) {
            // Queued device-to-device constant copies may still write them.
            const hipError_t e = hipStreamSynchronize(hs);
            if (e != hipSuccess) return mlxhip::hip_fail(e, "hipStreamSynchronize");
        }
        planes.entries.clear();
        for (void* p : plane_blocks) release_later(p);
        plane_blocks.clear();
        for (auto& kv : buffers)
            if (kv.second.owned) release_later(kv.second.ptr);
        buffers.clear();
        nodes.clear();
        cse.clear();
        consumers.clear();
        counted_views.clear();
        return MLXHIP_OK;
    }

    uint64_t add_node(const mlxhip::OpVal& op, std::vector<uint64_t> inputs, const mlxhip::MetaVal& meta, bool cse_ok) {
        std::string key;
        if (cse_ok) {
            if ((op.op.kind == MLXHIP_OP_ADD || op.op.kind == MLXHIP_OP_MUL) && inputs.size() == 2 &&
                inputs[0] > inputs[1])
                std::swap(inputs[0], inputs[1]);
            mlxhip_op_t o = op.op;
            o.shape = nullptr;
            o.axes = nullptr;
            mlxhip::append_bits(key, &o, sizeof o);
            key.push_back(op.has_shape ? 'S' : 's');
            mlxhip::append_bits(key, op.shape.data(), op.shape.size() * sizeof(int64_t));
            key.push_back(op.has_axes ? 'A' : 'a');
            mlxhip::append_bits(key, op.axes.data(), op.axes.size() * sizeof(int64_t));
            key.push_back('I');
            mlxhip::append_bits(key, inputs.data(), inputs.size() * sizeof(uint64_t));
            key.push_back('M');
            mlxhip::append_bits(key, &meta.dtype, sizeof meta.dtype);
            mlxhip::append_bits(key, meta.shape.data(), meta.shape.size() * sizeof(int64_t));
            auto it = cse.find(key);
            if (it != cse.end()) return it->second;
        }
        const uint64_t id = next_id++;
        for (uint64_t in : inputs) consumers[in]++;
        nodes.emplace(id, mlxhip::Node{id, op, std::move(inputs), meta});
        if (cse_ok) cse.emplace(std::move(key), id);
        return id;
    }

    // Depth-first post-order of the subgraph rooted at `outs` (graph.rs:268-294:
    // one shared visited set, outputs in order, inputs in order), iterative so
    // deep graphs cannot overflow the native stack.
    // stop_at_buffers: a node that holds its buffer needs none of its inputs,
    // so the walk does not go past it (evaluation); else the whole graph
    // behind `outs` (autograd).
    std::vector<uint64_t> topo_sort(const std::vector<uint64_t>& outs, bool stop_at_buffers = false) {
        std::vector<uint64_t> order;
        std::unordered_set<uint64_t> visited;
        std::vector<std::pair<uint64_t, size_t>> st;
        for (uint64_t out : outs) {
            if (!visited.insert(out).second) continue;
            st.emplace_back(out, 0);
            while (!st.empty()) {
                auto& top = st.back();
                auto it = nodes.find(top.first);
                // Past a node with a buffer, an evaluation would meet nodes
                // that were never materialised (a MatMul whose result went
                // into its bias Add's buffer, a fused chain's interior) and
                // evaluate them again.
                if (it != nodes.end() && !(stop_at_buffers && buffers.count(top.first)) &&
                    top.second < it->second.inputs.size()) {
                    const uint64_t nxt = it->second.inputs[top.second++];
                    if (visited.insert(nxt).second) st.emplace_back(nxt, 0);
                } else {
                    order.push_back(top.first);
                    st.pop_back();
                }
            }
        }
        return order;
    }

    mlxhip_input_t input_of(uint64_t id, const float* data) {
        const mlxhip::Node& n = nodes.at(id);
        return mlxhip_input_t{data, (size_t)n.meta.numel(), n.meta.shape.data(), n.meta.shape.size(), n.meta.dtype};
    }

    // Stream::add_constant (backend.rs:59-71): a Constant node (never CSE'd)
    // whose data is copied into a new HBM buffer at once, from host memory or,
    // with device_src, from device memory (ordered before every later kernel
    // on this stream).
    int add_constant(const float* data, size_t len, const mlxhip::MetaVal& mv, bool device_src, uint64_t* id) {
        if ((int64_t)len != mv.numel())
            return mlxhip::fail_shape({mv.numel()}, {(int64_t)len}, "stream_add_constant");
        // Device data is copied on this stream's queue, so the block may be
        // one the stream still has queued work on; host data is copied
        // outside the queue and needs a block no queued kernel uses.
        const size_t bytes = (len ? len : 1) * sizeof(float);
        float* p = static_cast<float*>(device_src ? stream_alloc(bytes) : mlxhip::pool_alloc(bytes));
        if (!p) return mlxhip::fail(MLXHIP_ERR_FFI_FAILED, "stream_add_constant: device allocation failed");
        // Device data: copied on this stream, ordered before its later kernels.
        // Host data (which the caller may free as soon as the call returns):
        // copied by a blocking hipMemcpy, which does not wait for this
        // (non-blocking) stream's queued work. The block is fresh from the
        // pool, where blocks only return once no kernel uses them, so nothing
        // queued touches it, and the kernels that read it are enqueued after
        // the copy has finished.
        if (len) {
            const hipError_t e = device_src ? hipMemcpyAsync(p, data, len * sizeof(float), hipMemcpyDeviceToDevice, hs)
                                            : hipMemcpy(p, data, len * sizeof(float), hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                release_later(p);
                return mlxhip::fail(MLXHIP_ERR_FFI_FAILED, "stream_add_constant: copy failed");
            }
        }
        mlxhip_op_t op{};
        op.kind = MLXHIP_OP_CONSTANT;
        *id = add_node(mlxhip::OpVal::from(op), {}, mv, false);
        buffers[*id] = mlxhip::DevBuf{p, len};
        return MLXHIP_OK;
    }

    // A Constant node that reads `data`, device memory the caller owns, in
    // place (no copy; the node does not own the memory, so clear and free
    // leave it alone). Kernels only ever read a node's inputs.
    int add_constant_view(const float* data, size_t len, const mlxhip::MetaVal& mv, uint64_t* id) {
        if ((int64_t)len != mv.numel()) return mlxhip::fail_shape({mv.numel()}, {(int64_t)len}, "stream_add_constant_view");
        if (reinterpret_cast<uintptr_t>(data) % 256)
            return mlxhip::fail(MLXHIP_ERR_INVALID_ARGUMENT,
                                "stream_add_constant_view: data must be 256-byte aligned (as pool blocks are)");
        mlxhip_op_t op{};
        op.kind = MLXHIP_OP_CONSTANT;
        *id = add_node(mlxhip::OpVal::from(op), {}, mv, false);
        buffers[*id] = mlxhip::DevBuf{const_cast<float*>(data), len, false};
        return MLXHIP_OK;
    }

    int alloc_out(uint64_t id, float** out) {
        const mlxhip::Node& n = nodes.at(id);
        const size_t len = (size_t)n.meta.numel();
        float* p = static_cast<float*>(stream_alloc((len ? len : 1) * sizeof(float)));
        if (!p) return mlxhip::fail(MLXHIP_ERR_FFI_FAILED, "stream: device allocation of %zu floats failed", len);
        buffers[id] = mlxhip::DevBuf{p, len};
        *out = p;
        return MLXHIP_OK;
    }

    // Evaluates every node in `outputs` (and what they depend on) in one
    // scheduling pass.
    int eval(const std::vector<uint64_t>& outputs);
};

