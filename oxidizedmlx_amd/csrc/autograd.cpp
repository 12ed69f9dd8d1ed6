// autograd.cpp — reverse-mode automatic differentiation over the Stream's
// graph (mlxhip_stream_grad).
//
// Restates value_and_grad / backward (crates/mlx-autograd/src/lib.rs:30-107)
// and the VJP table (crates/mlx-autograd/src/vjp.rs:8-178):
//   * the loss must have one element; it is evaluated first;
//   * the seed d(loss)/d(loss) is a Constant of ones of the loss's shape;
//   * nodes are visited in reverse topological order of the loss's subgraph
//     (the stream's topo_sort, graph.rs:268-294); a node's incoming gradient
//     is taken out of the table, its VJP adds new lazy nodes to the graph, and
//     each input's contribution is accumulated with Add in visiting order;
//   * Constant / Parameter nodes keep their gradient;
//   * a wrt node with no gradient is an error ("gradient not found").
// Differences from the reference, none of which changes a gradient value:
//   * several wrt nodes per call (the reference takes one, lib.rs:104-106);
//   * VJP nodes are built only for inputs from which some wrt node is
//     reachable: an input that cannot reach a wrt node contributes nothing to
//     any requested gradient. A node whose op has no VJP is an error only when
//     one of its inputs needs a gradient;
//   * MatMul of rank 3 ([B,M,K] @ [B,K,N], the batched form of
//     evals/tasks/003_matmul_batch_3d.json) differentiates like rank 2 with
//     the two matrix axes swapped by Transpose [0,2,1] instead of reversing
//     all axes.
// Shapes of the new nodes follow the Tensor methods that build them
// (crates/mlx-core/src/tensor.rs: add/sub/mul/div/neg 167-238, sum_axis
// 243-259, matmul 274-296, reshape 322-337, transpose 340-374, the VJP ops
// 454-580, broadcast_to 769-801).
#include <algorithm>
#include <exception>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "stream.hpp"

namespace mlxhip {
namespace {

// Status of the failure just recorded (INVALID_ARGUMENT if none was).
int recorded_status() {
    const int st = mlxhip_last_status();
    return st != MLXHIP_OK ? st : (int)MLXHIP_ERR_INVALID_ARGUMENT;
}

const char* op_name(int k) {
    static const char* names[MLXHIP_OP_COUNT_] = {
        "Constant", "Parameter", "Add", "Sub", "Mul", "Div", "Neg", "Exp", "Log", "Sum", "Mean", "Max",
        "MatMul", "Reshape", "Transpose", "Softmax", "Silu", "Gelu", "LayerNorm", "RmsNorm", "Rope",
        "Broadcast", "Embedding", "ScaledMaskedSoftmax", "Attention", "LayerNormVjp", "RmsNormVjp",
        "SoftmaxVjp", "SiluVjp", "GeluVjp", "Sqrt", "RoPE", "Narrow", "Concatenate", "HeadAttention",
        "HeadAttentionVjp"};
    return (k >= 0 && k < MLXHIP_OP_COUNT_) ? names[k] : "?";
}

// Adds lazy nodes to the stream (caller holds the stream's lock). Every
// builder returns 0 after recording the failure in the thread's error state,
// and returns 0 at once when given 0 (a failed operand) as an input.
struct Builder {
    mlxhip_stream_t& s;

    const MetaVal& meta(uint64_t id) const { return s.nodes.at(id).meta; }
    const std::vector<int64_t>& shape(uint64_t id) const { return meta(id).shape; }

    uint64_t node(const mlxhip_op_t& o, std::vector<uint64_t> ins, std::vector<int64_t> out_shape, int dtype,
                  const std::vector<int64_t>* op_shape = nullptr, const std::vector<int64_t>* op_axes = nullptr) {
        OpVal v;
        v.op = o;
        if (op_shape) {
            v.shape = *op_shape;
            v.has_shape = true;
        }
        if (op_axes) {
            v.axes = *op_axes;
            v.has_axes = true;
        }
        MetaVal m;
        m.shape = std::move(out_shape);
        m.dtype = dtype;
        return s.add_node(v, std::move(ins), m, true);
    }

    static mlxhip_op_t op(int kind) {
        mlxhip_op_t o{};
        o.kind = kind;
        return o;
    }

    uint64_t constant(const std::vector<float>& data, std::vector<int64_t> shp, int dtype) {
        MetaVal m;
        m.shape = std::move(shp);
        m.dtype = dtype;
        uint64_t id = 0;
        if (s.add_constant(data.data(), data.size(), m, false, &id) != MLXHIP_OK) return 0;
        return id;
    }

    bool same_shape(uint64_t a, uint64_t b, const char* what) {
        if (!a || !b) return false;
        if (shape(a) == shape(b)) return true;
        fail_shape(shape(a), shape(b), what);
        return false;
    }

    uint64_t binary(int kind, uint64_t a, uint64_t b) {
        if (!same_shape(a, b, op_name(kind))) return 0;
        return node(op(kind), {a, b}, shape(a), meta(a).dtype);
    }
    uint64_t add(uint64_t a, uint64_t b) { return binary(MLXHIP_OP_ADD, a, b); }
    uint64_t mul(uint64_t a, uint64_t b) { return binary(MLXHIP_OP_MUL, a, b); }
    uint64_t div(uint64_t a, uint64_t b) { return binary(MLXHIP_OP_DIV, a, b); }
    uint64_t neg(uint64_t a) { return a ? node(op(MLXHIP_OP_NEG), {a}, shape(a), meta(a).dtype) : 0; }

    // VJP ops: inputs [grad, x] (or [grad, softmax output]), output shaped as x.
    uint64_t vjp_op(mlxhip_op_t o, uint64_t g, uint64_t x) {
        if (!same_shape(g, x, op_name(o.kind))) return 0;
        return node(o, {g, x}, shape(x), meta(x).dtype);
    }

    uint64_t transpose(uint64_t a, const std::vector<int64_t>* perm) {
        if (!a) return 0;
        const std::vector<int64_t>& sh = shape(a);
        std::vector<int64_t> p(sh.size());
        if (perm) {
            p = *perm;
        } else {
            for (size_t i = 0; i < sh.size(); ++i) p[i] = (int64_t)(sh.size() - 1 - i);
        }
        std::vector<int64_t> out(sh.size());
        for (size_t i = 0; i < sh.size(); ++i) out[i] = sh[(size_t)p[i]];
        return node(op(MLXHIP_OP_TRANSPOSE), {a}, out, meta(a).dtype, nullptr, perm);
    }

    uint64_t matmul(uint64_t a, uint64_t b) {
        if (!a || !b) return 0;
        const std::vector<int64_t>&sa = shape(a), &sb = shape(b);
        const size_t r = sa.size();
        if (!((r == 2 && sb.size() == 2) || (r == 3 && sb.size() == 3 && sa[0] == sb[0])) ||
            sa[r - 1] != sb[r - 2]) {
            fail_shape(sa, sb, "MatMul");
            return 0;
        }
        std::vector<int64_t> out(sa.begin(), sa.end() - 1);
        out.push_back(sb[r - 1]);
        return node(op(MLXHIP_OP_MATMUL), {a, b}, out, meta(a).dtype);
    }

    uint64_t reshape(uint64_t a, const std::vector<int64_t>& shp) {
        if (!a) return 0;
        return node(op(MLXHIP_OP_RESHAPE), {a}, shp, meta(a).dtype, &shp);
    }

    uint64_t broadcast_to(uint64_t a, const std::vector<int64_t>& target) {
        if (!a) return 0;
        if (shape(a) == target) return a;  // tensor.rs:770-772
        return node(op(MLXHIP_OP_BROADCAST), {a}, target, meta(a).dtype, &target);
    }

    uint64_t sum_axis(uint64_t a, int64_t ax) {
        if (!a) return 0;
        mlxhip_op_t o = op(MLXHIP_OP_SUM);
        o.axis = (int32_t)ax;
        o.has_axis = 1;
        std::vector<int64_t> out = shape(a);
        out.erase(out.begin() + ax);
        return node(o, {a}, out, meta(a).dtype);
    }
};

// Gradients of `n`'s inputs for output gradient `g` (vjp.rs:8-178). Entries
// for inputs with need[i] false are left 0 and not built.
int vjp(Builder& b, uint64_t id, const Node& n, uint64_t g, const std::vector<bool>& need,
        std::vector<uint64_t>& out) {
    const std::vector<uint64_t>& in = n.inputs;
    out.assign(in.size(), 0);
    const int k = n.op.op.kind;
    auto arity = [&](size_t want) {
        if (in.size() >= want) return true;
        fail(MLXHIP_ERR_INVALID_ARGUMENT, "%s node has %zu inputs, expected %zu", op_name(k), in.size(), want);
        return false;
    };
#define MLXHIP_NEED(i) (need[i])
#define MLXHIP_SET(i, expr)                        \
    do {                                           \
        if (MLXHIP_NEED(i)) {                      \
            out[i] = (expr);                       \
            if (!out[i]) return recorded_status(); \
        }                                          \
    } while (0)
    switch (k) {
        case MLXHIP_OP_ADD:
            if (!arity(2)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, g);
            MLXHIP_SET(1, g);
            return MLXHIP_OK;
        case MLXHIP_OP_SUB:
            if (!arity(2)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, g);
            MLXHIP_SET(1, b.neg(g));
            return MLXHIP_OK;
        case MLXHIP_OP_MUL:
            if (!arity(2)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, b.mul(g, in[1]));
            MLXHIP_SET(1, b.mul(g, in[0]));
            return MLXHIP_OK;
        case MLXHIP_OP_DIV: {
            if (!arity(2)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, b.div(g, in[1]));
            if (need[1]) {
                const uint64_t neg_a = b.neg(in[0]);
                const uint64_t b_sq = b.mul(in[1], in[1]);
                MLXHIP_SET(1, b.div(b.mul(g, neg_a), b_sq));
            }
            return MLXHIP_OK;
        }
        case MLXHIP_OP_NEG:
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, b.neg(g));
            return MLXHIP_OK;
        case MLXHIP_OP_SUM: {
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            const std::vector<int64_t>& ish = b.shape(in[0]);
            if (!n.op.op.has_axis) {
                MLXHIP_SET(0, b.broadcast_to(g, ish));
            } else {
                int64_t ax = n.op.op.axis;
                if (ax < 0) ax += (int64_t)ish.size();
                std::vector<int64_t> unsq = b.shape(g);
                unsq.insert(unsq.begin() + std::min<int64_t>(std::max<int64_t>(ax, 0), (int64_t)unsq.size()), 1);
                MLXHIP_SET(0, b.broadcast_to(b.reshape(g, unsq), ish));
            }
            return MLXHIP_OK;
        }
        case MLXHIP_OP_MATMUL: {
            if (!arity(2)) return MLXHIP_ERR_INVALID_ARGUMENT;
            // Rank 2: Transpose(None); rank 3: swap the matrix axes only.
            static const std::vector<int64_t> swap3 = {0, 2, 1};
            const std::vector<int64_t>* perm = b.shape(in[0]).size() == 3 ? &swap3 : nullptr;
            MLXHIP_SET(0, b.matmul(g, b.transpose(in[1], perm)));
            MLXHIP_SET(1, b.matmul(b.transpose(in[0], perm), g));
            return MLXHIP_OK;
        }
        case MLXHIP_OP_RESHAPE:
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, b.reshape(g, b.shape(in[0])));
            return MLXHIP_OK;
        case MLXHIP_OP_TRANSPOSE: {
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            const size_t nd = b.shape(in[0]).size();
            std::vector<int64_t> perm(nd), inv(nd);
            for (size_t i = 0; i < nd; ++i) perm[i] = n.op.has_axes ? n.op.axes[i] : (int64_t)(nd - 1 - i);
            for (size_t i = 0; i < nd; ++i) inv[(size_t)perm[i]] = (int64_t)i;
            MLXHIP_SET(0, b.transpose(g, &inv));
            return MLXHIP_OK;
        }
        case MLXHIP_OP_LAYER_NORM:
        case MLXHIP_OP_RMS_NORM: {
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            mlxhip_op_t o = Builder::op(k == MLXHIP_OP_LAYER_NORM ? MLXHIP_OP_LAYER_NORM_VJP : MLXHIP_OP_RMS_NORM_VJP);
            o.eps = n.op.op.eps;
            MLXHIP_SET(0, b.vjp_op(o, g, in[0]));
            return MLXHIP_OK;
        }
        case MLXHIP_OP_SOFTMAX: {
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            if (need[0]) {
                // The forward node's own op over its own input: CSE returns
                // the forward node (an op differing in any field, such as
                // has_axis, would make a second Softmax that evaluates again),
                // then SoftmaxVjp [grad, softmax output].
                mlxhip_op_t so = n.op.op;
                so.shape = nullptr;
                so.shape_len = 0;
                so.axes = nullptr;
                so.axes_len = 0;
                const uint64_t sm = b.node(so, {in[0]}, b.shape(in[0]), b.meta(in[0]).dtype);
                mlxhip_op_t o = Builder::op(MLXHIP_OP_SOFTMAX_VJP);
                o.axis = n.op.op.axis;
                MLXHIP_SET(0, b.vjp_op(o, g, sm));
            }
            return MLXHIP_OK;
        }
        case MLXHIP_OP_HEAD_ATTENTION: {
            // One HeadAttentionVjp node [q, k, v, o = this node, g] gives
            // [3, <input shape>]; input i's gradient is its slice i (a Narrow
            // along the leading axis, which the stream reads in place).
            if (!arity(3)) return MLXHIP_ERR_INVALID_ARGUMENT;
            if (!b.same_shape(g, id, "HeadAttention")) return recorded_status();
            const std::vector<int64_t> sh = b.shape(id);
            {
                // The gradient kernels' shape limits, checked here so that an
                // unsupported shape fails when the gradient is built, not
                // when it is first evaluated.
                const int64_t hg = n.op.op.has_axis ? n.op.op.axis : 1;
                const int64_t t = sh.size() == 3 ? sh[1] : 0, w = sh.size() == 3 ? sh[2] : 0;
                if (sh.size() != 3 || hg < 1 || w % hg || !mlxhip::attention_vjp_supported(w / hg, t, t))
                    return fail(MLXHIP_ERR_INVALID_ARGUMENT,
                                "HeadAttention gradient: the fused gradient needs [heads, t, dh] operands with "
                                "dh = 64 and t a multiple of 64 (got t=%lld, %lld heads per row of %lld values); "
                                "compose the attention from MatMul and Softmax to differentiate other shapes",
                                (long long)t, (long long)hg, (long long)w);
            }
            std::vector<int64_t> vsh{3};
            vsh.insert(vsh.end(), sh.begin(), sh.end());
            mlxhip_op_t vo = Builder::op(MLXHIP_OP_HEAD_ATTENTION_VJP);
            vo.scale = n.op.op.scale;
            vo.causal = n.op.op.causal;
            vo.axis = n.op.op.axis;  // heads per row, as the forward's
            vo.has_axis = n.op.op.has_axis;
            const uint64_t all = b.node(vo, {in[0], in[1], in[2], id, g}, vsh, b.meta(id).dtype);
            if (!all) return recorded_status();
            std::vector<int64_t> one{1};
            one.insert(one.end(), sh.begin(), sh.end());
            for (int i = 0; i < 3; ++i) {
                mlxhip_op_t no = Builder::op(MLXHIP_OP_NARROW);
                no.axis = 0;
                no.has_axis = 1;
                no.start = i;
                no.length = 1;
                MLXHIP_SET(i, b.reshape(b.node(no, {all}, one, b.meta(id).dtype), sh));
            }
            return MLXHIP_OK;
        }
        case MLXHIP_OP_SILU:
        case MLXHIP_OP_GELU:
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            MLXHIP_SET(0, b.vjp_op(Builder::op(k == MLXHIP_OP_SILU ? MLXHIP_OP_SILU_VJP : MLXHIP_OP_GELU_VJP), g, in[0]));
            return MLXHIP_OK;
        case MLXHIP_OP_BROADCAST: {
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            if (!need[0]) return MLXHIP_OK;
            // Sum over the padded leading axes, then over the axes broadcast
            // from size 1, keeping them as size 1.
            const std::vector<int64_t> ish = b.shape(in[0]);
            uint64_t gi = g;
            if (b.shape(g).size() < ish.size())
                return fail_shape(ish, b.shape(g), "Broadcast gradient");
            const size_t pad = b.shape(g).size() - ish.size();
            for (size_t i = 0; i < pad && gi; ++i) gi = b.sum_axis(gi, 0);
            for (size_t i = 0; i < ish.size() && gi; ++i) {
                if (ish[i] == 1 && b.shape(gi)[i] != 1) {
                    gi = b.sum_axis(gi, (int64_t)i);
                    if (!gi) break;
                    std::vector<int64_t> dims = b.shape(gi);
                    dims.insert(dims.begin() + (int64_t)i, 1);
                    gi = b.reshape(gi, dims);
                }
            }
            MLXHIP_SET(0, gi);
            return MLXHIP_OK;
        }
        case MLXHIP_OP_SQRT: {
            if (!arity(1)) return MLXHIP_ERR_INVALID_ARGUMENT;
            if (!need[0]) return MLXHIP_OK;
            // grad / (2 * (sqrt(x) + f32::EPSILON)), with the output node as sqrt(x).
            const int dt = n.meta.dtype;
            const uint64_t eps = b.constant({1.1920929e-07f}, {}, dt);
            const uint64_t two = b.constant({2.0f}, {}, dt);
            if (!eps || !two) return recorded_status();
            const uint64_t safe = b.add(id, b.broadcast_to(eps, n.meta.shape));
            MLXHIP_SET(0, b.div(g, b.mul(safe, b.broadcast_to(two, n.meta.shape))));
            return MLXHIP_OK;
        }
        default:
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "VJP not implemented for %s", op_name(k));
    }
#undef MLXHIP_SET
#undef MLXHIP_NEED
}

}  // namespace
}  // namespace mlxhip

using namespace mlxhip;

namespace {

int stream_grad(mlxhip_stream_t* s, uint64_t loss, const uint64_t* wrt, size_t n_wrt, uint64_t* grads) {
    MLXHIP_HIP(hipSetDevice(s->device));
    auto ln = s->nodes.find(loss);
    if (ln == s->nodes.end()) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "stream_grad: unknown loss node");
    for (size_t i = 0; i < n_wrt; ++i)
        if (!s->nodes.count(wrt[i])) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "stream_grad: unknown wrt node");
    const int64_t numel = ln->second.meta.numel();
    if (numel != 1)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "grad requires scalar loss, got %lld elements", (long long)numel);
    MLXHIP_TRY(s->eval({loss}));

    const std::vector<uint64_t> order = s->topo_sort({loss});
    // need[x]: some wrt node is reachable from x (x depends on it).
    const std::unordered_set<uint64_t> targets(wrt, wrt + n_wrt);
    std::unordered_set<uint64_t> needs;
    for (uint64_t id : order) {  // inputs come before their consumers
        bool nd = targets.count(id) != 0;
        for (uint64_t in : s->nodes.at(id).inputs) nd = nd || needs.count(in);
        if (nd) needs.insert(id);
    }

    Builder b{*s};
    const MetaVal lm = ln->second.meta;
    const uint64_t seed = b.constant(std::vector<float>((size_t)numel, 1.0f), lm.shape, lm.dtype);
    if (!seed) return recorded_status();
    std::unordered_map<uint64_t, uint64_t> table;
    table[loss] = seed;
    std::unordered_map<uint64_t, uint64_t> done;  // gradients of source / wrt nodes
    std::vector<uint64_t> ig;
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        const uint64_t id = *it;
        auto gt = table.find(id);
        if (gt == table.end()) continue;
        const uint64_t g = gt->second;
        table.erase(gt);
        const Node n = s->nodes.at(id);  // copy: the builder may rehash `nodes`
        const int k = n.op.op.kind;
        if (targets.count(id)) done[id] = g;
        if (k == MLXHIP_OP_CONSTANT || k == MLXHIP_OP_PARAMETER) continue;
        std::vector<bool> need(n.inputs.size());
        bool any = false;
        for (size_t i = 0; i < n.inputs.size(); ++i) any |= (need[i] = needs.count(n.inputs[i]) != 0);
        if (!any) continue;
        MLXHIP_TRY(vjp(b, id, n, g, need, ig));
        for (size_t i = 0; i < n.inputs.size(); ++i) {
            if (!need[i]) continue;
            const uint64_t in = n.inputs[i];
            auto ex = table.find(in);
            if (ex == table.end()) {
                table[in] = ig[i];
            } else {
                const uint64_t sum = b.add(ex->second, ig[i]);
                if (!sum) return recorded_status();
                ex->second = sum;
            }
        }
    }
    for (size_t i = 0; i < n_wrt; ++i) {
        auto d = done.find(wrt[i]);
        if (d == done.end())
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gradient not found — input may not affect the loss");
        grads[i] = d->second;
    }
    return MLXHIP_OK;
}

}  // namespace

extern "C" int mlxhip_stream_grad(mlxhip_stream_t* s, uint64_t loss, const uint64_t* wrt, size_t n_wrt,
                                  uint64_t* grads) {
    if (!s || (n_wrt && (!wrt || !grads))) return fail(MLXHIP_ERR_NULL_PTR, "stream_grad: null argument");
    std::lock_guard<std::mutex> lock(s->mu);
    try {
        return stream_grad(s, loss, wrt, n_wrt, grads);
    } catch (const std::exception& e) {
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "stream_grad: %s", e.what());
    }
}
