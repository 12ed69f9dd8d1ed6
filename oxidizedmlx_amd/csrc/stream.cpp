// stream.cpp — Stream and Graph bound to HipBackend, with every buffer
// resident in HBM.
//
// Restates Stream (crates/mlx-core/src/backend.rs:37-185) and Graph
// (crates/mlx-core/src/graph.rs:170-305, CSE rules :495-515):
//   * add_constant never deduplicates (Constant/Parameter are not CSE
//     eligible) and materialises the data at once;
//   * add_op interns with CSE on (op, inputs, meta), Add/Mul inputs ordered
//     by node id first;
//   * eval topologically sorts the subgraph of the output and evaluates each
//     unmaterialised node once; results are memoised until the stream is freed.
// Differences, all below the Backend seam: buffers live in HBM (host copies
// only in get_buffer), and with fusion enabled the scheduler looks ahead:
//   * a chain of elementwise nodes whose intermediates have exactly one
//     consumer runs as one ew_chain kernel (intermediates are not
//     materialised; they are recomputed if asked for later);
//   * a rank-2 Transpose whose only consumer is a MatMul is not
//     materialised; the GEMM reads its source with the transposed layout.
// eval_count counts every node a backend call covered, so fused and unfused
// evaluation report the same count.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "backend.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "stream.hpp"

namespace mlxhip {
namespace {

bool is_elementwise(int k) {
    switch (k) {
        case MLXHIP_OP_ADD: case MLXHIP_OP_SUB: case MLXHIP_OP_MUL: case MLXHIP_OP_DIV:
        case MLXHIP_OP_NEG: case MLXHIP_OP_EXP: case MLXHIP_OP_LOG: case MLXHIP_OP_SQRT:
        case MLXHIP_OP_SILU: case MLXHIP_OP_GELU: case MLXHIP_OP_SILU_VJP: case MLXHIP_OP_GELU_VJP:
            return true;
        default: return false;
    }
}

bool is_binary(int k) {
    return k == MLXHIP_OP_ADD || k == MLXHIP_OP_SUB || k == MLXHIP_OP_MUL || k == MLXHIP_OP_DIV ||
           k == MLXHIP_OP_SILU_VJP || k == MLXHIP_OP_GELU_VJP;
}

int unary_ew(int k) {
    switch (k) {
        case MLXHIP_OP_NEG: return MLXHIP_EW_NEG;
        case MLXHIP_OP_EXP: return MLXHIP_EW_EXP;
        case MLXHIP_OP_LOG: return MLXHIP_EW_LOG;
        case MLXHIP_OP_SQRT: return MLXHIP_EW_SQRT;
        case MLXHIP_OP_SILU: return MLXHIP_EW_SILU;
        default: return MLXHIP_EW_GELU;
    }
}

// Chain instruction when the running value (acc) is input `acc_idx` of a
// binary node and the other input is the operand.
int binary_ew(int k, int acc_idx) {
    switch (k) {
        case MLXHIP_OP_ADD: return MLXHIP_EW_ADD;
        case MLXHIP_OP_MUL: return MLXHIP_EW_MUL;
        case MLXHIP_OP_SUB: return acc_idx == 0 ? MLXHIP_EW_SUB : MLXHIP_EW_RSUB;
        case MLXHIP_OP_DIV: return acc_idx == 0 ? MLXHIP_EW_DIV : MLXHIP_EW_RDIV;
        case MLXHIP_OP_SILU_VJP: return MLXHIP_EW_SILU_VJP;  // acc = x (input 1), operand = dy
        default: return MLXHIP_EW_GELU_VJP;
    }
}

}  // namespace
}  // namespace mlxhip

using namespace mlxhip;

namespace mlxhip {
namespace {

// A Transpose node that swaps the two matrix axes: [1,0] (or None) on rank
// 2, [0,2,1] on rank 3 (the batched operand of a rank-3 MatMul).
bool is_matrix_swap(const Node& t) {
    if (t.op.op.kind != MLXHIP_OP_TRANSPOSE) return false;
    const size_t nd = t.meta.shape.size();
    const std::vector<int64_t>& a = t.op.axes;
    if (nd == 2) return !t.op.has_axes || (a.size() == 2 && a[0] == 1 && a[1] == 0);
    return nd == 3 && t.op.has_axes && a.size() == 3 && a[0] == 0 && a[1] == 2 && a[2] == 1;
}

// A Transpose [B, S, H, dh] <-> [B, H, S, dh] (axes 0, 2, 1, 3): the split or
// merge of attention heads.
bool is_head_swap(const Node& t) {
    const std::vector<int64_t>& a = t.op.axes;
    return t.op.op.kind == MLXHIP_OP_TRANSPOSE && t.meta.shape.size() == 4 && t.op.has_axes && a.size() == 4 &&
           a[0] == 0 && a[1] == 2 && a[2] == 1 && a[3] == 3;
}

// Period P when broadcasting `src` to `dst` only repeats src: after padding
// src with leading 1s, src = [1,...,1, dst[j:]] for some j, so
// out[i] = src[i % P] with P = numel(dst[j:]). 0 when it is no such tiling.
int64_t tiling_period(const std::vector<int64_t>& src, const std::vector<int64_t>& dst) {
    if (src.size() > dst.size()) return 0;
    const size_t pad = dst.size() - src.size();
    std::vector<int64_t> s(pad, 1);
    s.insert(s.end(), src.begin(), src.end());
    for (size_t j = 0; j <= dst.size(); ++j) {
        bool ok = true;
        for (size_t i = 0; i < j && ok; ++i) ok = s[i] == 1;
        for (size_t i = j; i < dst.size() && ok; ++i) ok = s[i] == dst[i];
        if (ok) {
            int64_t p = 1;
            for (size_t i = j; i < dst.size(); ++i) p *= dst[i];
            return p;
        }
    }
    return 0;
}

}  // namespace
}  // namespace mlxhip

int mlxhip_stream_t::eval(const std::vector<uint64_t>& outputs) {
    std::vector<uint64_t> todo;
    for (uint64_t o : outputs) {
        if (!nodes.count(o)) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "missing graph node");
        if (!buffers.count(o)) todo.push_back(o);
    }
    if (todo.empty()) return MLXHIP_OK;
    const std::vector<uint64_t> order = topo_sort(todo, true);
    std::unordered_set<uint64_t> in_order(order.begin(), order.end());
    // Requested outputs are always materialised: never a chain interior or a
    // folded Transpose.
    const std::unordered_set<uint64_t> requested(todo.begin(), todo.end());

    // ── look-ahead planning ──────────────────────────────────────────────
    std::unordered_set<uint64_t> folded_transpose;                  // not materialised
    std::unordered_set<uint64_t> swapped_matmul;                    // Transpose computed as B^T A^T
    std::unordered_set<uint64_t> absorbed_matmul;                   // MatMul inside such a Transpose
    std::unordered_map<uint64_t, std::vector<uint64_t>> chain_of;   // chain end -> nodes
    std::unordered_map<uint64_t, int> acc_input;                    // node -> index of its acc input
    std::unordered_set<uint64_t> interior;                          // fused, not materialised
    // Broadcasts that only tile their source and whose every consumer in this
    // evaluation is elementwise: the chain kernel reads the source
    // periodically and the broadcast is not materialised. (A consumer already
    // evaluated needs nothing more; one evaluated later finds no buffer and
    // plans the broadcast again.)
    std::unordered_map<uint64_t, int64_t> virtual_bcast;            // node -> period (elements)
    // A rank-2 f32 MatMul whose one consumer is the Add of a bias row
    // broadcast over its rows (a linear layer): the product adds the bias as
    // it stores C, into the Add's buffer; neither the MatMul nor the Add is
    // evaluated on its own.
    struct BiasTerm {
        uint64_t add;   // the Add node, whose buffer the product writes
        uint64_t bcast; // the (virtual) Broadcast of the bias
        uint64_t src;   // the bias, [N] values
    };
    std::unordered_map<uint64_t, BiasTerm> bias_of;  // MatMul -> its bias Add
    // Heads of attention without the permutes. A [B*H, S, dh] operand that is
    // Reshape(Transpose{0,2,1,3}(Reshape [B, S, H, dh] (src))) and is read
    // only by batched MatMuls is read from src in place (head h of batch b at
    // src + (b S H + h) dh, rows H dh apart) by the thin kernels; a batched
    // product whose only reader is the reverse chain, Reshape [B, H, S, dh],
    // Transpose{0,2,1,3}, Reshape (the head merge), writes the merged layout
    // directly. The Transposes (and the views) are not materialised. When
    // the product does not fit the thin kernels after all, the permutes run
    // as before (head_materialise below).
    struct HeadView {
        uint64_t src;         // split: the [B*S, H*dh] source; merge: the merged node
        int64_t B, S, H, dh;
        uint64_t t, r;        // the Transpose and the inner Reshape
    };
    std::unordered_map<uint64_t, HeadView> head_in;   // split view node -> where its data lives
    std::unordered_map<uint64_t, HeadView> head_out;  // product -> the merge it writes
    std::unordered_set<uint64_t> head_skip;           // Transposes and inner Reshapes of both
    // MLXHIP_HEAD_VIEWS=0: the permutes always run (for comparisons).
    const bool head_views_on = !(getenv("MLXHIP_HEAD_VIEWS") && !strcmp(getenv("MLXHIP_HEAD_VIEWS"), "0"));
    if (fusion) {
        std::unordered_map<uint64_t, std::vector<uint64_t>> users;
        for (uint64_t id : order)
            for (uint64_t in : nodes.at(id).inputs) users[in].push_back(id);
        for (uint64_t id : order) {
            if (buffers.count(id) || requested.count(id)) continue;
            const Node& n = nodes.at(id);
            if (n.op.op.kind != MLXHIP_OP_BROADCAST || n.inputs.size() != 1) continue;
            const int64_t per = tiling_period(nodes.at(n.inputs[0]).meta.shape, n.meta.shape);
            if (per <= 0 || per != nodes.at(n.inputs[0]).meta.numel()) continue;
            const std::vector<uint64_t>& u = users[id];
            if (u.empty()) continue;
            bool ok = true;
            for (uint64_t c : u) {
                const Node& cn = nodes.at(c);
                const int ck = cn.op.op.kind;
                ok = ok && is_elementwise(ck) && !buffers.count(c) && cn.meta.numel() == n.meta.numel() &&
                     cn.inputs.size() == (is_binary(ck) ? 2u : 1u);
                for (uint64_t ci : cn.inputs) ok = ok && nodes.at(ci).meta.numel() == cn.meta.numel();
            }
            if (ok) virtual_bcast[id] = per;
        }

        // A Transpose that swaps the two matrix axes ([1,0] on rank 2,
        // [0,2,1] on rank 3) and is read only by MatMuls, directly or through
        // further such Transposes, is not materialised: each MatMul reads the
        // untransposed source with the transposed operand layout. Consumers
        // come later in the order, so walk it backwards.
        for (auto it = order.rbegin(); it != order.rend(); ++it) {
            const uint64_t id = *it;
            if (buffers.count(id) || requested.count(id)) continue;
            const Node& t = nodes.at(id);
            if (!is_matrix_swap(t) || t.inputs.empty()) continue;
            // Consumers outside this evaluation either hold their buffers
            // already or will plan this Transpose again when they run.
            const std::vector<uint64_t>& u = users[id];
            if (u.empty()) continue;
            bool ok = true;
            for (uint64_t c : u) {
                if (buffers.count(c) || folded_transpose.count(c)) continue;
                const Node& cn = nodes.at(c);
                ok = ok && cn.op.op.kind == MLXHIP_OP_MATMUL && cn.inputs.size() == 2 && cn.inputs[0] != cn.inputs[1];
            }
            if (ok) folded_transpose.insert(id);
        }
        // A materialised matrix-swap Transpose of a MatMul that nothing else
        // reads is computed as one product with swapped operands,
        // (A B)^T = B^T A^T; the MatMul itself is not materialised.
        for (uint64_t id : order) {
            if (buffers.count(id) || folded_transpose.count(id)) continue;
            const Node& t = nodes.at(id);
            if (!is_matrix_swap(t) || t.inputs.size() != 1) continue;
            const uint64_t m = t.inputs[0];
            auto mn = nodes.find(m);
            if (mn == nodes.end() || mn->second.op.op.kind != MLXHIP_OP_MATMUL || mn->second.inputs.size() != 2 ||
                mn->second.inputs[0] == mn->second.inputs[1] || buffers.count(m) || requested.count(m) ||
                consumers[m] != 1 || mn->second.meta.dtype != MLXHIP_DTYPE_F32)
                continue;
            swapped_matmul.insert(id);
            absorbed_matmul.insert(m);
        }
        if (head_views_on) {
            auto fresh = [&](uint64_t id) { return in_order.count(id) && !buffers.count(id) && !requested.count(id); };
            // Split views: every reader a rank-3 f32 MatMul (directly or
            // through folded matrix-swap Transposes).
            for (uint64_t id : order) {
                const Node& x = nodes.at(id);
                if (!fresh(id) || x.op.op.kind != MLXHIP_OP_RESHAPE || x.inputs.size() != 1 || x.meta.shape.size() != 3 ||
                    x.meta.dtype != MLXHIP_DTYPE_F32)
                    continue;
                const uint64_t t = x.inputs[0];
                const Node& tn = nodes.at(t);
                if (!fresh(t) || !is_head_swap(tn) || tn.inputs.size() != 1 || consumers[t] != 1) continue;
                const uint64_t r = tn.inputs[0];
                const Node& rn = nodes.at(r);
                if (rn.op.op.kind != MLXHIP_OP_RESHAPE || rn.inputs.size() != 1 || rn.meta.shape.size() != 4) continue;
                const std::vector<int64_t>& rs = rn.meta.shape;  // [B, S, H, dh]
                const std::vector<int64_t>& xs = x.meta.shape;   // [B*H, S, dh]
                if (xs[0] != rs[0] * rs[2] || xs[1] != rs[1] || xs[2] != rs[3] ||
                    nodes.at(rn.inputs[0]).meta.numel() != rn.meta.numel())
                    continue;
                const std::vector<uint64_t>& u = users[id];
                bool ok = !u.empty();
                for (uint64_t c : u) {
                    if (folded_transpose.count(c)) continue;
                    const Node& cn = nodes.at(c);
                    ok = ok && cn.op.op.kind == MLXHIP_OP_MATMUL && cn.inputs.size() == 2 && cn.inputs[0] != cn.inputs[1] &&
                         cn.meta.shape.size() == 3 && cn.meta.dtype == MLXHIP_DTYPE_F32;
                }
                if (!ok) continue;
                head_in[id] = HeadView{rn.inputs[0], rs[0], rs[1], rs[2], rs[3], t, r};
                head_skip.insert(t);
                if (consumers[r] == 1 && fresh(r)) head_skip.insert(r);
            }
            // Merges: a rank-3 f32 product (or a Transpose computed as one)
            // whose only reader is Reshape [B, H, S, dh], whose only reader is
            // the head swap, whose only reader is a Reshape.
            for (uint64_t id : order) {
                const Node& p = nodes.at(id);
                const bool prod = (p.op.op.kind == MLXHIP_OP_MATMUL && !absorbed_matmul.count(id)) || swapped_matmul.count(id);
                if (!prod || !fresh(id) || folded_transpose.count(id) || bias_of.count(id) || p.meta.shape.size() != 3 ||
                    p.meta.dtype != MLXHIP_DTYPE_F32 || consumers[id] != 1 || users[id].size() != 1)
                    continue;
                const uint64_t r1 = users[id][0];
                const Node& r1n = nodes.at(r1);
                if (!fresh(r1) || r1n.op.op.kind != MLXHIP_OP_RESHAPE || r1n.meta.shape.size() != 4 || consumers[r1] != 1 ||
                    users[r1].size() != 1)
                    continue;
                const std::vector<int64_t>& ps = p.meta.shape, &q = r1n.meta.shape;  // [B*H, S, dh], [B, H, S, dh]
                if (ps[0] != q[0] * q[1] || ps[1] != q[2] || ps[2] != q[3]) continue;
                const uint64_t t = users[r1][0];
                const Node& tn = nodes.at(t);
                if (!fresh(t) || !is_head_swap(tn) || consumers[t] != 1 || users[t].size() != 1) continue;
                const uint64_t r2 = users[t][0];
                const Node& r2n = nodes.at(r2);
                if (!in_order.count(r2) || buffers.count(r2) || r2n.op.op.kind != MLXHIP_OP_RESHAPE ||
                    r2n.meta.numel() != tn.meta.numel())
                    continue;
                head_out[id] = HeadView{r2, q[0], q[2], q[1], q[3], t, r1};
                head_skip.insert(t);
                head_skip.insert(r1);
            }
        }
        for (uint64_t id : order) {
            if (buffers.count(id) || folded_transpose.count(id)) continue;
            const Node& n = nodes.at(id);
            const int k = n.op.op.kind;
            if (!is_elementwise(k)) continue;
            const size_t need = is_binary(k) ? 2 : 1;
            if (n.inputs.size() < need) continue;  // let eval report the error
            if (is_binary(k)) {
                const int64_t l0 = nodes.at(n.inputs[0]).meta.numel(), l1 = nodes.at(n.inputs[1]).meta.numel();
                if (l0 != l1 || l0 != n.meta.numel()) continue;
            } else if (nodes.at(n.inputs[0]).meta.numel() != n.meta.numel()) {
                continue;
            }
            // Candidate acc inputs: the running value of the chain.
            std::vector<int> cand;
            if (k == MLXHIP_OP_SILU_VJP || k == MLXHIP_OP_GELU_VJP) cand = {1};
            else if (is_binary(k)) cand = {0, 1};
            else cand = {0};
            int chosen = -1;
            for (int c : cand) {
                const uint64_t in = n.inputs[c];
                if (is_binary(k) && n.inputs[0] == n.inputs[1]) break;  // x op x: keep both operands materialised
                if (!in_order.count(in) || buffers.count(in) || folded_transpose.count(in) || requested.count(in))
                    continue;
                auto ch = chain_of.find(in);
                if (ch == chain_of.end() || consumers[in] != 1) continue;
                // Limits of one ew_chain launch: instructions and distinct inputs.
                if (ch->second.size() + 1 > MLXHIP_EW_MAX_INSTR) continue;
                std::unordered_set<uint64_t> ins;
                for (uint64_t m : ch->second) {
                    const Node& mn = nodes.at(m);
                    if (m == ch->second.front()) ins.insert(mn.inputs[acc_input[m]]);
                    if (is_binary(mn.op.op.kind)) ins.insert(mn.inputs[1 - acc_input[m]]);
                }
                if (is_binary(k)) ins.insert(n.inputs[1 - c]);
                if (ins.size() > MLXHIP_EW_MAX_INPUTS) continue;
                chosen = c;
                break;
            }
            if (chosen >= 0) {
                const uint64_t prev = n.inputs[chosen];
                std::vector<uint64_t> ch = std::move(chain_of[prev]);
                chain_of.erase(prev);
                interior.insert(prev);
                ch.push_back(id);
                acc_input[id] = chosen;
                chain_of[id] = std::move(ch);
            } else {
                acc_input[id] = cand[0];
                chain_of[id] = {id};
            }
        }
    }

    // A chain that is a single Add of a MatMul and a virtual row broadcast
    // whose source already has its buffer becomes the MatMul's bias term.
    for (auto it = chain_of.begin(); fusion && it != chain_of.end();) {
        const uint64_t aid = it->first;
        const Node& an = nodes.at(aid);
        bool taken = false;
        if (it->second.size() == 1 && an.op.op.kind == MLXHIP_OP_ADD && an.inputs.size() == 2 &&
            an.inputs[0] != an.inputs[1] && an.meta.dtype == MLXHIP_DTYPE_F32 && an.meta.shape.size() == 2) {
            for (int c = 0; c < 2 && !taken; ++c) {
                const uint64_t mid = an.inputs[c], vid = an.inputs[1 - c];
                const Node& mn = nodes.at(mid);
                auto v = virtual_bcast.find(vid);
                if (mn.op.op.kind != MLXHIP_OP_MATMUL || mn.inputs.size() != 2 || mn.meta.dtype != MLXHIP_DTYPE_F32 ||
                    mn.meta.shape != an.meta.shape || !in_order.count(mid) || buffers.count(mid) ||
                    requested.count(mid) || consumers[mid] != 1 || absorbed_matmul.count(mid) || bias_of.count(mid) ||
                    v == virtual_bcast.end() || v->second != an.meta.shape[1])
                    continue;
                const uint64_t src = nodes.at(vid).inputs[0];
                if (!buffers.count(src) || nodes.at(src).meta.numel() != an.meta.shape[1]) continue;
                bias_of[mid] = BiasTerm{aid, vid, src};
                taken = true;
            }
        }
        if (taken) it = chain_of.erase(it);
        else ++it;
    }

    // ── evaluation ────────────────────────────────────────────────────────
    std::unordered_set<uint64_t> counted_virtual, counted_folded;  // eval_count covers each once
    Scratch scratch;
    scratch.planes = &planes;
    int rc = MLXHIP_OK;
    // Reshape keeps the data as it is (row-major, contiguous): the node
    // aliases its input's buffer, which lives as long as the stream. Narrow
    // along an axis with only size-1 axes before it takes a contiguous range
    // of its input: the node aliases that range (node buffers live until the
    // stream is cleared, like Reshape's). Sets node id's buffer and returns
    // true when id is such a node and its input has a buffer.
    auto alias = [&](uint64_t id) -> bool {
        const Node& n = nodes.at(id);
        if (n.inputs.size() != 1) return false;
        auto src = buffers.find(n.inputs[0]);
        if (src == buffers.end()) return false;
        if (n.op.op.kind == MLXHIP_OP_RESHAPE) {
            if ((int64_t)src->second.len != n.meta.numel()) return false;
            buffers[id] = DevBuf{src->second.ptr, src->second.len, false};
            return true;
        }
        if (n.op.op.kind != MLXHIP_OP_NARROW) return false;
        const std::vector<int64_t>& ish = nodes.at(n.inputs[0]).meta.shape;
        int64_t ax = n.op.op.axis;
        if (ax < 0) ax += (int64_t)ish.size();
        if (ax < 0 || ax >= (int64_t)ish.size()) return false;
        int64_t outer = 1, inner = 1;
        for (int64_t d = 0; d < ax; ++d) outer *= ish[d];
        for (int64_t d = ax + 1; d < (int64_t)ish.size(); ++d) inner *= ish[d];
        const int64_t st = n.op.op.start, ln = n.op.op.length;
        if (outer != 1 || st < 0 || ln < 0 || st + ln > ish[ax] || (int64_t)src->second.len != ish[ax] * inner ||
            ln * inner != n.meta.numel())
            return false;
        buffers[id] = DevBuf{src->second.ptr + st * inner, (size_t)(ln * inner), false};
        return true;
    };
    // Whether node id has a buffer, giving it one first if it is a chain of
    // aliases (above) over a node that has one (the sibling search's
    // operands: dQ/dK/dV are Narrow views of one gradient node).
    std::function<bool(uint64_t, int)> ready_alias = [&](uint64_t id, int depth) -> bool {
        if (buffers.count(id)) return true;
        if (depth > 8 || !in_order.count(id)) return false;
        const Node& n = nodes.at(id);
        if ((n.op.op.kind != MLXHIP_OP_RESHAPE && n.op.op.kind != MLXHIP_OP_NARROW) || n.inputs.size() != 1)
            return false;
        if (!ready_alias(n.inputs[0], depth + 1) || !alias(id)) return false;
        eval_calls += 1;
        return true;
    };
    // A MatMul operand's source node after folded Transposes, and how many
    // Transposes (mod 2) lie between: the GEMM reads the source with the
    // layout flipped that many times.
    auto resolve = [&](uint64_t src, int* hint) {
        while (folded_transpose.count(src)) {
            *hint ^= 1;
            src = nodes.at(src).inputs[0];
        }
        return src;
    };
    // The node whose buffer a MatMul's result goes to: its bias Add, if any.
    auto out_of = [&](uint64_t id) {
        auto b = bias_of.find(id);
        return b == bias_of.end() ? id : b->second.add;
    };
    // A bias term's share of eval_count: the Add, and its broadcast once.
    auto bias_covered = [&](uint64_t id) -> uint64_t {
        auto b = bias_of.find(id);
        if (b == bias_of.end()) return 0;
        return 1 + (counted_virtual.insert(b->second.bcast).second ? 1 : 0);
    };
    // Products waiting for their siblings (sibling grouping, below): their
    // operands, ready when they were reached, and their share of eval_count.
    struct Pending {
        uint64_t id;
        mlxhip_input_t in[2];
        int hint[2];
        bool swapped;
        uint64_t covered;
        size_t deadline;  // the first position that reads its result
    };
    std::vector<Pending> pending;
    std::unordered_map<uint64_t, size_t> pos;
    std::unordered_map<uint64_t, std::vector<uint64_t>> readers;
    for (size_t i = 0; i < order.size(); ++i) {
        pos[order[i]] = i;
        for (uint64_t in : nodes.at(order[i]).inputs) readers[in].push_back(order[i]);
    }
    // The first position of this evaluation at which a node reads id's buffer:
    // its readers, and through folded Transposes and Reshape / Narrow views
    // (which alias it), theirs.
    // Chains whose result an f32 product of this evaluation reads through
    // the split-f32 planes write those planes themselves (ew_chain_planes),
    // so that product skips the split of that operand: the stored operand
    // (the chain's result, or a Reshape of it) with rows and cols multiples
    // of 32. Value: the operand's stored rows, cols and batch.
    struct PlaneView {
        int64_t rows, cols, batch;
    };
    std::unordered_map<uint64_t, PlaneView> plane_out;
    if (fusion) {
        for (const auto& ce : chain_of) {
            const uint64_t cid = ce.first;
            const Node& cn = nodes.at(cid);
            if (cn.meta.dtype != MLXHIP_DTYPE_F32) continue;
            // Readers of cid, directly or through Reshape views and folded Transposes.
            std::vector<std::pair<uint64_t, uint64_t>> frontier{{cid, cid}};  // (reader, operand node as stored)
            bool found = false;
            for (size_t fi = 0; fi < frontier.size() && fi < 64 && !found; ++fi) {
                const uint64_t at = frontier[fi].first, stored = frontier[fi].second;
                auto rd = readers.find(at);
                if (rd == readers.end()) continue;
                for (uint64_t u : rd->second) {
                    const Node& un = nodes.at(u);
                    const int uk = un.op.op.kind;
                    if (folded_transpose.count(u)) {
                        frontier.push_back({u, stored});
                        continue;
                    }
                    if (uk == MLXHIP_OP_RESHAPE && un.meta.numel() == cn.meta.numel() && at == stored) {
                        frontier.push_back({u, u});
                        continue;
                    }
                    if (uk != MLXHIP_OP_MATMUL || un.inputs.size() != 2 || un.meta.dtype != MLXHIP_DTYPE_F32 ||
                        un.meta.shape.size() < 2 || buffers.count(u))
                        continue;
                    const std::vector<int64_t>& os = un.meta.shape;
                    const std::vector<int64_t>& as = nodes.at(un.inputs[0]).meta.shape;
                    const std::vector<int64_t>& ss = nodes.at(stored).meta.shape;
                    if (as.size() != os.size() || ss.size() != os.size() || (os.size() != 2 && os.size() != 3)) continue;
                    const int64_t batch = os.size() == 3 ? os[0] : 1;
                    const int64_t m = os[os.size() - 2], n = os[os.size() - 1], k = as[as.size() - 1];
                    const int64_t rows = ss[ss.size() - 2], cols = ss[ss.size() - 1];
                    if (!gemm_f32_reads_planes(m, n, k, batch) || rows % 32 || cols % 32) continue;
                    plane_out[cid] = PlaneView{rows, cols, batch};
                    found = true;
                    break;
                }
            }
        }
    }
    std::function<size_t(uint64_t, int)> first_read = [&](uint64_t id, int depth) -> size_t {
        size_t best = SIZE_MAX;
        auto it = readers.find(id);
        if (it == readers.end()) return best;
        for (uint64_t u : it->second) {
            best = std::min(best, pos.at(u));
            const int uk = nodes.at(u).op.op.kind;
            if (depth < 16 && (folded_transpose.count(u) || uk == MLXHIP_OP_RESHAPE || uk == MLXHIP_OP_NARROW))
                best = std::min(best, first_read(u, depth + 1));
        }
        return best;
    };
    // Head views (planned above). head_materialise: the split view x's
    // permute into the Transpose's buffer, x aliasing it. head_merge: the
    // merge of product id's buffer into the merged node's. The view's nodes
    // count in eval_count once per stream (a split view read by the loss and
    // again by the gradients is planned by both evaluations).
    auto head_count = [&](std::initializer_list<uint64_t> ids) {
        for (uint64_t h : ids)
            if (counted_views.insert(h).second) eval_calls += 1;
    };
    auto head_materialise = [&](uint64_t x, const HeadView& v) -> int {
        const Node& tn = nodes.at(v.t);
        const Node& rn = nodes.at(v.r);
        float* tb = nullptr;
        MLXHIP_TRY(alloc_out(v.t, &tb));
        const mlxhip_input_t in = {buffers.at(v.src).ptr, (size_t)rn.meta.numel(), rn.meta.shape.data(),
                                   rn.meta.shape.size(), rn.meta.dtype};
        const int r = eval_node_device(tn.op.c(), &in, 1, tn.meta.c(), tb, hs, scratch, nullptr);
        if (r != MLXHIP_OK) {
            release_later(tb);
            buffers.erase(v.t);
            return r;
        }
        buffers[x] = DevBuf{tb, (size_t)nodes.at(x).meta.numel(), false};
        launches += 1;
        head_count({v.t, x});
        if (head_skip.count(v.r)) head_count({v.r});
        return MLXHIP_OK;
    };
    auto head_merge = [&](uint64_t id, const HeadView& v) -> int {
        const Node& tn = nodes.at(v.t);
        const Node& r1n = nodes.at(v.r);
        float* ob = nullptr;
        MLXHIP_TRY(alloc_out(v.src, &ob));
        const mlxhip_input_t in = {buffers.at(id).ptr, (size_t)r1n.meta.numel(), r1n.meta.shape.data(),
                                   r1n.meta.shape.size(), r1n.meta.dtype};
        const int r = eval_node_device(tn.op.c(), &in, 1, tn.meta.c(), ob, hs, scratch, nullptr);
        if (r != MLXHIP_OK) {
            release_later(ob);
            buffers.erase(v.src);
            return r;
        }
        launches += 1;
        head_count({v.r, v.t, v.src});
        return MLXHIP_OK;
    };
    // A batched product with head views on the thin kernels: operands in
    // place, C into the merged node when it is a merge. *ran = false (and
    // nothing done) when the thin kernels do not take it.
    auto head_product = [&](uint64_t id, const mlxhip_input_t* ins, const int* hint, const uint64_t* msrc,
                            const HeadView* const* hv, const HeadView* ho, bool* ran) -> int {
        *ran = false;
        if (ins[0].ndim != 3 || ins[1].ndim != 3) return MLXHIP_OK;
        // Common head count and batch: every view's must agree.
        int64_t H = 0, B = 0;
        for (const HeadView* v : {hv[0], hv[1], ho}) {
            if (!v) continue;
            if (H && (v->H != H || v->B != B)) return MLXHIP_OK;
            H = v->H, B = v->B;
        }
        const int64_t G = ins[0].shape[0];
        if (ins[1].shape[0] != G || G != B * H || H > INT32_MAX) return MLXHIP_OK;
        ThinView op[2];
        for (int j = 0; j < 2; ++j) {
            const int64_t R = ins[j].shape[1], C = ins[j].shape[2];
            if (hv[j]) {
                const HeadView& v = *hv[j];
                op[j] = ThinView{buffers.at(v.src).ptr, v.H * v.dh, v.S * v.H * v.dh, v.dh};
            } else {
                op[j] = ThinView{ins[j].data, C, H * R * C, R * C};
            }
        }
        const int ta = hint[0], tb = hint[1];
        const int64_t m = ta ? ins[0].shape[2] : ins[0].shape[1], k = ta ? ins[0].shape[1] : ins[0].shape[2];
        const int64_t n = tb ? ins[1].shape[1] : ins[1].shape[2];
        if (ho && (m != ho->S || n != ho->dh)) return MLXHIP_OK;
        // C's placement is known before it exists: 256-byte-aligned pool blocks.
        const float* probe = reinterpret_cast<const float*>(uintptr_t(256));
        ThinView cv = ho ? ThinView{probe, H * n, m * H * n, n} : ThinView{probe, n, H * m * n, m * n};
        if (!gemm_thin_view_fits(ta, tb, m, n, k, G, (int)H, op[0], op[1], cv)) return MLXHIP_OK;
        float* out = nullptr;
        const uint64_t dst = ho ? ho->src : id;
        MLXHIP_TRY(alloc_out(dst, &out));
        cv.p = out;
        if (!gemm_thin_view_fits(ta, tb, m, n, k, G, (int)H, op[0], op[1], cv)) {
            // Not the placement the pool gives (256-byte blocks): run as before.
            release_later(out);
            buffers.erase(dst);
            return MLXHIP_OK;
        }
        const int r = gemm_thin_view(ta, tb, m, n, k, G, (int)H, op[0], op[1], cv, hs);
        if (r != MLXHIP_OK) {
            release_later(out);
            buffers.erase(dst);
            return r;
        }
        for (int j = 0; j < 2; ++j)
            if (hv[j]) {
                head_count({hv[j]->t, msrc[j]});
                if (head_skip.count(hv[j]->r)) head_count({hv[j]->r});
            }
        if (ho) head_count({ho->r, ho->t, ho->src});
        *ran = true;
        return MLXHIP_OK;
    };
    for (size_t oi = 0; oi < order.size(); ++oi) {
        const uint64_t id = order[oi];
        if (buffers.count(id) || folded_transpose.count(id) || interior.count(id) || virtual_bcast.count(id) ||
            absorbed_matmul.count(id) || buffers.count(out_of(id)) ||  // a product already run with its bias term
            head_skip.count(id) || head_in.count(id))                  // head views: read or written in place
            continue;
        const Node& n = nodes.at(id);
        auto ch = chain_of.find(id);
        auto reads_virtual = [&](const std::vector<uint64_t>& chain) {
            for (uint64_t m : chain)
                for (uint64_t in : nodes.at(m).inputs)
                    if (virtual_bcast.count(in)) return true;
            return false;
        };
        auto pv = plane_out.find(id);
        if (ch != chain_of.end() && (ch->second.size() > 1 || reads_virtual(ch->second) || pv != plane_out.end())) {
            // One fused kernel for the whole chain.
            const std::vector<uint64_t>& nodes_in_chain = ch->second;
            std::vector<const float*> ins;
            std::vector<int64_t> periods;
            std::vector<uint64_t> in_ids;
            auto ready = [&](uint64_t src) {
                auto v = virtual_bcast.find(src);
                return buffers.count(v != virtual_bcast.end() ? nodes.at(src).inputs[0] : src) != 0;
            };
            auto slot = [&](uint64_t src) -> int {
                for (size_t i = 0; i < in_ids.size(); ++i)
                    if (in_ids[i] == src) return (int)i;
                in_ids.push_back(src);
                auto v = virtual_bcast.find(src);
                if (v != virtual_bcast.end()) {
                    ins.push_back(buffers.at(nodes.at(src).inputs[0]).ptr);
                    periods.push_back(v->second);
                } else {
                    ins.push_back(buffers.at(src).ptr);
                    periods.push_back(0);
                }
                return (int)in_ids.size() - 1;
            };
            for (uint64_t m : nodes_in_chain)
                for (uint64_t in : nodes.at(m).inputs)
                    if (virtual_bcast.count(in) && counted_virtual.insert(in).second) eval_calls += 1;
            const Node& first = nodes.at(nodes_in_chain.front());
            const uint64_t base = first.inputs[acc_input[nodes_in_chain.front()]];
            if (!ready(base)) { rc = fail(MLXHIP_ERR_INVALID_ARGUMENT, "fusion: base not materialised"); break; }
            slot(base);
            std::vector<mlxhip_ew_instr_t> prog;
            for (uint64_t m : nodes_in_chain) {
                const Node& mn = nodes.at(m);
                const int k = mn.op.op.kind;
                if (is_binary(k)) {
                    const int ai = acc_input[m];
                    const uint64_t other = mn.inputs[1 - ai];
                    if (!ready(other)) { rc = fail(MLXHIP_ERR_INVALID_ARGUMENT, "fusion: operand not materialised"); break; }
                    prog.push_back({binary_ew(k, ai), slot(other)});
                } else {
                    prog.push_back({unary_ew(k), 0});
                }
            }
            if (rc != MLXHIP_OK) break;
            float* out = nullptr;
            if ((rc = alloc_out(id, &out)) != MLXHIP_OK) break;
            uint16_t* pl = nullptr;
            uint32_t* fl = nullptr;
            uint32_t gen = 0;
            if (pv != plane_out.end() &&
                (rc = x6_plane_block(&planes, out, pv->second.rows, pv->second.cols, pv->second.batch, &pl, &fl,
                                     &gen)) != MLXHIP_OK)
                break;
            bool written = false;
            rc = ew_chain_planes(prog.data(), (int)prog.size(), ins.data(), periods.data(), (int)ins.size(), out,
                                 n.meta.numel(), pl, fl, gen, &written, hs);
            if (pl && !written) planes.entries.pop_back();  // the product splits it after all
            eval_calls += nodes_in_chain.size();
            launches += 1;
            if (rc != MLXHIP_OK) {
                release_later(out);
                buffers.erase(id);
                break;
            }
            continue;
        }
        if (alias(id)) {
            eval_calls += 1;
            continue;
        }
        // Single node through HipBackend::eval_node. A MatMul operand that is
        // a folded Transpose (or a chain of them) is read from the source
        // with the operand layout flipped once per Transpose; a swapped
        // Transpose runs its MatMul as B^T A^T.
        std::vector<mlxhip_input_t> ins;
        int hint[2] = {0, 0};
        uint64_t msrc[2] = {0, 0};  // a MatMul's resolved operand sources
        const HeadView* hv[2] = {nullptr, nullptr};  // operands that are head-split views
        bool missing = false;
        const bool swapped = swapped_matmul.count(id) != 0;
        const Node& en = swapped ? nodes.at(n.inputs[0]) : n;  // the node whose op runs
        uint64_t covered = 1 + (swapped ? 1 : 0);
        for (size_t j = 0; j < en.inputs.size(); ++j) {
            const size_t i = swapped ? 1 - j : j;  // swapped: operands exchange places
            uint64_t src = en.inputs[i];
            if (en.op.op.kind == MLXHIP_OP_MATMUL && j < 2) {
                hint[j] = swapped ? 1 : 0;
                while (folded_transpose.count(src)) {
                    if (counted_folded.insert(src).second) covered += 1;
                    hint[j] ^= 1;
                    src = nodes.at(src).inputs[0];
                }
            }
            if (j < 2) msrc[j] = src;
            auto b = buffers.find(src);
            if (b == buffers.end() && en.op.op.kind == MLXHIP_OP_MATMUL && j < 2 && head_in.count(src) &&
                ready_alias(head_in.at(src).src, 0)) {
                hv[j] = &head_in.at(src);
                ins.push_back(input_of(src, nullptr));  // read in place, or materialised below
                continue;
            }
            if (b == buffers.end()) { missing = true; break; }
            ins.push_back(input_of(src, b->second.ptr));
        }
        if (missing) { rc = fail(MLXHIP_ERR_INVALID_ARGUMENT, "input node should be evaluated before dependents"); break; }
        auto ho = head_out.find(id);
        if (hv[0] || hv[1] || ho != head_out.end()) {
            bool ran = false;
            if ((rc = head_product(id, ins.data(), hint, msrc, hv, ho == head_out.end() ? nullptr : &ho->second, &ran)) !=
                MLXHIP_OK)
                break;
            if (ran) {
                eval_calls += covered;
                launches += 1;
                continue;
            }
            // Not for the thin kernels: the split views' permutes run now, the
            // merge's after the product (below).
            for (int j = 0; j < 2 && rc == MLXHIP_OK; ++j)
                if (hv[j]) {
                    rc = head_materialise(msrc[j], *hv[j]);
                    if (rc == MLXHIP_OK) ins[j] = input_of(msrc[j], buffers.at(msrc[j]).ptr);
                }
            if (rc != MLXHIP_OK) break;
        }
        // Sibling products: later MatMuls of this evaluation with operands of
        // the same shapes and layouts, both ready, run with this one in one
        // grouped launch (the Q/K/V projections of one input; the three
        // products of their input gradient). They get their buffers now, and
        // the loop skips them when it reaches them.
        // A swapped product (a Transpose computed as B^T A^T, every weight
        // gradient) groups with other swapped products, its operands taken
        // in the swapped order. A product whose siblings' operands are not
        // ready yet waits for them (pending) when nothing reads its result
        // before the last of them: the weight gradients of Q, K and V, whose
        // dQ/dK/dV come out of separate kernels.
        std::vector<uint64_t> sib;
        std::vector<mlxhip_input_t> gin;  // 2 per product after this one
        std::vector<size_t> pend;         // pending products that join this launch
        if (fusion && en.op.op.kind == MLXHIP_OP_MATMUL && ins.size() == 2 && ins[0].ndim == 2 &&
            ins[1].ndim == 2 && n.meta.dtype == MLXHIP_DTYPE_F32) {
            const int64_t m = hint[0] ? ins[0].shape[1] : ins[0].shape[0], k = hint[0] ? ins[0].shape[0] : ins[0].shape[1];
            const int64_t nn = hint[1] ? ins[1].shape[0] : ins[1].shape[1];
            const bool groupable = gemm_f32_groupable(m, nn, k);
            auto same_operands = [&](const mlxhip_input_t* o) {
                for (int j = 0; j < 2; ++j)
                    if (o[j].ndim != 2 || o[j].shape[0] != ins[j].shape[0] || o[j].shape[1] != ins[j].shape[1])
                        return false;
                return true;
            };
            for (size_t i = 0; groupable && i < pending.size() && pend.size() < 3; ++i) {
                const Pending& pm = pending[i];
                if (pm.swapped == swapped && pm.hint[0] == hint[0] && pm.hint[1] == hint[1] &&
                    nodes.at(pm.id).meta.shape == n.meta.shape && same_operands(pm.in) &&
                    bias_of.count(pm.id) == bias_of.count(id))
                    pend.push_back(i);
            }
            bool waiting = false;  // a later sibling whose operands are not ready
            size_t last = oi;      // the position of the last later sibling
            for (size_t oj = oi + 1; groupable && oj < order.size(); ++oj) {
                const uint64_t cid = order[oj];
                if (buffers.count(cid) || folded_transpose.count(cid) || absorbed_matmul.count(cid) ||
                    (swapped_matmul.count(cid) != 0) != swapped || bias_of.count(cid) != bias_of.count(id) ||
                    buffers.count(out_of(cid)))
                    continue;
                const Node& cn = nodes.at(cid);
                const Node& ce = swapped ? nodes.at(cn.inputs[0]) : cn;  // the node whose op runs
                if (ce.op.op.kind != MLXHIP_OP_MATMUL || ce.inputs.size() != 2 || cn.meta.dtype != MLXHIP_DTYPE_F32 ||
                    cn.meta.shape != n.meta.shape)
                    continue;
                int ch[2] = {swapped ? 1 : 0, swapped ? 1 : 0};
                const uint64_t cs[2] = {resolve(ce.inputs[swapped ? 1 : 0], &ch[0]),
                                        resolve(ce.inputs[swapped ? 0 : 1], &ch[1])};
                if (ch[0] != hint[0] || ch[1] != hint[1] || nodes.at(cs[0]).meta.shape != nodes.at(msrc[0]).meta.shape ||
                    nodes.at(cs[1]).meta.shape != nodes.at(msrc[1]).meta.shape)
                    continue;
                if (cs[0] == msrc[0] && cs[1] == msrc[1]) continue;  // the same product
                last = oj;
                if (!ready_alias(cs[0], 0) || !ready_alias(cs[1], 0)) {
                    waiting = true;
                    continue;
                }
                if (pend.size() + sib.size() < 3) {
                    sib.push_back(cid);
                    gin.push_back(input_of(cs[0], buffers.at(cs[0]).ptr));
                    gin.push_back(input_of(cs[1], buffers.at(cs[1]).ptr));
                }
            }
            // Waiting holds back the pending products it would join too.
            bool can_wait = waiting && pend.size() + sib.size() < 3;
            for (size_t i : pend) can_wait = can_wait && pending[i].deadline > last;
            const size_t deadline = can_wait ? first_read(id, 0) : 0;
            if (can_wait && deadline > last) {
                pending.push_back(Pending{id, {ins[0], ins[1]}, {hint[0], hint[1]}, swapped, covered, deadline});
                continue;
            }
        }
        if (!sib.empty() || !pend.empty()) {
            // Products: the pending ones, this one, the later ready ones.
            std::vector<uint64_t> ids;
            std::vector<mlxhip_input_t> all;
            for (size_t i : pend) {
                ids.push_back(pending[i].id);
                all.push_back(pending[i].in[0]);
                all.push_back(pending[i].in[1]);
                covered += pending[i].covered;
            }
            ids.push_back(id);
            all.push_back(ins[0]);
            all.push_back(ins[1]);
            ids.insert(ids.end(), sib.begin(), sib.end());
            all.insert(all.end(), gin.begin(), gin.end());
            for (size_t j = pend.size(); j-- > 0;) pending.erase(pending.begin() + (std::ptrdiff_t)pend[j]);
            std::vector<float*> outs(ids.size(), nullptr);
            for (size_t i = 0; i < ids.size() && rc == MLXHIP_OK; ++i) rc = alloc_out(out_of(ids[i]), &outs[i]);
            std::vector<int> hints;
            for (size_t i = 0; i < outs.size(); ++i) hints.insert(hints.end(), {hint[0], hint[1]});
            std::vector<const float*> biases;
            if (bias_of.count(id))
                for (uint64_t g : ids) {
                    biases.push_back(buffers.at(bias_of.at(g).src).ptr);
                    covered += bias_covered(g);
                }
            if (rc == MLXHIP_OK)
                rc = eval_matmul_group((int)outs.size(), all.data(), hints.data(), outs.data(), hs, scratch,
                                       biases.empty() ? nullptr : biases.data());
            if (rc != MLXHIP_OK) {
                for (uint64_t g : ids) {
                    auto b = buffers.find(out_of(g));
                    if (b != buffers.end()) {
                        release_later(b->second.ptr);
                        buffers.erase(b);
                    }
                }
                break;
            }
            for (uint64_t g : sib) {
                covered += swapped ? 2 : 1;
                for (uint64_t src : nodes.at(swapped ? nodes.at(g).inputs[0] : g).inputs)
                    while (folded_transpose.count(src)) {
                        if (counted_folded.insert(src).second) covered += 1;
                        src = nodes.at(src).inputs[0];
                    }
            }
            eval_calls += covered;
            launches += 1;
            continue;
        }
        if (bias_of.count(id)) {
            // The product and its bias term, into the Add's buffer.
            const BiasTerm& bt = bias_of.at(id);
            float* out = nullptr;
            if ((rc = alloc_out(bt.add, &out)) != MLXHIP_OK) break;
            eval_calls += covered + bias_covered(id);
            launches += 1;
            rc = eval_matmul_bias(ins.data(), n.meta.c(), out, hs, scratch, hint, buffers.at(bt.src).ptr);
            if (rc != MLXHIP_OK) {
                release_later(out);
                buffers.erase(bt.add);
                break;
            }
            continue;
        }
        float* out = nullptr;
        if ((rc = alloc_out(id, &out)) != MLXHIP_OK) break;
        const mlxhip_op_t op = en.op.c();
        const mlxhip_meta_t meta = n.meta.c();
        eval_calls += covered;
        launches += 1;
        // A leaf axis reduction over a long axis runs on the side queue
        // (MLXHIP_SIDE_QUEUE=0: on the stream's own queue, for comparisons).
        hipStream_t q = hs;
        const int kind = en.op.op.kind;
        static const bool side_ok = !(getenv("MLXHIP_SIDE_QUEUE") && !strcmp(getenv("MLXHIP_SIDE_QUEUE"), "0"));
        if (side_ok && (kind == MLXHIP_OP_SUM || kind == MLXHIP_OP_MEAN || kind == MLXHIP_OP_MAX) && en.op.op.has_axis &&
            !swapped && consumers[id] == 0 && ins.size() == 1 && ins[0].ndim >= 1) {
            int64_t ax = en.op.op.axis;
            if (ax < 0) ax += (int64_t)ins[0].ndim;
            if (ax >= 0 && ax < (int64_t)ins[0].ndim && ins[0].shape[ax] >= 512 && (rc = fork_side(&q)) != MLXHIP_OK)
                break;
        }
        rc = eval_node_device(op, ins.data(), ins.size(), meta, out, q, scratch, hint);
        if (rc != MLXHIP_OK) {
            release_later(out);
            buffers.erase(id);
            break;
        }
        if (ho != head_out.end() && (rc = head_merge(id, ho->second)) != MLXHIP_OK) break;
    }
    // A product still pending (its siblings failed to come) runs alone.
    for (size_t i = 0; rc == MLXHIP_OK && i < pending.size(); ++i) {
        const Pending& pm = pending[i];
        const Node& pn = nodes.at(pm.id);
        const Node& pe = pm.swapped ? nodes.at(pn.inputs[0]) : pn;
        float* out = nullptr;
        if ((rc = alloc_out(out_of(pm.id), &out)) != MLXHIP_OK) break;
        const mlxhip_op_t op = pe.op.c();
        const mlxhip_meta_t meta = pn.meta.c();
        if (bias_of.count(pm.id))
            rc = eval_matmul_bias(pm.in, meta, out, hs, scratch, pm.hint, buffers.at(bias_of.at(pm.id).src).ptr);
        else
            rc = eval_node_device(op, pm.in, 2, meta, out, hs, scratch, pm.hint);
        eval_calls += pm.covered + bias_covered(pm.id);
        launches += 1;
        if (rc != MLXHIP_OK) {
            release_later(out);
            buffers.erase(out_of(pm.id));
        }
    }
    {
        const int jr = join_side();
        if (rc == MLXHIP_OK) rc = jr;
    }
    // Scratch may only return to the pool after the kernels using it finish.
    if (async_eval) {
        for (void* p : scratch.blocks) release_later(p);
        scratch.blocks.clear();
        return rc;
    }
    hipError_t e = hipStreamSynchronize(hs);
    if (rc == MLXHIP_OK && e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    return rc;
}

extern "C" {

mlxhip_stream_t* mlxhip_stream_new(void) {
    if (ensure_device() != MLXHIP_OK) return nullptr;
    auto* s = new mlxhip_stream_t();
    (void)hipGetDevice(&s->device);
    if (hipStreamCreateWithFlags(&s->hs, hipStreamNonBlocking) != hipSuccess) {
        fail(MLXHIP_ERR_FFI_FAILED, "hipStreamCreate failed");
        delete s;
        return nullptr;
    }
    return s;
}

void mlxhip_stream_free(mlxhip_stream_t* s) { delete s; }

static MetaVal meta_from(const mlxhip_meta_t* m) {
    MetaVal v;
    if (m->ndim) v.shape.assign(m->shape, m->shape + m->ndim);
    v.dtype = m->dtype;
    return v;
}

static uint64_t add_constant(mlxhip_stream_t* s, const float* data, size_t len, const mlxhip_meta_t* meta,
                             bool device_src) {
    if (!s || !meta || (len && !data)) {
        fail(MLXHIP_ERR_NULL_PTR, "stream_add_constant: null argument");
        return 0;
    }
    if (meta->ndim && !meta->shape) {
        fail(MLXHIP_ERR_NULL_PTR, "stream_add_constant: null shape");
        return 0;
    }
    std::lock_guard<std::mutex> g(s->mu);
    if (hipSetDevice(s->device) != hipSuccess) {
        fail(MLXHIP_ERR_FFI_FAILED, "stream_add_constant: hipSetDevice failed");
        return 0;
    }
    uint64_t id = 0;
    if (s->add_constant(data, len, meta_from(meta), device_src, &id) != MLXHIP_OK) return 0;
    return id;
}

uint64_t mlxhip_stream_add_constant(mlxhip_stream_t* s, const float* data, size_t len, const mlxhip_meta_t* meta) {
    return add_constant(s, data, len, meta, false);
}

uint64_t mlxhip_stream_add_constant_view(mlxhip_stream_t* s, const float* data, size_t len,
                                         const mlxhip_meta_t* meta) {
    if (!s || !meta || (len && !data)) {
        fail(MLXHIP_ERR_NULL_PTR, "stream_add_constant_view: null argument");
        return 0;
    }
    if (meta->ndim && !meta->shape) {
        fail(MLXHIP_ERR_NULL_PTR, "stream_add_constant_view: null shape");
        return 0;
    }
    std::lock_guard<std::mutex> g(s->mu);
    uint64_t id = 0;
    if (s->add_constant_view(data, len, meta_from(meta), &id) != MLXHIP_OK) return 0;
    return id;
}

uint64_t mlxhip_stream_add_constant_dev(mlxhip_stream_t* s, const float* data, size_t len,
                                        const mlxhip_meta_t* meta) {
    return add_constant(s, data, len, meta, true);
}

uint64_t mlxhip_stream_add_op(mlxhip_stream_t* s, const mlxhip_op_t* op, const uint64_t* inputs, size_t n_inputs,
                              const mlxhip_meta_t* meta) {
    if (!s || !op || !meta || (n_inputs && !inputs) || (meta->ndim && !meta->shape)) {
        fail(MLXHIP_ERR_NULL_PTR, "stream_add_op: null argument");
        return 0;
    }
    std::lock_guard<std::mutex> g(s->mu);
    for (size_t i = 0; i < n_inputs; ++i)
        if (!s->nodes.count(inputs[i])) {
            fail(MLXHIP_ERR_INVALID_ARGUMENT, "stream_add_op: unknown input node %llu", (unsigned long long)inputs[i]);
            return 0;
        }
    const bool cse_ok = op->kind != MLXHIP_OP_CONSTANT && op->kind != MLXHIP_OP_PARAMETER;
    return s->add_node(OpVal::from(*op), std::vector<uint64_t>(inputs, inputs + n_inputs), meta_from(meta), cse_ok);
}

int mlxhip_stream_eval(mlxhip_stream_t* s, uint64_t node) {
    if (!s) return fail(MLXHIP_ERR_NULL_PTR, "stream_eval: null stream");
    std::lock_guard<std::mutex> g(s->mu);
    MLXHIP_HIP(hipSetDevice(s->device));
    return s->eval({node});
}

int mlxhip_stream_eval_many(mlxhip_stream_t* s, const uint64_t* nodes, size_t n) {
    if (!s || (n && !nodes)) return fail(MLXHIP_ERR_NULL_PTR, "stream_eval_many: null argument");
    std::lock_guard<std::mutex> g(s->mu);
    MLXHIP_HIP(hipSetDevice(s->device));
    return s->eval(std::vector<uint64_t>(nodes, nodes + n));
}

int mlxhip_stream_get_buffer(mlxhip_stream_t* s, uint64_t node, float* out, size_t len) {
    if (!s || (len && !out)) return fail(MLXHIP_ERR_NULL_PTR, "stream_get_buffer: null argument");
    std::lock_guard<std::mutex> g(s->mu);
    auto it = s->buffers.find(node);
    if (it == s->buffers.end()) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "stream_get_buffer: node not materialised");
    if (len != it->second.len)
        return fail_shape({(int64_t)it->second.len}, {(int64_t)len}, "stream_get_buffer");
    if (!len) return MLXHIP_OK;
    MLXHIP_HIP(hipSetDevice(s->device));
    MLXHIP_HIP(hipMemcpyAsync(out, it->second.ptr, len * sizeof(float), hipMemcpyDeviceToHost, s->hs));
    return s->drain();
}

uint64_t mlxhip_stream_eval_count(const mlxhip_stream_t* s) { return s ? s->eval_calls.load() : 0; }

size_t mlxhip_stream_cache_len(const mlxhip_stream_t* s) {
    if (!s) return 0;
    auto* m = const_cast<mlxhip_stream_t*>(s);
    std::lock_guard<std::mutex> g(m->mu);
    return m->buffers.size();
}

uint64_t mlxhip_stream_launch_count(const mlxhip_stream_t* s) { return s ? s->launches.load() : 0; }

int mlxhip_stream_set_async(mlxhip_stream_t* s, int enabled) {
    if (!s) return fail(MLXHIP_ERR_NULL_PTR, "stream_set_async: null stream");
    std::lock_guard<std::mutex> g(s->mu);
    MLXHIP_HIP(hipSetDevice(s->device));
    if (!enabled && s->async_eval) MLXHIP_TRY(s->drain());
    s->async_eval = enabled != 0;
    return MLXHIP_OK;
}

int mlxhip_stream_clear(mlxhip_stream_t* s) {
    if (!s) return fail(MLXHIP_ERR_NULL_PTR, "stream_clear: null stream");
    std::lock_guard<std::mutex> g(s->mu);
    MLXHIP_HIP(hipSetDevice(s->device));
    return s->clear();
}

int mlxhip_stream_synchronize(mlxhip_stream_t* s) {
    if (!s) return fail(MLXHIP_ERR_NULL_PTR, "stream_synchronize: null stream");
    std::lock_guard<std::mutex> g(s->mu);
    MLXHIP_HIP(hipSetDevice(s->device));
    return s->drain();
}

int mlxhip_stream_set_fusion(mlxhip_stream_t* s, int enabled) {
    if (!s) return fail(MLXHIP_ERR_NULL_PTR, "stream_set_fusion: null stream");
    std::lock_guard<std::mutex> g(s->mu);
    s->fusion = enabled != 0;
    return MLXHIP_OK;
}

}  // extern "C"
