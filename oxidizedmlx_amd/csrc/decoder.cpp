// decoder.cpp — greedy decoding of a decoder-only language model on one GPU:
// the token loop of crates/mlx-conformance/tests/ttft_behavior.rs:101-216
// (project the new token, append K/V to the cache, attend over the whole
// cache) for a stack of pre-norm transformer blocks built from mlx-nn layers
// (Embedding crates/mlx-nn/src/embed.rs, Linear linear.rs:34-43, RmsNorm
// norm.rs:43-67, attention as in attention.rs:47-111, SiLU MLP), with the
// reference's host-side KV vectors and host argmax moved into HBM.
//
// Everything the loop touches stays on the device: bf16 weights (one
// allocation), the f32 KV cache of every layer, the residual stream, the
// token history and a step counter t. One step is 5 launches per layer plus
// the LM head and a finishing launch (argmax, next token's embedding, t += 1);
// every launch reads t from the counter, so the step is captured once as a
// HIP graph and replayed for every position.
// Prompt tokens are consumed one position per step (the cached attention of
// position t over 0..t is the causal attention of the full prompt row t).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "backend.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace mlxhip;

constexpr int N_LAYER_PARAMS = 12;  // MLXHIP_DEC_WQ .. MLXHIP_DEC_B2

uint16_t bf16_rne_host(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;  // NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

size_t align_elems(size_t n) { return (n + 127) & ~size_t(127); }  // 256-byte alignment of bf16 arrays

}  // namespace

struct mlxhip_decoder_t {
    mlxhip_decoder_config_t cfg{};
    int device = 0;
    int head_dim = 0;
    float scale = 0.0f;
    std::mutex mu;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    float last_ms = -1.0f;
    int last_steps = 0;

    // bf16 parameters (element offsets into `w`)
    uint16_t* w = nullptr;
    size_t w_elems = 0;
    size_t off_emb = 0, off_lm = 0;
    std::vector<size_t> off_layer;  // per layer: wqkv, bqkv, wo, bo, w1, b1, w2, b2 (8 entries)
    std::vector<uint8_t> set;       // which parameters were loaded

    // activations and state: the residual stream x (f32 and its bf16
    // planes xs), q, and the planes of the attention output (os) and of the
    // SiLU output (us); planes are [3][DEC_MAX_BATCH][width]
    float *x = nullptr, *q = nullptr;
    uint16_t *xs = nullptr, *os = nullptr, *us = nullptr;
    float *kc = nullptr, *vc = nullptr;  // [L][max_batch][H][hd][max_seq], [L][max_batch][H][max_seq][hd]
    int* tokens = nullptr;               // [(max_seq + 1)][batch]
    int* argmax = nullptr;               // [max_seq][batch]
    int* tctr = nullptr;
    uint64_t* part = nullptr;
    int part_capacity = 0;

    float* logits = nullptr;             // [batch][steps][vocab], grown on demand
    size_t logits_cap = 0;

    // Instantiated step graphs by shape, most recent last.
    struct StepGraph {
        int batch, prompt_len, logit_steps;  // logit_steps = 0: no logits written
        hipGraph_t graph;
        hipGraphExec_t exec;
    };
    std::vector<StepGraph> graphs;
    static constexpr size_t MAX_GRAPHS = 8;

    void drop_graphs() {
        for (auto& g : graphs) {
            (void)hipGraphExecDestroy(g.exec);
            (void)hipGraphDestroy(g.graph);
        }
        graphs.clear();
    }

    ~mlxhip_decoder_t() {
        (void)hipSetDevice(device);
        if (stream) (void)hipStreamSynchronize(stream);
        drop_graphs();
        for (void* p : {(void*)w, (void*)x, (void*)q, (void*)xs, (void*)os, (void*)us, (void*)kc, (void*)vc, (void*)tokens,
                        (void*)argmax, (void*)tctr, (void*)part, (void*)logits})
            if (p) (void)hipFree(p);
        if (ev0) (void)hipEventDestroy(ev0);
        if (ev1) (void)hipEventDestroy(ev1);
        if (stream) (void)hipStreamDestroy(stream);
    }

    const uint16_t* lw(int l, int i) const { return w + off_layer[(size_t)l * 8 + i]; }

    size_t param_index(int layer, int which) const {
        if (which == MLXHIP_DEC_EMBEDDING) return 0;
        if (which == MLXHIP_DEC_LM_HEAD) return 1;
        return 2 + (size_t)layer * N_LAYER_PARAMS + (which - MLXHIP_DEC_WQ);
    }

    // Enqueues one decode step (position t read from tctr; x holds the
    // embedding of token t) on `s`. It ends with the argmax, the next token's
    // embedding in x and t += 1.
    int enqueue_step(int batch, int prompt_len, bool want_logits, int steps_total, hipStream_t s) {
        const auto& c = cfg;
        const int d = c.d_model, H = c.n_heads, hd = head_dim;
        const size_t kv_layer = (size_t)c.max_batch * H * hd * c.max_seq;
        for (int l = 0; l < c.n_layers; ++l) {
            float* kcl = kc + (size_t)l * kv_layer;
            float* vcl = vc + (size_t)l * kv_layer;
            DecGemv g;
            g.batch = batch;
            g.eps = c.eps;
            g.tctr = tctr;
            // q | k | v = rms_norm(x) Wqkv^T + bqkv
            g.w = lw(l, 0); g.bias = lw(l, 1);
            g.xs = xs; g.ldxs = d; g.n = 3 * d; g.k = d;
            g.out = q; g.ldo = d;
            g.kc = kcl; g.vc = vcl; g.dmodel = d; g.heads = H; g.head_dim = hd; g.tmax = c.max_seq;
            MLXHIP_TRY(dec_gemv(DEC_EPI_QKV, true, g, s));
            MLXHIP_TRY(dec_attention(q, kcl, vcl, os, batch, H, hd, c.max_seq, scale, tctr, s));
            // x = x + (o Wo^T + bo)
            g = DecGemv();
            g.batch = batch; g.tctr = tctr;
            g.w = lw(l, 2); g.bias = lw(l, 3);
            g.xs = os; g.ldxs = d; g.n = d; g.k = d;
            g.out = x; g.ldo = d; g.outs = xs; g.ldos = d;
            MLXHIP_TRY(dec_gemv(DEC_EPI_RESID, false, g, s));
            // u = silu(rms_norm(x) W1^T + b1)
            g = DecGemv();
            g.batch = batch; g.tctr = tctr; g.eps = c.eps;
            g.w = lw(l, 4); g.bias = lw(l, 5);
            g.xs = xs; g.ldxs = d; g.n = c.hidden; g.k = d;
            g.outs = us; g.ldos = c.hidden;
            MLXHIP_TRY(dec_gemv(DEC_EPI_SILU, true, g, s));
            // x = x + (u W2^T + b2)
            g = DecGemv();
            g.batch = batch; g.tctr = tctr;
            g.w = lw(l, 6); g.bias = lw(l, 7);
            g.xs = us; g.ldxs = c.hidden; g.n = d; g.k = c.hidden;
            g.out = x; g.ldo = d; g.outs = xs; g.ldos = d;
            MLXHIP_TRY(dec_gemv(DEC_EPI_RESID, false, g, s));
        }
        // logits = rms_norm(x) Wlm^T, argmax per workgroup
        DecGemv g;
        g.batch = batch; g.tctr = tctr; g.eps = c.eps;
        g.w = w + off_lm;
        g.xs = xs; g.ldxs = d; g.n = c.vocab; g.k = d;
        g.out = want_logits ? logits : nullptr;
        g.ldo = (int64_t)steps_total * c.vocab;
        g.part = part; g.part_capacity = part_capacity;
        MLXHIP_TRY(dec_gemv(DEC_EPI_ARGMAX, true, g, s));
        return dec_finish(part, dec_gemv_groups(c.vocab, d), tokens, argmax, w + off_emb, x, xs, d, c.vocab, batch,
                          prompt_len, tctr, s);
    }

    // Position counter to 0, x = embedding of token 0.
    int enqueue_start(int batch, hipStream_t s) {
        MLXHIP_TRY(dec_set_counter(tctr, 0, s));
        return dec_embed(w + off_emb, tokens, x, xs, cfg.d_model, cfg.vocab, batch, tctr, s);
    }
};

namespace {

int validate_config(const mlxhip_decoder_config_t& c) {
    if (c.n_layers < 1 || c.d_model < 1 || c.n_heads < 1 || c.hidden < 1 || c.vocab < 1 || c.max_batch < 1 ||
        c.max_seq < 1)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: every size must be positive");
    if (c.max_batch > DEC_MAX_BATCH)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: max_batch %d exceeds %d", c.max_batch,
                    DEC_MAX_BATCH);
    if (c.d_model % c.n_heads)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: d_model %d is not a multiple of n_heads %d",
                    c.d_model, c.n_heads);
    const int hd = c.d_model / c.n_heads;
    if (256 % hd || hd < 8)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: head_dim %d must be 8, 16, 32, 64, 128 or 256",
                    hd);
    if (c.d_model % 32 || c.hidden % 32)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: d_model and hidden must be multiples of 32");
    // d_model feeds the RMS-normalising GEMVs (Q/K/V, up, LM head), whose
    // LDS holds the squares of the activation.
    if (dec_gemv_lds_bytes(c.d_model, 16, 1, true, true) > (size_t)DEC_LDS_LIMIT ||
        dec_gemv_lds_bytes(c.hidden, 16, 1, false, false) > (size_t)DEC_LDS_LIMIT)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: d_model %d / hidden %d exceed the GEMV's LDS staging",
                    c.d_model, c.hidden);
    if (dec_attn_lds_bytes(hd, c.max_seq) > 64 * 1024)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: max_seq %d too long", c.max_seq);
    if (!(c.eps >= 0.0f)) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder config: eps must be >= 0");
    return MLXHIP_OK;
}

template <class T>
int dev_alloc(T** p, size_t count) {
    if (forced_alloc_failure())
        return fail(MLXHIP_ERR_FFI_FAILED, "decoder: device allocation of %zu bytes failed (forced)",
                    std::max<size_t>(count, 1) * sizeof(T));
    MLXHIP_HIP(hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(count, 1) * sizeof(T)));
    return MLXHIP_OK;
}

int init_decoder(mlxhip_decoder_t* D) {
    const auto& c = D->cfg;
    MLXHIP_HIP(hipGetDevice(&D->device));
    MLXHIP_TRY(dec_prepare());
    MLXHIP_HIP(hipStreamCreateWithFlags(&D->stream, hipStreamNonBlocking));
    MLXHIP_HIP(hipEventCreate(&D->ev0));
    MLXHIP_HIP(hipEventCreate(&D->ev1));
    const size_t d = c.d_model, V = c.vocab, Hd = c.hidden;
    size_t off = 0;
    D->off_emb = off; off += align_elems(V * d);
    D->off_lm = off; off += align_elems((size_t)ceil_div(V, 16) * 16 * d);  // rows padded to the 16-row tile
    D->off_layer.resize((size_t)c.n_layers * 8);
    const size_t sizes[8] = {3 * d * d, 3 * d, d * d, d, Hd * d, Hd, d * Hd, d};
    for (int l = 0; l < c.n_layers; ++l)
        for (int i = 0; i < 8; ++i) {
            D->off_layer[(size_t)l * 8 + i] = off;
            off += align_elems(sizes[i]);
        }
    D->w_elems = off;
    D->set.assign(2 + (size_t)c.n_layers * N_LAYER_PARAMS, 0);
    MLXHIP_TRY(dev_alloc(&D->w, off));
    const size_t B = c.max_batch, S = c.max_seq, H = c.n_heads;
    MLXHIP_TRY(dev_alloc(&D->x, B * d));
    MLXHIP_TRY(dev_alloc(&D->q, B * d));
    // Planes are allocated for DEC_MAX_BATCH rows (the GEMV's MFMA reads all
    // of them; rows of absent sequences only feed discarded columns) and
    // cleared, so every row holds finite values.
    const size_t planes = 3 * (size_t)DEC_MAX_BATCH;
    MLXHIP_TRY(dev_alloc(&D->xs, planes * d));
    MLXHIP_TRY(dev_alloc(&D->os, planes * d));
    MLXHIP_TRY(dev_alloc(&D->us, planes * Hd));
    MLXHIP_HIP(hipMemsetAsync(D->xs, 0, planes * d * 2, D->stream));
    MLXHIP_HIP(hipMemsetAsync(D->os, 0, planes * d * 2, D->stream));
    MLXHIP_HIP(hipMemsetAsync(D->us, 0, planes * Hd * 2, D->stream));
    const size_t kv = (size_t)c.n_layers * B * H * D->head_dim * S;
    MLXHIP_TRY(dev_alloc(&D->kc, kv));
    MLXHIP_TRY(dev_alloc(&D->vc, kv));
    MLXHIP_TRY(dev_alloc(&D->tokens, (S + 1) * B));
    MLXHIP_TRY(dev_alloc(&D->argmax, S * B));
    MLXHIP_TRY(dev_alloc(&D->tctr, 1));
    D->part_capacity = dec_gemv_groups(c.vocab, c.d_model);
    MLXHIP_TRY(dev_alloc(&D->part, (size_t)D->part_capacity * DEC_MAX_BATCH));
    // The cache is read only at positions already written; clear it anyway so
    // no uninitialised memory is ever read.
    MLXHIP_HIP(hipMemsetAsync(D->kc, 0, kv * sizeof(float), D->stream));
    MLXHIP_HIP(hipMemsetAsync(D->vc, 0, kv * sizeof(float), D->stream));
    MLXHIP_HIP(hipStreamSynchronize(D->stream));
    return MLXHIP_OK;
}

// The instantiated graph of one step for this shape (captured on first use).
int step_graph(mlxhip_decoder_t* D, int batch, int prompt_len, int steps, bool want_logits, hipGraphExec_t* out) {
    const int ls = want_logits ? steps : 0;
    auto& G = D->graphs;
    for (size_t i = 0; i < G.size(); ++i)
        if (G[i].batch == batch && G[i].prompt_len == prompt_len && G[i].logit_steps == ls) {
            std::rotate(G.begin() + i, G.begin() + i + 1, G.end());
            *out = G.back().exec;
            return MLXHIP_OK;
        }
    hipStream_t s = D->stream;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    MLXHIP_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int rc = D->enqueue_step(batch, prompt_len, want_logits, steps, s);
    const hipError_t ec = hipStreamEndCapture(s, &graph);
    if (rc != MLXHIP_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (ec != hipSuccess) return hip_fail(ec, "hipStreamEndCapture");
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(ei, "hipGraphInstantiate");
    }
    if (G.size() == mlxhip_decoder_t::MAX_GRAPHS) {
        (void)hipGraphExecDestroy(G.front().exec);
        (void)hipGraphDestroy(G.front().graph);
        G.erase(G.begin());
    }
    G.push_back({batch, prompt_len, ls, graph, exec});
    *out = exec;
    return MLXHIP_OK;
}

int run_steps(mlxhip_decoder_t* D, int batch, int prompt_len, int steps, bool want_logits, bool eager) {
    hipStream_t s = D->stream;
    if (eager) {
        MLXHIP_HIP(hipEventRecord(D->ev0, s));
        MLXHIP_TRY(D->enqueue_start(batch, s));
        for (int t = 0; t < steps; ++t) MLXHIP_TRY(D->enqueue_step(batch, prompt_len, want_logits, steps, s));
        MLXHIP_HIP(hipEventRecord(D->ev1, s));
        return MLXHIP_OK;
    }
    hipGraphExec_t exec = nullptr;
    MLXHIP_TRY(step_graph(D, batch, prompt_len, steps, want_logits, &exec));
    MLXHIP_HIP(hipEventRecord(D->ev0, s));
    MLXHIP_TRY(D->enqueue_start(batch, s));
    for (int t = 0; t < steps; ++t) MLXHIP_HIP(hipGraphLaunch(exec, s));
    MLXHIP_HIP(hipEventRecord(D->ev1, s));
    return MLXHIP_OK;
}

}  // namespace

extern "C" {

mlxhip_decoder_t* mlxhip_decoder_new(const mlxhip_decoder_config_t* cfg) {
    if (!cfg) {
        fail(MLXHIP_ERR_NULL_PTR, "decoder_new: null config");
        return nullptr;
    }
    if (validate_config(*cfg) != MLXHIP_OK) return nullptr;
    if (ensure_device() != MLXHIP_OK) return nullptr;
    auto* D = new mlxhip_decoder_t();
    D->cfg = *cfg;
    D->head_dim = cfg->d_model / cfg->n_heads;
    D->scale = (float)(1.0 / std::sqrt((double)D->head_dim));
    const int rc = init_decoder(D);
    if (rc != MLXHIP_OK) {
        std::string msg = last_error();
        delete D;
        fail(rc, "decoder_new: %s", msg.c_str());
        return nullptr;
    }
    return D;
}

void mlxhip_decoder_free(mlxhip_decoder_t* dec) { delete dec; }

int mlxhip_decoder_set_param(mlxhip_decoder_t* D, int32_t layer, int32_t which, const float* values, size_t len) {
    if (!D || (!values && len)) return fail(MLXHIP_ERR_NULL_PTR, "decoder_set_param: null argument");
    const auto& c = D->cfg;
    const size_t d = c.d_model, V = c.vocab, Hd = c.hidden;
    size_t want = 0, off = 0;
    switch (which) {
        case MLXHIP_DEC_EMBEDDING: want = V * d; off = D->off_emb; break;
        case MLXHIP_DEC_LM_HEAD: want = V * d; off = D->off_lm; break;
        default: {
            if (which < MLXHIP_DEC_WQ || which > MLXHIP_DEC_B2)
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_set_param: unknown parameter %d", which);
            if (layer < 0 || layer >= c.n_layers)
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_set_param: layer %d out of range [0, %d)", layer,
                            c.n_layers);
            const size_t L = (size_t)layer * 8;
            switch (which) {
                case MLXHIP_DEC_WQ: want = d * d; off = D->off_layer[L + 0]; break;
                case MLXHIP_DEC_WK: want = d * d; off = D->off_layer[L + 0] + d * d; break;
                case MLXHIP_DEC_WV: want = d * d; off = D->off_layer[L + 0] + 2 * d * d; break;
                case MLXHIP_DEC_BQ: want = d; off = D->off_layer[L + 1]; break;
                case MLXHIP_DEC_BK: want = d; off = D->off_layer[L + 1] + d; break;
                case MLXHIP_DEC_BV: want = d; off = D->off_layer[L + 1] + 2 * d; break;
                case MLXHIP_DEC_WO: want = d * d; off = D->off_layer[L + 2]; break;
                case MLXHIP_DEC_BO: want = d; off = D->off_layer[L + 3]; break;
                case MLXHIP_DEC_W1: want = Hd * d; off = D->off_layer[L + 4]; break;
                case MLXHIP_DEC_B1: want = Hd; off = D->off_layer[L + 5]; break;
                case MLXHIP_DEC_W2: want = d * Hd; off = D->off_layer[L + 6]; break;
                case MLXHIP_DEC_B2: want = d; off = D->off_layer[L + 7]; break;
            }
        }
    }
    if (len != want)
        return fail_shape({(int64_t)want}, {(int64_t)len}, "decoder_set_param");
    // GEMV weights go in the GEMV's fragment order (the LM head's rows padded
    // with zeros to whole 16-row tiles); the embedding and biases stay plain.
    size_t cols = 0;
    switch (which) {
        case MLXHIP_DEC_LM_HEAD: case MLXHIP_DEC_WQ: case MLXHIP_DEC_WK: case MLXHIP_DEC_WV: case MLXHIP_DEC_WO:
        case MLXHIP_DEC_W1: cols = d; break;
        case MLXHIP_DEC_W2: cols = Hd; break;
        default: break;
    }
    std::vector<uint16_t> h;
    if (cols) {
        const size_t rows = len / cols;
        h.assign((size_t)ceil_div((int64_t)rows, 16) * 16 * cols, 0);
        for (size_t n = 0; n < rows; ++n)
            for (size_t k = 0; k < cols; ++k) h[dec_tiled_index(n, k, cols)] = bf16_rne_host(values[n * cols + k]);
    } else {
        h.resize(len);
        for (size_t i = 0; i < len; ++i) h[i] = bf16_rne_host(values[i]);
    }
    std::lock_guard<std::mutex> g(D->mu);
    MLXHIP_HIP(hipSetDevice(D->device));
    MLXHIP_HIP(hipMemcpyAsync(D->w + off, h.data(), h.size() * 2, hipMemcpyHostToDevice, D->stream));
    MLXHIP_HIP(hipStreamSynchronize(D->stream));
    D->set[D->param_index(layer, which)] = 1;
    return MLXHIP_OK;
}

int mlxhip_decoder_generate(mlxhip_decoder_t* D, const int32_t* prompt, int32_t batch, int32_t prompt_len,
                            int32_t n_new, int32_t* tokens_out, int32_t* argmax_out, float* logits_out,
                            int32_t flags) {
    if (!D || !prompt || !tokens_out) return fail(MLXHIP_ERR_NULL_PTR, "decoder_generate: null argument");
    const auto& c = D->cfg;
    if (batch < 1 || batch > c.max_batch)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_generate: batch %d outside [1, %d]", batch, c.max_batch);
    if (prompt_len < 1 || n_new < 1)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_generate: prompt_len and n_new must be >= 1");
    const int64_t steps = (int64_t)prompt_len + n_new - 1;
    if (steps > c.max_seq)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_generate: %lld positions exceed max_seq %d",
                    (long long)steps, c.max_seq);
    if (flags & ~MLXHIP_DEC_EAGER) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_generate: unknown flags");
    std::lock_guard<std::mutex> g(D->mu);
    for (size_t i = 0; i < D->set.size(); ++i)
        if (!D->set[i]) {
            const int layer = i < 2 ? -1 : (int)((i - 2) / N_LAYER_PARAMS);
            const int which = i < 2 ? (int)i : MLXHIP_DEC_WQ + (int)((i - 2) % N_LAYER_PARAMS);
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_generate: parameter %d of layer %d was never set",
                        which, layer);
        }
    MLXHIP_HIP(hipSetDevice(D->device));
    hipStream_t s = D->stream;
    // Token history [t][b]: rows 0..prompt_len-1 hold the prompt.
    std::vector<int32_t> tok((size_t)prompt_len * batch);
    for (int b = 0; b < batch; ++b)
        for (int t = 0; t < prompt_len; ++t) tok[(size_t)t * batch + b] = prompt[(size_t)b * prompt_len + t];
    MLXHIP_HIP(hipMemcpyAsync(D->tokens, tok.data(), tok.size() * 4, hipMemcpyHostToDevice, s));
    const bool want_logits = logits_out != nullptr;
    if (want_logits) {
        const size_t need = (size_t)batch * steps * c.vocab;
        if (need > D->logits_cap) {
            MLXHIP_HIP(hipStreamSynchronize(s));
            D->drop_graphs();  // captured graphs hold the old logits address
            if (D->logits) MLXHIP_HIP(hipFree(D->logits));
            D->logits = nullptr;
            D->logits_cap = 0;
            MLXHIP_TRY(dev_alloc(&D->logits, need));
            D->logits_cap = need;
        }
    }
    MLXHIP_TRY(run_steps(D, batch, prompt_len, (int)steps, want_logits, (flags & MLXHIP_DEC_EAGER) != 0));
    MLXHIP_HIP(hipStreamSynchronize(s));
    float ms = 0.0f;
    MLXHIP_HIP(hipEventElapsedTime(&ms, D->ev0, D->ev1));
    D->last_ms = ms;
    D->last_steps = (int)steps;
    std::vector<int32_t> am((size_t)steps * batch);
    MLXHIP_HIP(hipMemcpy(am.data(), D->argmax, am.size() * 4, hipMemcpyDeviceToHost));
    for (int b = 0; b < batch; ++b) {
        for (int i = 0; i < n_new; ++i) tokens_out[(size_t)b * n_new + i] = am[(size_t)(prompt_len - 1 + i) * batch + b];
        if (argmax_out)
            for (int t = 0; t < steps; ++t) argmax_out[(size_t)b * steps + t] = am[(size_t)t * batch + b];
    }
    if (want_logits)
        MLXHIP_HIP(hipMemcpy(logits_out, D->logits, (size_t)batch * steps * c.vocab * sizeof(float),
                             hipMemcpyDeviceToHost));
    return MLXHIP_OK;
}

int mlxhip_decoder_last_timing(const mlxhip_decoder_t* D, float* ms, int32_t* steps) {
    if (!D || !ms || !steps) return fail(MLXHIP_ERR_NULL_PTR, "decoder_last_timing: null argument");
    if (D->last_ms < 0.0f) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "decoder_last_timing: nothing generated yet");
    *ms = D->last_ms;
    *steps = D->last_steps;
    return MLXHIP_OK;
}

size_t mlxhip_decoder_weight_bytes(const mlxhip_decoder_t* D) { return D ? D->w_elems * 2 : 0; }

}  // extern "C"
