// backend.cpp — HipBackend::eval_node (the reference's Backend trait,
// crates/mlx-core/src/backend.rs:27-35) and the library-level C ABI: errors,
// devices, device buffers, the host-vector eval_node, direct kernel entry
// points and event timing.
//
// Op coverage and error behaviour follow CpuRefBackend::eval_node
// (crates/mlx-core/src/cpu_kernels.rs:13-102): the same validation errors
// (InvalidArgument / ShapeMismatch) for the same inputs, Constant/Parameter
// rejected, empty tensors return empty results.
#include "backend.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxhip {

// ── errors ────────────────────────────────────────────────────────────────

std::string& last_error() {
    static thread_local std::string msg;
    return msg;
}

static thread_local int t_last_status = MLXHIP_OK;
// expected / got of the last ShapeMismatch on this thread (cleared by every
// other failure).
static thread_local std::vector<int64_t> t_shape_expected, t_shape_got;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    last_error() = buf;
    t_last_status = code;
    t_shape_expected.clear();
    t_shape_got.clear();
    return code;
}

namespace {
std::string dims_str(const std::vector<int64_t>& d) {
    std::string r = "[";
    for (size_t i = 0; i < d.size(); ++i) r += (i ? ", " : "") + std::to_string(d[i]);
    return r + "]";
}
}  // namespace

int fail_shape(std::vector<int64_t> expected, std::vector<int64_t> got, const char* context) {
    fail(MLXHIP_ERR_SHAPE_MISMATCH, "%s%sShape mismatch: expected %s, got %s", context ? context : "",
         context ? ": " : "", dims_str(expected).c_str(), dims_str(got).c_str());
    t_shape_expected = std::move(expected);
    t_shape_got = std::move(got);
    return MLXHIP_ERR_SHAPE_MISMATCH;
}

int hip_fail(hipError_t e, const char* what) {
    // A failed runtime call also sets the thread's last error, which the next
    // launch check would report again for an unrelated kernel: consume it.
    (void)hipGetLastError();
    return fail(MLXHIP_ERR_FFI_FAILED, "%s failed: %s", what, hipGetErrorString(e));
}

// ── devices ───────────────────────────────────────────────────────────────

namespace {
int g_device_count = -1;
std::once_flag g_count_once;
thread_local int t_device = -1;

int device_count() {
    std::call_once(g_count_once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        g_device_count = n;
    });
    return g_device_count;
}
}  // namespace

int ensure_device() {
    if (t_device >= 0) return MLXHIP_OK;
    if (device_count() <= 0) return fail(MLXHIP_ERR_BACKEND_UNAVAILABLE, "mlx-hip: no HIP device available");
    MLXHIP_HIP(hipSetDevice(0));
    t_device = 0;
    return MLXHIP_OK;
}

namespace {
// The calling thread's own stream per device, destroyed when the thread ends
// (every call that uses it synchronises before returning, so no work is
// pending then).
struct ThreadStreams {
    hipStream_t s[64] = {};
    ~ThreadStreams() {
        int cur = 0;
        (void)hipGetDevice(&cur);
        for (int d = 0; d < 64; ++d)
            if (s[d]) {
                (void)hipSetDevice(d);
                if (hipStreamSynchronize(s[d]) == hipSuccess) release_stream_workspaces(s[d]);
                (void)hipStreamDestroy(s[d]);
            }
        (void)hipSetDevice(cur);
        (void)hipGetLastError();
    }
};
}  // namespace

hipStream_t thread_stream() {
    static thread_local ThreadStreams ts;
    const int dev = t_device < 0 ? 0 : t_device;
    if (!ts.s[dev]) {
        if (hipStreamCreateWithFlags(&ts.s[dev], hipStreamNonBlocking) != hipSuccess) {
            (void)hipGetLastError();
            ts.s[dev] = nullptr;
        }
    }
    return ts.s[dev];
}

// ── device memory pool ────────────────────────────────────────────────────

namespace {
struct Pool {
    std::mutex mu;
    std::multimap<size_t, void*> free_blocks[64];    // per device, by size
    std::map<void*, std::pair<int, size_t>> owned;   // ptr -> (device, size)
};
Pool& pool() {
    static Pool* p = new Pool();  // never destroyed: outlives late frees at exit
    return *p;
}
size_t round_size(size_t b) {
    if (b < 256) return 256;
    if (b <= (1u << 20)) return (b + 255) & ~size_t(255);
    return (b + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);  // 1 MiB granules
}
}  // namespace

namespace {
// Successful device allocations left before every further one fails: -1 off,
// -2 not yet read from MLXHIP_FAIL_ALLOC_AFTER.
std::atomic<int64_t> g_alloc_budget{-2};
}  // namespace

bool forced_alloc_failure() {
    int64_t b = g_alloc_budget.load();
    if (b == -2) {
        const char* e = std::getenv("MLXHIP_FAIL_ALLOC_AFTER");
        int64_t v = -1;
        if (e && *e) {
            char* end = nullptr;
            const long long n = std::strtoll(e, &end, 10);
            if (end && *end == '\0' && n >= 0) v = n;
        }
        g_alloc_budget.compare_exchange_strong(b, v);
        b = g_alloc_budget.load();
    }
    while (b >= 0) {
        if (b == 0) return true;
        if (g_alloc_budget.compare_exchange_weak(b, b - 1)) return false;
    }
    return false;
}

void* pool_alloc(size_t bytes) {
    if (forced_alloc_failure()) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    const size_t sz = round_size(bytes);
    Pool& P = pool();
    {
        std::lock_guard<std::mutex> g(P.mu);
        auto& fl = P.free_blocks[dev];
        auto it = fl.lower_bound(sz);
        if (it != fl.end() && it->first <= sz + sz / 2) {
            void* p = it->second;
            fl.erase(it);
            return p;
        }
    }
    void* p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) {
        // A failed hipMalloc also sets the thread's last error, which the next
        // launch check would report for an unrelated kernel: consume it. Then
        // drop cached blocks of this device and retry once.
        (void)hipGetLastError();
        std::vector<void*> drop;
        {
            std::lock_guard<std::mutex> g(P.mu);
            for (auto& kv : P.free_blocks[dev]) drop.push_back(kv.second);
            P.free_blocks[dev].clear();
            for (void* q : drop) P.owned.erase(q);
        }
        for (void* q : drop) (void)hipFree(q);
        // Stream-ordered scratch (StreamBuf) returns to the device's default
        // async pool, which keeps freed blocks (release threshold UINT64_MAX):
        // hand those back to the driver too before the retry.
        hipMemPool_t ap;
        if (hipDeviceSynchronize() == hipSuccess && hipDeviceGetDefaultMemPool(&ap, dev) == hipSuccess)
            (void)hipMemPoolTrimTo(ap, 0);
        (void)hipGetLastError();
        if (hipMalloc(&p, sz) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    std::lock_guard<std::mutex> g(P.mu);
    P.owned[p] = {dev, sz};
    return p;
}

size_t pool_round(size_t bytes) { return round_size(bytes); }

size_t pool_block_size(void* p) {
    Pool& P = pool();
    std::lock_guard<std::mutex> g(P.mu);
    auto it = P.owned.find(p);
    return it == P.owned.end() ? 0 : it->second.second;
}

void pool_release(void* p) {
    if (!p) return;
    Pool& P = pool();
    std::lock_guard<std::mutex> g(P.mu);
    auto it = P.owned.find(p);
    if (it == P.owned.end()) return;
    P.free_blocks[it->second.first].emplace(it->second.second, p);
}

// ── per-stream workspaces ─────────────────────────────────────────────────

namespace {
struct WsBlock {
    void* p = nullptr;
    size_t cap = 0;
};
struct WsKey {
    int dev;
    hipStream_t s;
    int slot;
    bool operator<(const WsKey& o) const {
        if (dev != o.dev) return dev < o.dev;
        if (s != o.s) return s < o.s;
        return slot < o.slot;
    }
};
struct WsCache {
    std::mutex mu;
    std::map<WsKey, WsBlock> live;
    std::multimap<std::pair<int, hipStream_t>, void*> retired;
};
WsCache& ws_cache() {
    static WsCache* c = new WsCache();  // never destroyed: outlives late calls at exit
    return *c;
}
}  // namespace

int stream_workspace(hipStream_t s, int slot, size_t bytes, void** out) {
    int dev = 0;
    MLXHIP_HIP(hipGetDevice(&dev));
    WsCache& C = ws_cache();
    std::lock_guard<std::mutex> g(C.mu);
    WsBlock& b = C.live[WsKey{dev, s, slot}];
    if (b.cap < bytes || !b.p) {
        // Grow geometrically (256-byte granules) so a slowly growing sequence
        // of requests allocates O(log) times.
        size_t cap = std::max<size_t>(bytes, b.cap + b.cap / 2);
        cap = std::max<size_t>((cap + 255) & ~size_t(255), 256);
        // During stream capture (mlxhip_graph_begin) an allocation is not a
        // stream operation: switch this thread to relaxed capture mode around
        // it, then back. The block outlives the recorded graph (retired
        // blocks are kept), so a replay never sees freed memory.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        const bool exchanged = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
        void* p = pool_alloc(cap);
        if (exchanged) (void)hipThreadExchangeStreamCaptureMode(&mode);
        (void)hipGetLastError();
        if (!p) return fail(MLXHIP_ERR_FFI_FAILED, "workspace: device allocation of %zu bytes failed", cap);
        if (b.p) C.retired.emplace(std::make_pair(dev, s), b.p);
        b.p = p;
        b.cap = cap;
    }
    *out = b.p;
    return MLXHIP_OK;
}

void release_stream_workspaces(hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    WsCache& C = ws_cache();
    std::lock_guard<std::mutex> g(C.mu);
    for (auto it = C.live.begin(); it != C.live.end();) {
        if (it->first.dev == dev && it->first.s == s) {
            pool_release(it->second.p);
            it = C.live.erase(it);
        } else {
            ++it;
        }
    }
    auto range = C.retired.equal_range(std::make_pair(dev, s));
    for (auto it = range.first; it != range.second; ++it) pool_release(it->second);
    C.retired.erase(range.first, range.second);
}

float* Scratch::get(size_t n_floats) { return static_cast<float*>(get_bytes(n_floats * sizeof(float))); }

void* Scratch::get_bytes(size_t bytes) {
    void* p = pool_alloc(bytes ? bytes : 1);
    if (p) blocks.push_back(p);
    return p;
}

void Scratch::release_all() {
    for (void* p : blocks) pool_release(p);
    blocks.clear();
    own_planes.entries.clear();
}

// ── eval_node on device operands ──────────────────────────────────────────

namespace {

bool same_shape(const mlxhip_input_t& a, const mlxhip_input_t& b) {
    if (a.ndim != b.ndim) return false;
    for (size_t i = 0; i < a.ndim; ++i)
        if (a.shape[i] != b.shape[i]) return false;
    return true;
}

std::string shape_str(const int64_t* s, size_t n) {
    std::string r = "[";
    for (size_t i = 0; i < n; ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

int resolve_axis(int axis, size_t ndim, const char* what, size_t* out) {
    const int nd = (int)ndim;
    const int ax = axis < 0 ? nd + axis : axis;
    if (ax < 0 || ax >= nd)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "%saxis %d out of range for ndim %d", what, axis, nd);
    *out = (size_t)ax;
    return MLXHIP_OK;
}

int64_t prod(const int64_t* s, size_t lo, size_t hi) {
    int64_t p = 1;
    for (size_t i = lo; i < hi; ++i) p *= s[i];
    return p;
}

// Output size the op produces must match the buffer sized from out_meta.
int expect_len(int64_t have, int64_t want, const char* op) {
    if (have != want) return fail_shape({want}, {have}, op);
    return MLXHIP_OK;
}

int copy_dev(float* dst, const float* src, int64_t n, hipStream_t s) {
    if (n == 0 || dst == src) return MLXHIP_OK;
    MLXHIP_HIP(hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, s));
    return MLXHIP_OK;
}

int ew1(int ew_op, const float* x, float* out, int64_t n, hipStream_t s) {
    mlxhip_ew_instr_t ins{ew_op, 0};
    const float* in[1] = {x};
    return ew_chain(&ins, 1, in, 1, out, n, s);
}

int ew2(int ew_op, const float* acc, const float* other, float* out, int64_t n, hipStream_t s) {
    mlxhip_ew_instr_t ins{ew_op, 1};
    const float* in[2] = {acc, other};
    return ew_chain(&ins, 1, in, 2, out, n, s);
}

#define REQUIRE(idx)                                                                        \
    do {                                                                                    \
        if ((size_t)(idx) >= n_inputs)                                                      \
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "expected input at index %d", (int)(idx)); \
    } while (0)

int eval_matmul(const mlxhip_input_t* in, size_t n_inputs, const mlxhip_meta_t& meta, float* out,
                hipStream_t s, Scratch& scratch, const int* trans_hint, const float* bias = nullptr) {
    // Rank 2: matmul (cpu_kernels.rs:197-230). Rank 3: [B,M,K] @ [B,K,N] ->
    // [B,M,N], one product per batch slice, the batched form the reference
    // specifies for matmul (evals/tasks/003_matmul_batch_3d.json); ranks must
    // agree and so must the batch sizes.
    REQUIRE(0);
    REQUIRE(1);
    const mlxhip_input_t &a = in[0], &b = in[1];
    if (!((a.ndim == 2 && b.ndim == 2) || (a.ndim == 3 && b.ndim == 3)))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "matmul requires 2D tensors (or two 3D batched tensors)");
    const size_t r = a.ndim - 2;  // index of the first matrix dimension
    const int64_t batch = a.ndim == 3 ? a.shape[0] : 1;
    if (a.ndim == 3 && b.shape[0] != batch)
        return fail_shape(std::vector<int64_t>(a.shape, a.shape + a.ndim),
                          std::vector<int64_t>(b.shape, b.shape + b.ndim), "matmul batch");
    const bool ta = trans_hint && trans_hint[0], tb = trans_hint && trans_hint[1];
    // With a folded Transpose the input holds the source [K, M] / [N, K].
    const int64_t m = ta ? a.shape[r + 1] : a.shape[r], k = ta ? a.shape[r] : a.shape[r + 1];
    const int64_t k2 = tb ? b.shape[r + 1] : b.shape[r], n = tb ? b.shape[r] : b.shape[r + 1];
    if (k != k2) return fail_shape({m, k}, {k2, n});
    MLXHIP_TRY(expect_len(batch * m * n, numel_of(meta.shape, meta.ndim), "matmul"));
    const int64_t lda = ta ? m : k, ldb = tb ? k : n;
    // The reference stores every logical dtype as f32 (crates/mlx-core/src/tensor.rs:105-125)
    // and its matmul multiplies those stored values (cpu_kernels.rs:197-230),
    // whatever the dtype tag: a bf16/f16-tagged MatMul node is an f32 product
    // here too. The 16-bit MFMA path (operands held as bf16/f16) is the
    // explicit mlxhip_gemm with ab_dtype BF16/F16.
    return gemm(MLXHIP_DTYPE_F32, MLXHIP_DTYPE_F32, ta, tb, m, n, k, batch, a.data, lda, m * k, b.data, ldb,
                k * n, out, n, m * n, s, scratch.planes, bias);
}

int eval_attention(const mlxhip_op_t& op, const mlxhip_input_t* in, size_t n_inputs,
                   const mlxhip_meta_t& meta, float* out, hipStream_t s, Scratch& scratch) {
    // cpu_attention (cpu_kernels.rs:738-812): scores = Q K^T, scaled causal
    // softmax, Y = P V. K^T is read in place by the NT GEMM.
    if (n_inputs != 3) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Attention requires exactly 3 inputs [Q, K, V]");
    const mlxhip_input_t &q = in[0], &k = in[1], &v = in[2];
    if (q.ndim != 2 || k.ndim != 2 || v.ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Attention inputs must be 2D");
    const int64_t tq = q.shape[0], dh = q.shape[1], tk = k.shape[0], dhk = k.shape[1];
    const int64_t tkv = v.shape[0], dhv = v.shape[1];
    if (dh != dhk) return fail_shape({tq, dh}, {tk, dhk});
    if (tk != tkv || dh != dhv) return fail_shape({tk, dh}, {tkv, dhv});
    MLXHIP_TRY(expect_len(tq * dh, numel_of(meta.shape, meta.ndim), "attention"));
    if (tq * dh == 0) return MLXHIP_OK;
    if (tk > 0 && attention_fused_supported(dh, tq, tk) &&
        ((reinterpret_cast<uintptr_t>(q.data) | reinterpret_cast<uintptr_t>(k.data) |
          reinterpret_cast<uintptr_t>(v.data) | reinterpret_cast<uintptr_t>(out)) % 16) == 0)
        return attention_fused(q.data, k.data, v.data, out, 1, tq, tk, dh, 0, 0, 0, 0, op.scale, op.causal, s);
    float* scores = scratch.get((size_t)std::max<int64_t>(1, tq * tk));
    float* probs = scratch.get((size_t)std::max<int64_t>(1, tq * tk));
    if (!scores || !probs) return fail(MLXHIP_ERR_FFI_FAILED, "attention: scratch allocation failed");
    MLXHIP_TRY(gemm(MLXHIP_DTYPE_F32, MLXHIP_DTYPE_F32, 0, 1, tq, tk, dh, 1, q.data, dh, 0, k.data, dh, 0,
                    scores, tk, 0, s));
    MLXHIP_TRY(row_op(ROW_SCALED_MASKED_SOFTMAX, scores, nullptr, probs, tq, tk, op.scale, op.causal, s));
    return gemm(MLXHIP_DTYPE_F32, MLXHIP_DTYPE_F32, 0, 0, tq, dh, tk, 1, probs, tk, 0, v.data, dh, 0, out,
                dh, 0, s);
}

// HeadAttention: the Attention op's arithmetic for every head of
// [heads, t, dh] operands, in one fused launch when the shape and alignment
// allow it, else head by head through eval_attention.
// HeadAttention: heads of Q [.., tq, ..], K / V [.., tk, ..]. Without an
// axis: [heads, t, dh], one head per leading index. With axis = H (has_axis):
// [groups, t, H * dh], H heads side by side in each row (the layout of a
// [batch * t, d_model] projection viewed as [batch, t, d_model]); the output
// takes the inputs' layout.
int eval_head_attention(const mlxhip_op_t& op, const mlxhip_input_t* in, size_t n_inputs,
                        const mlxhip_meta_t& meta, float* out, hipStream_t s, Scratch& scratch) {
    if (n_inputs != 3) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttention requires exactly 3 inputs [Q, K, V]");
    const mlxhip_input_t &q = in[0], &k = in[1], &v = in[2];
    if (q.ndim != 3 || k.ndim != 3 || v.ndim != 3)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttention inputs must be 3-D [heads, t, dh]");
    const int64_t g = q.shape[0], tq = q.shape[1], w = q.shape[2], tk = k.shape[1];
    if (k.shape[0] != g || v.shape[0] != g || k.shape[2] != w || v.shape[1] != tk || v.shape[2] != w)
        return fail_shape({g, tk, w}, {k.shape[0], k.shape[1], k.shape[2]}, "HeadAttention");
    const int64_t hg = op.has_axis ? op.axis : 1;
    if (hg < 1 || w % hg)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttention: %lld heads per row of %lld values", (long long)hg,
                    (long long)w);
    const int64_t h = g * hg, dh = w / hg;
    MLXHIP_TRY(expect_len(g * tq * w, numel_of(meta.shape, meta.ndim), "HeadAttention"));
    if (g * tq * w == 0) return MLXHIP_OK;
    if (tk == 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttention: no keys");
    const uintptr_t al = reinterpret_cast<uintptr_t>(q.data) | reinterpret_cast<uintptr_t>(k.data) |
                         reinterpret_cast<uintptr_t>(v.data) | reinterpret_cast<uintptr_t>(out);
    if (attention_fused_supported(dh, tq, tk) && al % 16 == 0 && dh % 4 == 0 && w % 4 == 0)
        return attention_fused(q.data, k.data, v.data, out, h, tq, tk, dh, tq * w, tk * w, tk * w, tq * w,
                               op.scale, op.causal, s, hg, w);
    if (hg > 1)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT,
                    "HeadAttention with heads side by side in rows needs the fused kernel (dh 16, 32, 64 or 128, "
                    "16-byte aligned rows): dh=%lld", (long long)dh);
    const int64_t qs[2] = {tq, dh}, ks[2] = {tk, dh};
    for (int64_t i = 0; i < h; ++i) {
        mlxhip_input_t hi[3] = {{q.data + i * tq * dh, (size_t)(tq * dh), qs, 2, q.dtype},
                                {k.data + i * tk * dh, (size_t)(tk * dh), ks, 2, k.dtype},
                                {v.data + i * tk * dh, (size_t)(tk * dh), ks, 2, v.dtype}};
        mlxhip_meta_t m = meta;
        m.shape = qs;
        m.ndim = 2;
        MLXHIP_TRY(eval_attention(op, hi, 3, m, out + i * tq * dh, s, scratch));
    }
    return MLXHIP_OK;
}

// HeadAttentionVjp: [Q, K, V, O, dO] -> [3, ...] = dQ, dK, dV, each in the
// inputs' layout (axis as for HeadAttention).
int eval_head_attention_vjp(const mlxhip_op_t& op, const mlxhip_input_t* in, size_t n_inputs,
                            const mlxhip_meta_t& meta, float* out, hipStream_t s) {
    if (n_inputs != 5)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttentionVjp requires exactly 5 inputs [Q, K, V, O, dO]");
    const mlxhip_input_t& q = in[0];
    if (q.ndim != 3) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttentionVjp inputs must be 3-D [heads, t, dh]");
    for (size_t i = 1; i < 5; ++i)
        if (in[i].ndim != 3 || in[i].shape[0] != q.shape[0] || in[i].shape[1] != q.shape[1] ||
            in[i].shape[2] != q.shape[2])
            return fail_shape(std::vector<int64_t>(q.shape, q.shape + 3),
                              std::vector<int64_t>(in[i].shape, in[i].shape + in[i].ndim), "HeadAttentionVjp");
    const int64_t g = q.shape[0], t = q.shape[1], w = q.shape[2], n = g * t * w;
    const int64_t hg = op.has_axis ? op.axis : 1;
    if (hg < 1 || w % hg)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "HeadAttentionVjp: %lld heads per row of %lld values",
                    (long long)hg, (long long)w);
    MLXHIP_TRY(expect_len(3 * n, numel_of(meta.shape, meta.ndim), "HeadAttentionVjp"));
    if (n == 0) return MLXHIP_OK;
    return attention_vjp(in[0].data, in[1].data, in[2].data, in[3].data, in[4].data, out, out + n, out + 2 * n,
                         g * hg, t, w / hg, op.scale, op.causal, s, hg, w);
}

}  // namespace

int eval_matmul_group(int groups, const mlxhip_input_t* in, const int* hints, float* const* outs, hipStream_t s,
                      Scratch& scratch, const float* const* biases) {
    if (groups < 2 || groups > 4) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "matmul group of %d", groups);
    const mlxhip_input_t &a = in[0], &b = in[1];
    if (a.ndim != 2 || b.ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "matmul group: rank-2 operands only");
    const bool ta = hints[0] != 0, tb = hints[1] != 0;
    const int64_t m = ta ? a.shape[1] : a.shape[0], k = ta ? a.shape[0] : a.shape[1];
    const int64_t k2 = tb ? b.shape[1] : b.shape[0], n = tb ? b.shape[0] : b.shape[1];
    if (k != k2) return fail_shape({m, k}, {k2, n});
    const float* pa[4];
    const float* pb[4];
    for (int i = 0; i < groups; ++i) {
        const mlxhip_input_t &ai = in[2 * i], &bi = in[2 * i + 1];
        if (ai.ndim != 2 || bi.ndim != 2 || ai.shape[0] != a.shape[0] || ai.shape[1] != a.shape[1] ||
            bi.shape[0] != b.shape[0] || bi.shape[1] != b.shape[1] || hints[2 * i] != hints[0] ||
            hints[2 * i + 1] != hints[1])
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "matmul group: products of different shapes");
        if ((int64_t)ai.len != a.shape[0] * a.shape[1] || (int64_t)bi.len != b.shape[0] * b.shape[1])
            return fail_shape({a.shape[0] * a.shape[1]}, {(int64_t)ai.len}, "matmul group operand length");
        pa[i] = ai.data;
        pb[i] = bi.data;
    }
    return gemm_f32_grouped(ta, tb, m, n, k, groups, pa, ta ? m : k, pb, tb ? k : n, outs, n, s, scratch.planes,
                            biases);
}

int eval_matmul_bias(const mlxhip_input_t* in, const mlxhip_meta_t& meta, float* out, hipStream_t s,
                     Scratch& scratch, const int* trans_hint, const float* bias) {
    if (in[0].ndim != 2 || in[1].ndim != 2)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "matmul with a bias term: rank-2 operands only");
    return eval_matmul(in, 2, meta, out, s, scratch, trans_hint, bias);
}

int eval_node_device(const mlxhip_op_t& op, const mlxhip_input_t* in, size_t n_inputs,
                     const mlxhip_meta_t& meta, float* out, hipStream_t s, Scratch& scratch,
                     const int* trans_hint) {
    const int64_t out_n = numel_of(meta.shape, meta.ndim);
    // Kernels index by shape: every operand must hold exactly numel(shape) values.
    for (size_t i = 0; i < n_inputs; ++i) {
        if (in[i].ndim && !in[i].shape) return fail(MLXHIP_ERR_NULL_PTR, "input %zu has a null shape", i);
        if ((int64_t)in[i].len != numel_of(in[i].shape, in[i].ndim))
            return fail_shape({numel_of(in[i].shape, in[i].ndim)}, {(int64_t)in[i].len}, "input length");
        if (in[i].len && !in[i].data) return fail(MLXHIP_ERR_NULL_PTR, "input %zu is null", i);
    }
    if (meta.ndim && !meta.shape) return fail(MLXHIP_ERR_NULL_PTR, "out_meta has a null shape");
    switch (op.kind) {
        case MLXHIP_OP_CONSTANT:
        case MLXHIP_OP_PARAMETER:
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Constant/Parameter nodes should be pre-materialized");
        case MLXHIP_OP_ADD:
        case MLXHIP_OP_SUB:
        case MLXHIP_OP_MUL:
        case MLXHIP_OP_DIV: {
            REQUIRE(0);
            REQUIRE(1);
            if (in[0].len != in[1].len)
                return fail_shape(std::vector<int64_t>(in[0].shape, in[0].shape + in[0].ndim),
                              std::vector<int64_t>(in[1].shape, in[1].shape + in[1].ndim));
            MLXHIP_TRY(expect_len((int64_t)in[0].len, out_n, "binary"));
            const int ew = op.kind == MLXHIP_OP_ADD ? MLXHIP_EW_ADD
                           : op.kind == MLXHIP_OP_SUB ? MLXHIP_EW_SUB
                           : op.kind == MLXHIP_OP_MUL ? MLXHIP_EW_MUL
                                                      : MLXHIP_EW_DIV;
            return ew2(ew, in[0].data, in[1].data, out, out_n, s);
        }
        case MLXHIP_OP_NEG:
        case MLXHIP_OP_EXP:
        case MLXHIP_OP_LOG:
        case MLXHIP_OP_SQRT:
        case MLXHIP_OP_SILU:
        case MLXHIP_OP_GELU: {
            REQUIRE(0);
            MLXHIP_TRY(expect_len((int64_t)in[0].len, out_n, "unary"));
            const int ew = op.kind == MLXHIP_OP_NEG ? MLXHIP_EW_NEG
                           : op.kind == MLXHIP_OP_EXP ? MLXHIP_EW_EXP
                           : op.kind == MLXHIP_OP_LOG ? MLXHIP_EW_LOG
                           : op.kind == MLXHIP_OP_SQRT ? MLXHIP_EW_SQRT
                           : op.kind == MLXHIP_OP_SILU ? MLXHIP_EW_SILU
                                                       : MLXHIP_EW_GELU;
            return ew1(ew, in[0].data, out, out_n, s);
        }
        case MLXHIP_OP_SILU_VJP:
        case MLXHIP_OP_GELU_VJP: {
            REQUIRE(0);
            REQUIRE(1);
            if (in[0].len != in[1].len)
                return fail_shape(std::vector<int64_t>(in[1].shape, in[1].shape + in[1].ndim),
                              std::vector<int64_t>(in[0].shape, in[0].shape + in[0].ndim));
            MLXHIP_TRY(expect_len((int64_t)in[0].len, out_n, "activation vjp"));
            // acc = x (input 1), operand = dy (input 0)
            return ew2(op.kind == MLXHIP_OP_SILU_VJP ? MLXHIP_EW_SILU_VJP : MLXHIP_EW_GELU_VJP, in[1].data,
                       in[0].data, out, out_n, s);
        }
        case MLXHIP_OP_SUM:
        case MLXHIP_OP_MEAN:
        case MLXHIP_OP_MAX: {
            REQUIRE(0);
            const int kind = op.kind == MLXHIP_OP_SUM ? 0 : op.kind == MLXHIP_OP_MEAN ? 1 : 2;
            if (!op.has_axis) {
                MLXHIP_TRY(expect_len(1, out_n, "reduce"));
                return reduce_all(kind, in[0].data, out, (int64_t)in[0].len, s);
            }
            size_t ax;
            MLXHIP_TRY(resolve_axis(op.axis, in[0].ndim, "", &ax));
            const int64_t outer = prod(in[0].shape, 0, ax), dim = in[0].shape[ax];
            const int64_t inner = prod(in[0].shape, ax + 1, in[0].ndim);
            MLXHIP_TRY(expect_len(outer * inner, out_n, "reduce"));
            return reduce_axis(kind, in[0].data, out, outer, dim, inner, s);
        }
        case MLXHIP_OP_MATMUL: return eval_matmul(in, n_inputs, meta, out, s, scratch, trans_hint);
        case MLXHIP_OP_RESHAPE:
            REQUIRE(0);
            MLXHIP_TRY(expect_len((int64_t)in[0].len, out_n, "reshape"));
            return copy_dev(out, in[0].data, out_n, s);
        case MLXHIP_OP_TRANSPOSE: {
            REQUIRE(0);
            const mlxhip_input_t& a = in[0];
            const size_t nd = a.ndim;
            if (nd > 8) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose: rank %zu > 8", nd);
            int64_t perm[8];
            if (op.axes) {
                if (op.axes_len != nd)
                    return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose axes length must match ndim");
                for (size_t i = 0; i < nd; ++i) perm[i] = op.axes[i];
            } else {
                for (size_t i = 0; i < nd; ++i) perm[i] = (int64_t)(nd - 1 - i);
            }
            MLXHIP_TRY(expect_len((int64_t)a.len, out_n, "transpose"));
            if (nd <= 1) return copy_dev(out, a.data, out_n, s);
            return permute(a.data, out, a.shape, perm, (int)nd, s);
        }
        case MLXHIP_OP_SOFTMAX: {
            REQUIRE(0);
            const mlxhip_input_t& a = in[0];
            size_t ax;
            MLXHIP_TRY(resolve_axis(op.axis, a.ndim, "", &ax));
            MLXHIP_TRY(expect_len((int64_t)a.len, out_n, "softmax"));
            const int64_t outer = prod(a.shape, 0, ax), dim = a.shape[ax], inner = prod(a.shape, ax + 1, a.ndim);
            if (inner == 1) return row_op(ROW_SOFTMAX, a.data, nullptr, out, outer, dim, 0.f, 0, s);
            return fibre_softmax(false, a.data, nullptr, out, outer, dim, inner, s);
        }
        case MLXHIP_OP_LAYER_NORM:
        case MLXHIP_OP_RMS_NORM: {
            REQUIRE(0);
            const mlxhip_input_t& a = in[0];
            MLXHIP_TRY(expect_len((int64_t)a.len, out_n, "norm"));
            if (a.ndim == 0) return copy_dev(out, a.data, out_n, s);
            const int64_t d = a.shape[a.ndim - 1];
            if (d == 0) return MLXHIP_OK;
            return row_op(op.kind == MLXHIP_OP_LAYER_NORM ? ROW_LAYERNORM : ROW_RMSNORM, a.data, nullptr, out,
                          (int64_t)a.len / d, d, op.eps, 0, s);
        }
        case MLXHIP_OP_ROPE: {
            REQUIRE(0);
            if (meta.ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Rope input must be 2-D [tokens, head_dim]");
            const int64_t tokens = meta.shape[0], hd = meta.shape[1], rd = (int64_t)op.rotary_dim;
            if (rd > hd || rd % 2 != 0)
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "rotary_dim must be even and <= head_dim");
            MLXHIP_TRY(expect_len((int64_t)in[0].len, out_n, "rope"));
            return rope_interleaved(in[0].data, out, tokens, hd, rd, (int64_t)op.pos_offset, op.theta,
                                    (int64_t)in[0].len, s);
        }
        case MLXHIP_OP_ROPE_MLX: {
            REQUIRE(0);
            const mlxhip_input_t& a = in[0];
            if (a.ndim < 1) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "RoPE requires at least 1 dimension");
            const int64_t hd = a.shape[a.ndim - 1];
            if (hd % 2 != 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "RoPE head_dim must be even, got %lld", (long long)hd);
            MLXHIP_TRY(expect_len((int64_t)a.len, out_n, "RoPE"));
            if (hd == 0) return MLXHIP_OK;
            return rope_mlx(a.data, out, (int64_t)a.len / hd, hd, (int64_t)op.offset, op.base, op.traditional, s);
        }
        case MLXHIP_OP_BROADCAST: {
            REQUIRE(0);
            if (!op.shape && op.shape_len) return fail(MLXHIP_ERR_NULL_PTR, "broadcast: null target shape");
            MLXHIP_TRY(expect_len(numel_of(op.shape, op.shape_len), out_n, "broadcast"));
            return broadcast(in[0].data, out, in[0].shape, (int)in[0].ndim, op.shape, (int)op.shape_len, s);
        }
        case MLXHIP_OP_EMBEDDING: {
            REQUIRE(0);
            REQUIRE(1);
            const mlxhip_input_t &w = in[0], &idx = in[1];
            if (w.ndim != 2)
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Embedding weight must be 2D [num_embeddings, embedding_dim]");
            const int64_t dim = w.shape[1];
            if ((int64_t)idx.len * dim > out_n)
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "embedding: output smaller than indices x dim");
            if ((int64_t)idx.len * dim < out_n) MLXHIP_TRY(fill(out, 0.0f, out_n, s));
            return embedding(w.data, idx.data, out, (int64_t)idx.len, w.shape[0], dim, s);
        }
        case MLXHIP_OP_SCALED_MASKED_SOFTMAX: {
            REQUIRE(0);
            const mlxhip_input_t& a = in[0];
            if (a.ndim != 2) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "ScaledMaskedSoftmax requires 2D input [Tq, Tk]");
            MLXHIP_TRY(expect_len(a.shape[0] * a.shape[1], out_n, "scaled_masked_softmax"));
            return row_op(ROW_SCALED_MASKED_SOFTMAX, a.data, nullptr, out, a.shape[0], a.shape[1], op.scale,
                          op.causal, s);
        }
        case MLXHIP_OP_ATTENTION: return eval_attention(op, in, n_inputs, meta, out, s, scratch);
        case MLXHIP_OP_HEAD_ATTENTION: return eval_head_attention(op, in, n_inputs, meta, out, s, scratch);
        case MLXHIP_OP_HEAD_ATTENTION_VJP: return eval_head_attention_vjp(op, in, n_inputs, meta, out, s);
        case MLXHIP_OP_LAYER_NORM_VJP:
        case MLXHIP_OP_RMS_NORM_VJP: {
            REQUIRE(0);
            REQUIRE(1);
            const mlxhip_input_t &dy = in[0], &x = in[1];
            if (!same_shape(dy, x) || dy.len != x.len)
                return fail_shape(std::vector<int64_t>(x.shape, x.shape + x.ndim),
                              std::vector<int64_t>(dy.shape, dy.shape + dy.ndim));
            MLXHIP_TRY(expect_len((int64_t)x.len, out_n, "norm vjp"));
            if (x.ndim == 0) return copy_dev(out, dy.data, out_n, s);
            const int64_t d = x.shape[x.ndim - 1];
            if (d == 0 || x.len == 0) return fill(out, 0.0f, out_n, s);
            return row_op(op.kind == MLXHIP_OP_LAYER_NORM_VJP ? ROW_LAYERNORM_VJP : ROW_RMSNORM_VJP, dy.data,
                          x.data, out, (int64_t)x.len / d, d, op.eps, 0, s);
        }
        case MLXHIP_OP_SOFTMAX_VJP: {
            REQUIRE(0);
            REQUIRE(1);
            const mlxhip_input_t &dy = in[0], &sm = in[1];
            if (dy.len != sm.len)
                return fail_shape(std::vector<int64_t>(sm.shape, sm.shape + sm.ndim),
                              std::vector<int64_t>(dy.shape, dy.shape + dy.ndim));
            size_t ax;
            MLXHIP_TRY(resolve_axis(op.axis, sm.ndim, "", &ax));
            MLXHIP_TRY(expect_len((int64_t)sm.len, out_n, "softmax vjp"));
            const int64_t outer = prod(sm.shape, 0, ax), dim = sm.shape[ax], inner = prod(sm.shape, ax + 1, sm.ndim);
            if (inner == 1) return row_op(ROW_SOFTMAX_VJP, dy.data, sm.data, out, outer, dim, 0.f, 0, s);
            return fibre_softmax(true, dy.data, sm.data, out, outer, dim, inner, s);
        }
        case MLXHIP_OP_NARROW: {
            REQUIRE(0);
            const mlxhip_input_t& a = in[0];
            size_t ax;
            MLXHIP_TRY(resolve_axis(op.axis, a.ndim, "narrow: ", &ax));
            const int64_t ds = a.shape[ax];
            if (op.start < 0 || op.start + op.length > ds)
                return fail(MLXHIP_ERR_INVALID_ARGUMENT, "narrow: start %lld + length %lld exceeds dim size %lld",
                            (long long)op.start, (long long)op.length, (long long)ds);
            const int64_t outer = prod(a.shape, 0, ax), inner = prod(a.shape, ax + 1, a.ndim);
            MLXHIP_TRY(expect_len(outer * op.length * inner, out_n, "narrow"));
            return narrow(a.data, out, outer, ds, inner, op.start, op.length, s);
        }
        case MLXHIP_OP_CONCATENATE: {
            if (n_inputs == 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Concatenate requires at least one input");
            const mlxhip_input_t& f = in[0];
            size_t ax;
            MLXHIP_TRY(resolve_axis(op.axis, f.ndim, "concatenate: ", &ax));
            int64_t total = 0;
            for (size_t i = 0; i < n_inputs; ++i) {
                if (in[i].ndim != f.ndim)
                    return fail(MLXHIP_ERR_INVALID_ARGUMENT, "Concatenate: all inputs must have same ndim");
                for (size_t d = 0; d < f.ndim; ++d)
                    if (d != ax && in[i].shape[d] != f.shape[d])
                        return fail_shape(std::vector<int64_t>(f.shape, f.shape + f.ndim),
                              std::vector<int64_t>(in[i].shape, in[i].shape + in[i].ndim));
                total += in[i].shape[ax];
            }
            const int64_t outer = prod(f.shape, 0, ax), inner = prod(f.shape, ax + 1, f.ndim);
            MLXHIP_TRY(expect_len(outer * total * inner, out_n, "concatenate"));
            int64_t at = 0;
            for (size_t i = 0; i < n_inputs; ++i) {
                MLXHIP_TRY(concat_part(in[i].data, out, outer, in[i].shape[ax], inner, total, at, s));
                at += in[i].shape[ax];
            }
            return MLXHIP_OK;
        }
        default: return fail(MLXHIP_ERR_INVALID_ARGUMENT, "mlx-hip: unsupported op %d", op.kind);
    }
}

}  // namespace mlxhip

// ══ C ABI ═══════════════════════════════════════════════════════════════════

using namespace mlxhip;

struct mlxhip_buffer_t {
    void* ptr;
    size_t bytes;
    int device;
};

struct mlxhip_event_t {
    hipEvent_t ev;
};

extern "C" {

int mlxhip_abi_version(void) { return MLXHIP_ABI_VERSION; }

int mlxhip_debug_fail_allocations(int64_t after) {
    g_alloc_budget.store(after < 0 ? -1 : after);
    return MLXHIP_OK;
}

const char* mlxhip_last_error(void) { return last_error().c_str(); }

int mlxhip_last_status(void) { return t_last_status; }

int mlxhip_last_shape_mismatch(int64_t* expected, size_t* expected_ndim, int64_t* got, size_t* got_ndim,
                               size_t cap) {
    if (t_last_status != MLXHIP_ERR_SHAPE_MISMATCH || (t_shape_expected.empty() && t_shape_got.empty()))
        return MLXHIP_ERR_INVALID_ARGUMENT;  // not recorded through fail(): leaves the last error as it is
    if (expected_ndim) *expected_ndim = t_shape_expected.size();
    if (got_ndim) *got_ndim = t_shape_got.size();
    for (size_t i = 0; expected && i < t_shape_expected.size() && i < cap; ++i) expected[i] = t_shape_expected[i];
    for (size_t i = 0; got && i < t_shape_got.size() && i < cap; ++i) got[i] = t_shape_got[i];
    return MLXHIP_OK;
}

int mlxhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int mlxhip_init(int device) {
    int n = mlxhip_device_count();
    if (n <= 0) return fail(MLXHIP_ERR_BACKEND_UNAVAILABLE, "mlx-hip: no HIP device available");
    if (device < 0 || device >= n) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "mlx-hip: device %d of %d", device, n);
    MLXHIP_HIP(hipSetDevice(device));
    MLXHIP_HIP(hipFree(nullptr));  // creates the context now rather than on first use
    t_device = device;
    return MLXHIP_OK;
}

int mlxhip_synchronize(void* stream) {
    MLXHIP_TRY(ensure_device());
    if (stream) MLXHIP_HIP(hipStreamSynchronize(as_stream(stream)));
    else MLXHIP_HIP(hipDeviceSynchronize());
    return MLXHIP_OK;
}

int mlxhip_eval_node(const mlxhip_op_t* op, const mlxhip_input_t* inputs, size_t n_inputs,
                     const mlxhip_meta_t* out_meta, float* out_host, size_t out_len) {
    if (!op || !out_meta || (n_inputs && !inputs)) return fail(MLXHIP_ERR_NULL_PTR, "eval_node: null argument");
    const int64_t want = numel_of(out_meta->shape, out_meta->ndim);
    if ((int64_t)out_len != want)
        return fail_shape({want}, {(int64_t)out_len}, "eval_node out_len");
    if (want && !out_host) return fail(MLXHIP_ERR_NULL_PTR, "eval_node: null output");
    MLXHIP_TRY(ensure_device());
    hipStream_t s = thread_stream();
    Scratch scratch;
    std::vector<mlxhip_input_t> dev(n_inputs);
    for (size_t i = 0; i < n_inputs; ++i) {
        dev[i] = inputs[i];
        if (inputs[i].len && !inputs[i].data) return fail(MLXHIP_ERR_NULL_PTR, "eval_node: input %zu is null", i);
        float* d = scratch.get(inputs[i].len ? inputs[i].len : 1);
        if (!d) return fail(MLXHIP_ERR_FFI_FAILED, "eval_node: device allocation failed");
        if (inputs[i].len)
            MLXHIP_HIP(hipMemcpyAsync(d, inputs[i].data, inputs[i].len * sizeof(float), hipMemcpyHostToDevice, s));
        dev[i].data = d;
    }
    float* dout = scratch.get(want ? (size_t)want : 1);
    if (!dout) return fail(MLXHIP_ERR_FFI_FAILED, "eval_node: device allocation failed");
    int rc = eval_node_device(*op, dev.data(), n_inputs, *out_meta, dout, s, scratch);
    if (rc == MLXHIP_OK && want)
        rc = hipMemcpyAsync(out_host, dout, (size_t)want * sizeof(float), hipMemcpyDeviceToHost, s) == hipSuccess
                 ? MLXHIP_OK
                 : fail(MLXHIP_ERR_FFI_FAILED, "eval_node: copy to host failed");
    hipError_t e = hipStreamSynchronize(s);
    if (rc == MLXHIP_OK && e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    return rc;  // scratch returns to the pool after the synchronise
}

mlxhip_buffer_t* mlxhip_buffer_alloc(size_t bytes) {
    if (ensure_device() != MLXHIP_OK) return nullptr;
    void* p = nullptr;
    if (bytes && forced_alloc_failure()) {
        fail(MLXHIP_ERR_FFI_FAILED, "hipMalloc(%zu) failed (forced by the allocation-failure hook)", bytes);
        return nullptr;
    }
    if (bytes && hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();  // not to be reported by a later launch check
        fail(MLXHIP_ERR_FFI_FAILED, "hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    return new mlxhip_buffer_t{p, bytes, dev};
}

void mlxhip_buffer_free(mlxhip_buffer_t* buf) {
    if (!buf) return;
    if (buf->ptr) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (cur != buf->device) (void)hipSetDevice(buf->device);
        (void)hipDeviceSynchronize();  // no queued work may still use it
        (void)hipFree(buf->ptr);
        if (cur != buf->device) (void)hipSetDevice(cur);
    }
    delete buf;
}

void* mlxhip_buffer_ptr(const mlxhip_buffer_t* buf) { return buf ? buf->ptr : nullptr; }

size_t mlxhip_buffer_size(const mlxhip_buffer_t* buf) { return buf ? buf->bytes : 0; }

int mlxhip_buffer_upload(mlxhip_buffer_t* buf, size_t offset, const void* host, size_t bytes) {
    if (!buf || (bytes && !host)) return fail(MLXHIP_ERR_NULL_PTR, "buffer_upload: null argument");
    if (offset > buf->bytes || bytes > buf->bytes - offset)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "buffer_upload: %zu bytes at %zu exceed %zu", bytes, offset, buf->bytes);
    if (!bytes) return MLXHIP_OK;
    MLXHIP_TRY(ensure_device());
    MLXHIP_HIP(hipMemcpy(static_cast<char*>(buf->ptr) + offset, host, bytes, hipMemcpyHostToDevice));
    return MLXHIP_OK;
}

int mlxhip_buffer_download(const mlxhip_buffer_t* buf, size_t offset, void* host, size_t bytes) {
    if (!buf || (bytes && !host)) return fail(MLXHIP_ERR_NULL_PTR, "buffer_download: null argument");
    if (offset > buf->bytes || bytes > buf->bytes - offset)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "buffer_download: %zu bytes at %zu exceed %zu", bytes, offset, buf->bytes);
    if (!bytes) return MLXHIP_OK;
    MLXHIP_TRY(ensure_device());
    MLXHIP_HIP(hipDeviceSynchronize());
    MLXHIP_HIP(hipMemcpy(host, static_cast<const char*>(buf->ptr) + offset, bytes, hipMemcpyDeviceToHost));
    return MLXHIP_OK;
}

int mlxhip_eval_node_dev(const mlxhip_op_t* op, const mlxhip_input_t* inputs, size_t n_inputs,
                         const mlxhip_meta_t* out_meta, float* out, void* stream) {
    if (!op || !out_meta || (n_inputs && !inputs)) return fail(MLXHIP_ERR_NULL_PTR, "eval_node_dev: null argument");
    const int64_t want = numel_of(out_meta->shape, out_meta->ndim);
    if (want && !out) return fail(MLXHIP_ERR_NULL_PTR, "eval_node_dev: null output");
    MLXHIP_TRY(ensure_device());
    hipStream_t s = as_stream(stream);
    Scratch scratch;
    int rc = eval_node_device(*op, inputs, n_inputs, *out_meta, out, s, scratch);
    if (!scratch.blocks.empty()) {
        // Temporaries may only return to the pool once the kernels using them end.
        hipError_t e = hipStreamSynchronize(s);
        if (rc == MLXHIP_OK && e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    return rc;
}

int mlxhip_gemm(int32_t ab_dtype, int32_t c_dtype, int32_t trans_a, int32_t trans_b, int64_t m, int64_t n,
                int64_t k, int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b,
                int64_t ldb, int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, void* stream) {
    MLXHIP_TRY(ensure_device());
    return gemm(ab_dtype, c_dtype, trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, c, ldc,
                stride_c, as_stream(stream));
}

int mlxhip_gemm_noalloc(int32_t ab_dtype, int32_t c_dtype, int32_t trans_a, int32_t trans_b, int64_t m,
                        int64_t n, int64_t k, int64_t batch, const void* a, int64_t lda, int64_t stride_a,
                        const void* b, int64_t ldb, int64_t stride_b, void* c, int64_t ldc, int64_t stride_c,
                        void* stream) {
    MLXHIP_TRY(ensure_device());
    return gemm_noalloc(ab_dtype, c_dtype, trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, c,
                        ldc, stride_c, as_stream(stream));
}

size_t mlxhip_gemm_noalloc_scratch_bytes(void) { return GEMM_NOALLOC_SCRATCH_BYTES; }

int mlxhip_softmax_rows(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
    if ((rows * cols) && (!x || !y)) return fail(MLXHIP_ERR_NULL_PTR, "softmax_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_SOFTMAX, x, nullptr, y, rows, cols, 0.f, 0, as_stream(stream));
}

int mlxhip_scaled_masked_softmax_rows(const float* x, float* y, int64_t rows, int64_t cols, float scale,
                                      int32_t causal, void* stream) {
    if ((rows * cols) && (!x || !y)) return fail(MLXHIP_ERR_NULL_PTR, "scaled_masked_softmax_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_SCALED_MASKED_SOFTMAX, x, nullptr, y, rows, cols, scale, causal, as_stream(stream));
}

int mlxhip_layernorm_rows(const float* x, float* y, int64_t rows, int64_t cols, float eps, void* stream) {
    if ((rows * cols) && (!x || !y)) return fail(MLXHIP_ERR_NULL_PTR, "layernorm_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_LAYERNORM, x, nullptr, y, rows, cols, eps, 0, as_stream(stream));
}

int mlxhip_rmsnorm_rows(const float* x, float* y, int64_t rows, int64_t cols, float eps, void* stream) {
    if ((rows * cols) && (!x || !y)) return fail(MLXHIP_ERR_NULL_PTR, "rmsnorm_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_RMSNORM, x, nullptr, y, rows, cols, eps, 0, as_stream(stream));
}

int mlxhip_softmax_vjp_rows(const float* dy, const float* s, float* dx, int64_t rows, int64_t cols, void* stream) {
    if ((rows * cols) && (!dy || !s || !dx)) return fail(MLXHIP_ERR_NULL_PTR, "softmax_vjp_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_SOFTMAX_VJP, dy, s, dx, rows, cols, 0.f, 0, as_stream(stream));
}

int mlxhip_layernorm_vjp_rows(const float* dy, const float* x, float* dx, int64_t rows, int64_t cols, float eps,
                              void* stream) {
    if ((rows * cols) && (!dy || !x || !dx)) return fail(MLXHIP_ERR_NULL_PTR, "layernorm_vjp_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_LAYERNORM_VJP, dy, x, dx, rows, cols, eps, 0, as_stream(stream));
}

int mlxhip_rmsnorm_vjp_rows(const float* dy, const float* x, float* dx, int64_t rows, int64_t cols, float eps,
                            void* stream) {
    if ((rows * cols) && (!dy || !x || !dx)) return fail(MLXHIP_ERR_NULL_PTR, "rmsnorm_vjp_rows: null pointer");
    MLXHIP_TRY(ensure_device());
    return row_op(ROW_RMSNORM_VJP, dy, x, dx, rows, cols, eps, 0, as_stream(stream));
}

int mlxhip_ew_chain(const mlxhip_ew_instr_t* prog, size_t n_instr, const float* const* inputs, size_t n_inputs,
                    float* out, int64_t numel, void* stream) {
    if ((n_instr && !prog) || !inputs || (numel && !out)) return fail(MLXHIP_ERR_NULL_PTR, "ew_chain: null argument");
    MLXHIP_TRY(ensure_device());
    return ew_chain(prog, (int)n_instr, inputs, (int)n_inputs, out, numel, as_stream(stream));
}

int mlxhip_attention(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t tq,
                     int64_t tk, int64_t dh, float scale, int32_t causal, void* stream) {
    MLXHIP_TRY(ensure_device());
    if (batch < 0 || tq < 0 || tk < 0 || dh < 0)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: negative size");
    if (batch == 0 || tq == 0 || dh == 0) return MLXHIP_OK;
    if (!q || !k || !v || !o) return fail(MLXHIP_ERR_NULL_PTR, "attention: null operand");
    if (tk == 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention: no keys");
    return attention_fused(q, k, v, o, batch, tq, tk, dh, tq * dh, tk * dh, tk * dh, tq * dh, scale, causal,
                           as_stream(stream));
}

int mlxhip_attention_vjp(const float* q, const float* k, const float* v, const float* o, const float* dout,
                         float* dq, float* dk, float* dv, int64_t batch, int64_t t, int64_t dh, float scale,
                         int32_t causal, void* stream) {
    MLXHIP_TRY(ensure_device());
    if (batch < 0 || t < 0 || dh < 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "attention vjp: negative size");
    if (batch == 0 || t == 0 || dh == 0) return MLXHIP_OK;
    if (!q || !k || !v || !o || !dout || !dq || !dk || !dv)
        return fail(MLXHIP_ERR_NULL_PTR, "attention vjp: null operand");
    return attention_vjp(q, k, v, o, dout, dq, dk, dv, batch, t, dh, scale, causal, as_stream(stream));
}

int mlxhip_transpose2d(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
    if ((rows * cols) && (!x || !y)) return fail(MLXHIP_ERR_NULL_PTR, "transpose2d: null pointer");
    if (rows < 0 || cols < 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "transpose2d: negative size");
    MLXHIP_TRY(ensure_device());
    return transpose2d(x, y, rows, cols, as_stream(stream));
}

int mlxhip_cast(const void* x, int32_t src_dtype, void* y, int32_t dst_dtype, int64_t n, void* stream) {
    if (n && (!x || !y)) return fail(MLXHIP_ERR_NULL_PTR, "cast: null pointer");
    if (n < 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "cast: negative size");
    MLXHIP_TRY(ensure_device());
    return cast(x, src_dtype, y, dst_dtype, n, as_stream(stream));
}

mlxhip_event_t* mlxhip_event_create(void) {
    if (ensure_device() != MLXHIP_OK) return nullptr;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) {
        fail(MLXHIP_ERR_FFI_FAILED, "hipEventCreate failed");
        return nullptr;
    }
    return new mlxhip_event_t{e};
}

void mlxhip_event_destroy(mlxhip_event_t* e) {
    if (!e) return;
    (void)hipEventDestroy(e->ev);
    delete e;
}

int mlxhip_event_record(mlxhip_event_t* e, void* stream) {
    if (!e) return fail(MLXHIP_ERR_NULL_PTR, "event_record: null event");
    MLXHIP_HIP(hipEventRecord(e->ev, as_stream(stream)));
    return MLXHIP_OK;
}

int mlxhip_event_elapsed_ms(const mlxhip_event_t* start, const mlxhip_event_t* end, float* ms) {
    if (!start || !end || !ms) return fail(MLXHIP_ERR_NULL_PTR, "event_elapsed: null argument");
    MLXHIP_HIP(hipEventSynchronize(end->ev));
    MLXHIP_HIP(hipEventElapsedTime(ms, start->ev, end->ev));
    return MLXHIP_OK;
}

void* mlxhip_stream_create_hip(void) {
    if (ensure_device() != MLXHIP_OK) return nullptr;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        fail(MLXHIP_ERR_FFI_FAILED, "hipStreamCreate failed");
        return nullptr;
    }
    return s;
}

void mlxhip_stream_destroy_hip(void* stream) {
    if (!stream) return;
    // The stream's cached workspaces go back to the pool once its work ends.
    if (hipStreamSynchronize(as_stream(stream)) == hipSuccess) release_stream_workspaces(as_stream(stream));
    (void)hipGetLastError();
    (void)hipStreamDestroy(as_stream(stream));
}

struct mlxhip_graph_t {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int mlxhip_graph_begin(void* stream) {
    MLXHIP_TRY(ensure_device());
    if (!stream) return fail(MLXHIP_ERR_NULL_PTR, "graph_begin: the null stream cannot be recorded");
    MLXHIP_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
    return MLXHIP_OK;
}

mlxhip_graph_t* mlxhip_graph_end(void* stream) {
    if (!stream) {
        fail(MLXHIP_ERR_NULL_PTR, "graph_end: null stream");
        return nullptr;
    }
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(as_stream(stream), &g);
    if (e != hipSuccess || !g) {
        if (g) (void)hipGraphDestroy(g);
        hip_fail(e != hipSuccess ? e : hipErrorInvalidValue, "hipStreamEndCapture");
        return nullptr;
    }
    hipGraphExec_t x = nullptr;
    const hipError_t ei = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(g);
        hip_fail(ei, "hipGraphInstantiate");
        return nullptr;
    }
    return new mlxhip_graph_t{g, x};
}

int mlxhip_graph_launch(mlxhip_graph_t* g, void* stream) {
    if (!g) return fail(MLXHIP_ERR_NULL_PTR, "graph_launch: null graph");
    MLXHIP_HIP(hipGraphLaunch(g->exec, as_stream(stream)));
    return MLXHIP_OK;
}

void mlxhip_graph_free(mlxhip_graph_t* g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
}

}  // extern "C"
