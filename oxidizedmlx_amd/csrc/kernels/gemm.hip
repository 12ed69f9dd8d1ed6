// gemm.hip — host-side validation and dispatch of the MFMA GEMM
// (kernel in gemm_impl.hpp, instantiated per input dtype in gemm_{f32,bf16,f16}.hip).
#include "../common.hpp"
#include "../kernels.hpp"
#include "gemm_impl.hpp"
#include "gemm16_impl.hpp"

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace mlxhip {
namespace {

// The per-element helper kernels below walk [0, n) of one matrix with a
// grid-stride loop; elem_grid caps their x extent so no launch exceeds the
// 32-bit work-item count of a dispatch, whatever the matrix size.
#define FOR_EACH_ELEMENT(i, n) \
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (n); i += (int64_t)gridDim.x * 256)

dim3 elem_grid(int64_t n, int64_t batch) {
    return dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), int64_t(1) << 18), (unsigned)batch);
}

__global__ __launch_bounds__(256) void zero_c_kernel(char* c, int64_t ldc, int64_t sc, int64_t m,
                                                     int64_t n, int elem) {
    FOR_EACH_ELEMENT(f, m * n) {
        const int64_t r = f / n, col = f % n;
        char* p = c + ((int64_t)blockIdx.y * sc + r * ldc + col) * elem;
        for (int e = 0; e < elem; ++e) p[e] = 0;
    }
}

int elem_size(int dt) { return dt == MLXHIP_DTYPE_F32 ? 4 : 2; }

// Sum of the split-K partials in split order (deterministic), converted to C.
// ws holds batch * splits slices of [m, n] f32 with row pitch ldw, slice
// (b, s) at (b*splits+s)*m*ldw. Thread (row, 4-column group): a block holds
// RED_ROWS rows x RED_COLS groups, blockIdx.x enumerates (row block, column
// block) pairs and strides over the row blocks, blockIdx.y the batch. VEC: ldw and the partials are 16-byte aligned,
// so each split contributes one float4 load per thread.
constexpr int RED_COLS = 64;  // 4-column groups per row of work items
constexpr int RED_ROWS = 4;
constexpr int SPLIT_MAX = 8;  // every split plan uses at most 8 splits
template <int CT, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, void* c, int64_t m,
                                                            int64_t n, int64_t ldw, int64_t ldc, int64_t sc,
                                                            int splits, const float* __restrict__ bias, bool c_vec) {
    const int64_t b = blockIdx.y;
    const int64_t groups = (n + 3) / 4;
    const int gx = threadIdx.x % RED_COLS, gy = threadIdx.x / RED_COLS;
    const int64_t slice = m * ldw;
    // blockIdx.x = row block * col_blocks + column block: every thread owns
    // one 4-column group, so all of a thread's loads are in flight at once.
    const int64_t col_blocks = (groups + RED_COLS - 1) / RED_COLS;
    const int64_t rblocks = gridDim.x / col_blocks;
    const int64_t g = (blockIdx.x % col_blocks) * RED_COLS + gx;
    if (g >= groups) return;
    // A bias term (f32 C only): the thread's four columns, loaded once.
    float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias)
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = bias[std::min<int64_t>(4 * g + e, n - 1)];
    for (int64_t row = (int64_t)(blockIdx.x / col_blocks) * RED_ROWS + gy; row < m; row += rblocks * RED_ROWS) {
        const float* pr = ws + b * splits * slice + row * ldw;
        {
            const int64_t col = 4 * g;
            // Every split's values are loaded before the first add (one memory
            // latency, not one per split), then summed in split order.
            float v[SPLIT_MAX][4];
#pragma unroll
            for (int s = 0; s < SPLIT_MAX; ++s) {
                if (s >= splits) break;
                const float* p = pr + (int64_t)s * slice + col;
                if (VEC) {
                    const float4 t = *reinterpret_cast<const float4*>(p);
                    v[s][0] = t.x, v[s][1] = t.y, v[s][2] = t.z, v[s][3] = t.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[s][e] = p[std::min<int64_t>(e, n - 1 - col)];  // clamped, unguarded
                }
            }
            float acc[4] = {v[0][0], v[0][1], v[0][2], v[0][3]};
#pragma unroll
            for (int s = 1; s < SPLIT_MAX; ++s) {
                if (s >= splits) break;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] += v[s][e];
            }
            // The bias term: one f32 addition to the sum.
            if (bias)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] += bv[e];
            if (CT == MLXHIP_DTYPE_F32 && c_vec && col + 4 <= n) {
                // f32 C with 16-byte aligned rows: one 16-byte store.
                *reinterpret_cast<float4*>(static_cast<float*>(c) + b * sc + row * ldc + col) =
                    float4{acc[0], acc[1], acc[2], acc[3]};
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < n) gemm_detail::store_c<CT>(c, b * sc + row * ldc + col + e, acc[e]);
            }
        }
    }
}

int splitk_reduce(int c_dtype, const float* ws, void* c, int64_t m, int64_t n, int64_t ldw, int64_t ldc,
                  int64_t sc, int splits, int64_t batch, hipStream_t s, const float* bias = nullptr) {
    if (bias && c_dtype != MLXHIP_DTYPE_F32) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "splitk_reduce: bias needs f32 C");
    // VEC: every float4 read stays inside a row of the partials (ldw a
    // multiple of 4; reads past n up to ldw stay in the row padding).
    const bool vec = ldw % 4 == 0 && reinterpret_cast<uintptr_t>(ws) % 16 == 0 && ceil_div(n, 4) * 4 <= ldw;
    if (m == 0 || n == 0) return MLXHIP_OK;
    const int64_t col_blocks = ceil_div(ceil_div(n, 4), RED_COLS);
    if (col_blocks > (int64_t(1) << 22)) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "splitk_reduce: rows too long");
    const int64_t row_blocks = std::max<int64_t>(
        1, std::min<int64_t>({ceil_div(m, RED_ROWS), 65535, (int64_t(1) << 22) / col_blocks}));
    const dim3 grid((unsigned)(row_blocks * col_blocks), (unsigned)batch);
    // f32 C whose every row (and batch slice) starts 16-byte aligned.
    const bool c_vec = c_dtype == MLXHIP_DTYPE_F32 && reinterpret_cast<uintptr_t>(c) % 16 == 0 && ldc % 4 == 0 &&
                       (batch == 1 || sc % 4 == 0);
#define MLXHIP_RED(CT)                                                                                       \
    do {                                                                                                    \
        if (vec) hipLaunchKernelGGL((splitk_reduce_kernel<CT, true>), grid, dim3(256), 0, s, ws, c, m, n, ldw, \
                                    ldc, sc, splits, bias, c_vec);                                           \
        else hipLaunchKernelGGL((splitk_reduce_kernel<CT, false>), grid, dim3(256), 0, s, ws, c, m, n, ldw,    \
                                ldc, sc, splits, bias, c_vec);                                               \
    } while (0)
    switch (c_dtype) {
        case MLXHIP_DTYPE_F32: MLXHIP_RED(MLXHIP_DTYPE_F32); break;
        case MLXHIP_DTYPE_BF16: MLXHIP_RED(MLXHIP_DTYPE_BF16); break;
        default: MLXHIP_RED(MLXHIP_DTYPE_F16); break;
    }
#undef MLXHIP_RED
    return launch_check("splitk_reduce_kernel");
}

// C[i][j] += bias[j] over an f32 [m, n] C with row pitch ldc: the bias term
// of a product whose kernel has no bias in its store.
__global__ __launch_bounds__(256) void add_bias_kernel(float* __restrict__ c, int64_t m, int64_t n, int64_t ldc,
                                                       const float* __restrict__ bias) {
    const int64_t total = m * n;
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / n, j = i - r * n;
        c[r * ldc + j] += bias[j];
    }
}

int add_bias(float* c, int64_t m, int64_t n, int64_t ldc, const float* bias, hipStream_t s) {
    if (m == 0 || n == 0) return MLXHIP_OK;
    const int64_t blocks = std::min<int64_t>(ceil_div(m * n, 256), 4096);
    hipLaunchKernelGGL(add_bias_kernel, dim3((unsigned)blocks), dim3(256), 0, s, c, m, n, ldc, bias);
    return launch_check("add_bias_kernel");
}

// One operand to copy into a zero-padded rows_p x cols_p buffer per batch
// slice: dst[r][c] = src[r][c] for r < rows, c < cols, zero elsewhere.
struct PackOp {
    const void* src;
    int64_t ld, sstride, rows, cols;
    void* dst;
    int64_t rows_p, cols_p;
};
struct PackPair {
    PackOp op[2];
};

// One 16-byte chunk of a destination row: columns c0 .. c0 + CH - 1 of
// source row r, zero outside rows x cols. Every element is loaded, from a
// row and column clamped into range, before any is selected: a guarded load
// per element compiles to a branch that waits for its own load.
template <typename T, int CH>
__device__ inline uint4 pack_chunk(const T* sb, int64_t ld, int64_t rows, int64_t cols, int64_t r, int64_t c0) {
    union {
        uint4 v;
        T e[CH];
    } u;
    const T* src = sb + (r < rows ? r : rows - 1) * ld;
    T t[CH];
#pragma unroll
    for (int e = 0; e < CH; ++e) t[e] = src[c0 + e < cols ? c0 + e : cols - 1];
#pragma unroll
    for (int e = 0; e < CH; ++e) u.e[e] = (r < rows && c0 + e < cols) ? t[e] : T(0);
    return u.v;
}

// Both operands of one GEMM in one launch (blockIdx.z picks the operand,
// blockIdx.y the batch slice). Each thread writes one 16-byte chunk of a
// destination row (cols_p is a multiple of the chunk and the destination is
// 16-byte aligned); the source, whose rows need not be aligned, is read
// element by element. An empty source (no rows or no columns) packs zeros.
template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(PackPair pp) {
    constexpr int CH = 16 / sizeof(T);
    const PackOp& p = pp.op[blockIdx.z];
    const int64_t b = blockIdx.y;
    const bool empty = p.rows <= 0 || p.cols <= 0;
    const int chunks = (int)(p.cols_p / CH);  // per destination row (host-checked to fit 32 bits)
    const T* sb = static_cast<const T*>(p.src) + b * p.sstride;
    uint4* db = reinterpret_cast<uint4*>(static_cast<T*>(p.dst) + b * p.rows_p * p.cols_p);
    // Threads walk (row, chunk) pairs; rows advance by the grid's row count,
    // so no index needs a 64-bit division.
    const int per_block = 256 / chunks > 0 ? 256 / chunks : 1;       // whole rows per block when they fit
    const int t = threadIdx.x;
    if (chunks <= 256) {
        const int rloc = t / chunks, q = t - rloc * chunks;
        if (rloc >= per_block) return;
        for (int64_t r = (int64_t)blockIdx.x * per_block + rloc; r < p.rows_p; r += (int64_t)gridDim.x * per_block)
            db[r * chunks + q] = empty ? make_uint4(0, 0, 0, 0) : pack_chunk<T, CH>(sb, p.ld, p.rows, p.cols, r, q * CH);
    } else {
        for (int64_t r = blockIdx.x; r < p.rows_p; r += gridDim.x) {
            for (int q = t; q < chunks; q += 256)
                db[r * chunks + q] = empty ? make_uint4(0, 0, 0, 0) : pack_chunk<T, CH>(sb, p.ld, p.rows, p.cols, r, q * CH);
        }
    }
}

int pack2(int dt, const PackPair& pp, int64_t batch, hipStream_t s) {
    const int ch = dt == MLXHIP_DTYPE_F32 ? 4 : 8;
    int64_t blocks = 1;
    for (const PackOp& p : pp.op) {
        if (p.cols_p % ch || reinterpret_cast<uintptr_t>(p.dst) % 16)
            return fail(MLXHIP_ERR_INVALID_ARGUMENT, "pack: destination rows must be whole 16-byte chunks");
        const int64_t chunks = p.cols_p / ch;
        if (chunks > INT32_MAX) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "pack: rows too long");
        const int64_t per_block = chunks <= 256 ? 256 / chunks : 1;
        blocks = std::max(blocks, ceil_div(p.rows_p, per_block));
    }
    const dim3 grid((unsigned)std::min<int64_t>(blocks, int64_t(1) << 16), (unsigned)batch, 2);
    if (dt == MLXHIP_DTYPE_F32) hipLaunchKernelGGL(pack_kernel<uint32_t>, grid, dim3(256), 0, s, pp);
    else hipLaunchKernelGGL(pack_kernel<uint16_t>, grid, dim3(256), 0, s, pp);
    return launch_check("pack_kernel");
}

// MLXHIP_GEMM_PATH: unset/"auto" = choose by shape, "general" = always the
// general kernel, "lds16" = the direct-to-LDS 16-bit kernel whenever the
// operands allow it ("lds16_256" / "lds16_128": with that block size),
// "x6" = every f32 product through the split-f32 kernel, "small16" = every
// 16-bit product through the one-launch 64 x 64 kernel. Read on every call
// so one process (the tests) can cover every kernel.
int gemm_path() {
    const char* e = getenv("MLXHIP_GEMM_PATH");
    if (!e) return 0;
    if (!strcmp(e, "general")) return 1;
    if (!strcmp(e, "lds16")) return 2;
    if (!strcmp(e, "lds16_256")) return 3;
    if (!strcmp(e, "lds16_128")) return 4;
    if (!strcmp(e, "x6")) return 5;
    if (!strcmp(e, "small16")) return 6;
    return 0;
}

// MLXHIP_GEMM_GENERAL="wt,splits" forces the general kernel's block tile
// (64*wt, wt = 1, 2 or 4) and split-K factor (1..8) for aligned operands;
// unset = chosen by shape. Read on every call (tuning and tests).
bool general_override(int* wt, int* splits) {
    const char* e = getenv("MLXHIP_GEMM_GENERAL");
    int w = 0, sp = 0;
    if (!e || sscanf(e, "%d,%d", &w, &sp) != 2) return false;
    if (!(w == 1 || w == 2 || w == 4) || sp < 1 || sp > 8) return false;
    *wt = w;
    *splits = sp;
    return true;
}

}  // namespace

// ── Fixed device scratch of gemm_noalloc ─────────────────────────────────
// The split-K partials, the zero-padded operand copies and the split-f32
// planes of gemm_noalloc live in this array instead of stream-ordered
// allocations. Each device that
// loads the library holds its own copy until the process ends. In host code
// `scratch` names a host-side stand-in, never the device memory: the device
// address comes from hipGetSymbolAddress, once per device, and only that
// address reaches kernels.
static __device__ __align__(256) unsigned char scratch[GEMM_NOALLOC_SCRATCH_BYTES];

namespace {

// Bump allocator over one call's share of the fixed scratch (nullptr in the
// allocating path). Every region it hands out is written in full by the
// kernel that uses it before any kernel reads it (each split-K slice covers
// all of [m, n]; a packed copy writes its zero padding too, and so does the
// split into planes), so nothing is cleared between calls. The one word
// that is not (a split's non-finite flag) is compared with a number no
// earlier call used.
struct FixedScratch {
    char* base;
    size_t cap;
    size_t used;
};

// `bytes` of device workspace for this call: the stream's cached block of
// `slot` (fs == nullptr), or the next 256-byte aligned region of the fixed
// scratch.
int take_workspace(FixedScratch* fs, hipStream_t s, int slot, size_t bytes, void** out) {
    if (!fs) return stream_workspace(s, slot, bytes, out);
    const size_t at = (fs->used + 255) & ~size_t(255);
    if (at > fs->cap || bytes > fs->cap - at)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT,
                    "gemm_noalloc: this product needs %zu bytes of device scratch, more than the %zu bytes "
                    "of the fixed scratch (C is unchanged); use mlxhip_gemm",
                    at + bytes, fs->cap);
    *out = fs->base + at;
    fs->used = at + bytes;
    return MLXHIP_OK;
}

// Per device: the device address of `scratch` (null until resolved), and
// the stream of the last call outside graph capture with an event recorded
// after that call's kernels, so that a call on another stream can tell
// whether the scratch is still in use. g_scratch_mu is held for a whole
// call, from that check to the recording of its own event.
struct ScratchState {
    void* dev_ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool used = false;
};
std::mutex g_scratch_mu;
ScratchState g_scratch[64];

// The current device's scratch state, resolved on the first call on that
// device (with that device current): the symbol's device address and the
// event (no device memory is allocated). Caller holds g_scratch_mu.
int fixed_scratch_locked(ScratchState** out) {
    int dev = 0;
    MLXHIP_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm_noalloc: device %d", dev);
    ScratchState& st = g_scratch[dev];
    if (!st.dev_ptr) {
        void* p = nullptr;
        MLXHIP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(MLXHIP_ERR_FFI_FAILED, "gemm_noalloc: scratch has no device address");
        MLXHIP_HIP(hipEventCreateWithFlags(&st.done, hipEventDisableTiming));
        st.dev_ptr = p;
    }
    *out = &st;
    return MLXHIP_OK;
}

int gemm_impl(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
              int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
              int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s, bool padded,
              FixedScratch* fs, PlaneCache* cache = nullptr);

// Generation numbers of split-f32 products: each call's flag value.
std::atomic<uint32_t> g_x6_gen{0};

uint32_t next_x6_gen() {
    uint32_t g = 0;
    while (g == 0) g = ++g_x6_gen;
    return g;
}

// A plane block: three planes of `plane` elements, rounded up to 256 bytes,
// then the flag word (256 bytes of room).
constexpr size_t X6_FLAG_ROOM = 256;
size_t x6_planes_bytes(int64_t plane) { return ((size_t)(3 * plane * 2) + 255) & ~size_t(255); }

// f32 products through the bf16 planes (gemm16_x6.hip): `groups` products
// of one shape and layout (groups > 1: batch 1, one launch, product i in
// batch slot i). One launch (or one per five operands) splits the operands
// that `cache` does not already hold, one runs the plane products (and, when
// split over K, one sums the partials). Planes and partials come from the
// stream's workspaces, or from the fixed scratch (fs, no cache). Sets *ran =
// false, doing nothing, when the planes would not fit the kernel's 32-bit
// buffer offsets.
//
// Planes hold the operand as stored ([rows][cols] per batch slice) with both
// extents padded with zeros to multiples of 32, which serves it in either
// role and either orientation: K, whichever extent it is, becomes whole K
// tiles, and the padded M / N rows only feed C elements that are not stored.
int gemm_x6(int ta, int tb, int64_t m, int64_t n, int64_t k, int64_t batch, int groups, const float* const* a,
            int64_t lda, int64_t stride_a, const float* const* b, int64_t ldb, int64_t stride_b, float* const* c,
            int64_t ldc, int64_t stride_c, hipStream_t s, PlaneCache* cache, FixedScratch* fs, bool* ran,
            const float* const* bias = nullptr) {
    *ran = false;
    if (bias && batch != 1) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: a bias term needs batch 1");
    if (groups < 1 || groups > gemm16::Args::MAX_GROUPS || (groups > 1 && batch != 1))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: %d grouped products", groups);
    const int64_t kp = ceil_div(k, 32) * 32;  // segment length: whole K tiles
    // Operand 2i is product i's A, 2i + 1 its B.
    const int nops = 2 * groups;
    X6SplitOp op[2 * gemm16::Args::MAX_GROUPS];
    bool fresh[2 * gemm16::Args::MAX_GROUPS];
    int same_as[2 * gemm16::Args::MAX_GROUPS];  // an earlier operand with the same planes, or -1
    const int64_t lds[2] = {lda, ldb}, strides[2] = {stride_a, stride_b};
    const int64_t rows[2] = {ta ? k : m, tb ? n : k}, cols[2] = {ta ? m : k, tb ? k : n};
    for (int i = 0; i < nops; ++i) {
        const int r = i & 1;
        X6SplitOp& o = op[i];
        o = X6SplitOp{};
        o.src = r ? b[i / 2] : a[i / 2];
        o.ld = lds[r];
        o.stride = batch > 1 ? strides[r] : 0;
        o.rows = rows[r];
        o.cols = cols[r];
        o.rows_p = ceil_div(rows[r], 32) * 32;
        o.cols_p = ceil_div(cols[r], 32) * 32;
        o.plane = batch * o.rows_p * o.cols_p;
        o.chunks = o.plane / 8;
        // The descriptor of one slice spans two whole planes plus the slice.
        if (o.chunks >= ((int64_t)1 << 31) ||
            (2 * o.plane + o.rows_p * o.cols_p) * 2 >= (int64_t)gemm16::OOB - 4096)
            return MLXHIP_OK;
        fresh[i] = true;
        same_as[i] = -1;
        for (int j = 0; j < i; ++j)
            if (op[j].src == o.src && op[j].ld == o.ld && op[j].stride == o.stride && op[j].rows == o.rows &&
                op[j].cols == o.cols) {
                same_as[i] = j;
                fresh[i] = false;
                break;
            }
    }
    auto new_gen = [] { return next_x6_gen(); };
    const size_t flag_room = X6_FLAG_ROOM;
    auto plane_bytes = [](const X6SplitOp& o) { return x6_planes_bytes(o.plane); };
    auto copy_planes = [](X6SplitOp& to, const X6SplitOp& from) {
        to.dst = from.dst;
        to.flag = from.flag;
        to.gen = from.gen;
    };
    const int64_t slots = groups > 1 ? groups : batch;  // gridDim.y before splits

    // Block tile and split (measured on the config-4 shapes, split and
    // partial sums included): the interleaved kernel, whose 144 KiB of LDS
    // stages allow one workgroup per CU; 256x128 blocks when they alone come
    // to about one per CU (2048x4096x1024: 94 us, against 123 us for the
    // segment-by-segment kernel), else 128x128 blocks split over K to one
    // workgroup per CU (2048x1024x1024 split 2: 41 us against 54 us;
    // 1024x1024x2048 split 4: 42 us against 55 us; 4096x1024x2048 unsplit:
    // 104 us against 124 us). Grouped products count every group's tiles and
    // run unsplit. MLXHIP_X6="cfg,splits" forces them (tuning; cfg 0-2 the
    // segment-by-segment kernel with 256x256, 128x128 and 256x128 blocks,
    // 3-4 the interleaved one with 256x128 and 128x128).
    const int64_t wide_tiles = ceil_div(m, 256) * ceil_div(n, 128) * slots;
    const int64_t mid_tiles = ceil_div(m, 128) * ceil_div(n, 128) * slots;
    int cfg = 3, sp_k = 1;
    if (wide_tiles < 224) {
        cfg = 4;
        while (sp_k < 8 && mid_tiles * sp_k < 256 && kp / (2 * sp_k) >= 128) sp_k *= 2;
    }
    if (const char* e = getenv("MLXHIP_X6")) {
        int cf = 0, v = 0;
        if (sscanf(e, "%d,%d", &cf, &v) == 2 && cf >= 0 && cf <= 4 && v >= 1 && v <= 8) {
            cfg = cf;
            sp_k = v;
        }
    }
    if (groups > 1) {
        sp_k = 1;
        if (cfg < 3) cfg = 3;
    }
    if (slots * sp_k > 65535) sp_k = 1;
    // The f32 partials of a product split over K (sp_k > 1).
    const int64_t kspan = cfg >= 3 ? kp : gemm16::X6_SEGS * kp;
    const int64_t k_chunk = sp_k > 1 ? ceil_div(ceil_div(kspan, sp_k), 32) * 32 : 0;
    const int splits = sp_k > 1 ? (int)ceil_div(kspan, k_chunk) : 1;
    const int64_t ldw = ceil_div(n, 4) * 4;
    const size_t part_bytes = sp_k > 1 ? (size_t)(batch * splits * m * ldw) * sizeof(float) : 0;
    if (fs) {
        // Fixed scratch (gemm_noalloc): when the planes and partials do not
        // fit, the product runs on the direct f32 MFMA kernel instead, which
        // needs no planes (within the f32 bound, not bit-identical to the
        // split-f32 result).
        size_t need = 0;
        for (int i = 0; i < nops; ++i)
            if (fresh[i]) need += plane_bytes(op[i]) + flag_room;
        need = ((need + 255) & ~size_t(255)) + part_bytes + 256;
        const size_t used = (fs->used + 255) & ~size_t(255);
        if (used > fs->cap || need > fs->cap - used) return MLXHIP_OK;
    }
    if (cache && cache->alloc && !fs) {
        for (int i = 0; i < nops; ++i) {
            X6SplitOp& o = op[i];
            if (same_as[i] >= 0) {
                copy_planes(o, op[same_as[i]]);
                continue;
            }
            for (const PlaneCache::Entry& e : cache->entries)
                if (e.src == o.src && e.ld == o.ld && e.stride == o.stride && e.rows == o.rows && e.cols == o.cols &&
                    e.batch == batch) {
                    o.dst = e.planes;
                    o.flag = e.flag;
                    o.gen = e.gen;
                    fresh[i] = false;
                    break;
                }
            if (!fresh[i]) continue;
            const size_t pb = plane_bytes(o);
            char* blk = static_cast<char*>(cache->alloc(cache->ctx, pb + flag_room));
            if (!blk) return fail(MLXHIP_ERR_FFI_FAILED, "gemm: device allocation of %zu bytes failed", pb + flag_room);
            o.dst = reinterpret_cast<uint16_t*>(blk);
            o.flag = reinterpret_cast<uint32_t*>(blk + pb);
            o.gen = new_gen();
            cache->entries.push_back(PlaneCache::Entry{o.src, o.ld, o.stride, o.rows, o.cols, batch, o.dst, o.flag,
                                                       o.gen});
        }
    } else {
        size_t total = 0;
        for (int i = 0; i < nops; ++i)
            if (fresh[i]) total += plane_bytes(op[i]) + flag_room;
        void* ws = nullptr;
        MLXHIP_TRY(take_workspace(fs, s, WS_PACK, total, &ws));
        char* at = static_cast<char*>(ws);
        for (int i = 0; i < nops; ++i) {
            X6SplitOp& o = op[i];
            if (!fresh[i]) {
                copy_planes(o, op[same_as[i]]);
                continue;
            }
            const size_t pb = plane_bytes(o);
            o.dst = reinterpret_cast<uint16_t*>(at);
            o.flag = reinterpret_cast<uint32_t*>(at + pb);
            o.gen = new_gen();
            at += pb + flag_room;
        }
    }

    gemm16::Args h{};
    const X6SplitOp &oa = op[0], &ob = op[1];
    h.m = m;
    h.n = n;
    h.k = kp;
    h.a = oa.dst;
    h.lda = oa.cols_p;
    h.sa = oa.rows_p * oa.cols_p;
    h.b = ob.dst;
    h.ldb = ob.cols_p;
    h.sb = ob.rows_p * ob.cols_p;
    h.c = c[0];
    h.ldc = ldc;
    h.sc = stride_c;
    h.a_bytes = (uint32_t)((2 * oa.plane + h.sa) * 2);
    h.b_bytes = (uint32_t)((2 * ob.plane + h.sb) * 2);
    h.plane_a = (uint32_t)(oa.plane * 2);
    h.plane_b = (uint32_t)(ob.plane * 2);
    h.fa = a[0];
    h.flda = lda;
    h.fsa = stride_a;
    h.fb = b[0];
    h.fldb = ldb;
    h.fsb = stride_b;
    h.fk = k;
    h.flag_a = oa.flag;
    h.gen_a = oa.gen;
    h.flag_b = ob.flag;
    h.gen_b = ob.gen;
    if (groups > 1) {
        h.groups = groups;
        for (int i = 0; i < groups; ++i) {
            const X6SplitOp &ga = op[2 * i], &gb = op[2 * i + 1];
            h.grp[i] = gemm16::Args::Group{ga.dst, gb.dst, c[i], a[i], b[i], ga.flag, gb.flag, ga.gen, gb.gen,
                                           bias ? bias[i] : nullptr};
        }
    }

    X6SplitPair sp{};
    for (int i = 0; i < nops; ++i) {
        if (!fresh[i]) continue;
        sp.op[sp.n++] = op[i];
        if (sp.n == X6SplitPair::MAX) {
            MLXHIP_TRY(x6_split(sp, s));
            sp.n = 0;
        }
    }
    if (sp.n) MLXHIP_TRY(x6_split(sp, s));
    if (sp_k == 1) {
        // The interleaved kernel adds the bias as it stores C; the other one
        // (a forced setting) leaves it to one more launch per product.
        if (bias && cfg >= 3) h.bias = bias[0];
        MLXHIP_TRY(gemm16_x6(ta, tb, h, slots, cfg, s));
        if (bias && cfg < 3)
            for (int i = 0; i < groups; ++i) MLXHIP_TRY(add_bias(c[i], m, n, ldc, bias[i], s));
        *ran = true;
        return MLXHIP_OK;
    }
    // The interleaved kernel (cfg 3 / 4) runs all six products per K tile:
    // its splits divide the planes' K, the other kernel's the 6 segments.
    h.k_chunk = k_chunk;
    h.splits = splits;
    void* part = nullptr;
    MLXHIP_TRY(take_workspace(fs, s, WS_SPLITK, part_bytes, &part));
    h.c = part;
    h.ldc = ldw;
    h.sc = m * ldw;
    MLXHIP_TRY(gemm16_x6(ta, tb, h, batch, cfg, s));
    MLXHIP_TRY(splitk_reduce(MLXHIP_DTYPE_F32, static_cast<const float*>(part), c[0], m, n, ldw, ldc, stride_c,
                             h.splits, batch, s, bias ? bias[0] : nullptr));
    *ran = true;
    return MLXHIP_OK;
}

// Whether an f32 product goes through the split-f32 kernel (path 0: by
// shape).
bool use_x6(int path, int64_t m, int64_t n, int64_t k, int64_t batch) {
    if (path == 5) return true;
    if (path != 0) return false;
    return m >= 256 && n >= 256 && k >= 256 && (double)m * (double)n * (double)k * (double)batch >= 2147483648.0;
}
}  // namespace

bool gemm_f32_reads_planes(int64_t m, int64_t n, int64_t k, int64_t batch) {
    const int path = gemm_path();
    return (path == 0 || path == 5) && use_x6(path, m, n, k, batch);
}

int x6_plane_block(PlaneCache* cache, const void* src, int64_t rows, int64_t cols, int64_t batch, uint16_t** planes,
                   uint32_t** flag, uint32_t* gen) {
    *planes = nullptr;
    if (!cache || !cache->alloc || rows % 32 || cols % 32 || rows <= 0 || cols <= 0 || batch <= 0) return MLXHIP_OK;
    const int64_t plane = batch * rows * cols;
    const size_t pb = x6_planes_bytes(plane);
    char* blk = static_cast<char*>(cache->alloc(cache->ctx, pb + X6_FLAG_ROOM));
    if (!blk) return fail(MLXHIP_ERR_FFI_FAILED, "gemm: device allocation of %zu bytes failed", pb + X6_FLAG_ROOM);
    *planes = reinterpret_cast<uint16_t*>(blk);
    *flag = reinterpret_cast<uint32_t*>(blk + pb);
    *gen = next_x6_gen();
    cache->entries.push_back(PlaneCache::Entry{src, cols, batch > 1 ? rows * cols : 0, rows, cols, batch, *planes,
                                               *flag, *gen});
    return MLXHIP_OK;
}

// MLXHIP_GEMM_GROUPS=0 turns grouping off (each product its own launch;
// read on every call, for comparisons).
bool gemm_f32_groupable(int64_t m, int64_t n, int64_t k) {
    const char* e = getenv("MLXHIP_GEMM_GROUPS");
    if (e && !strcmp(e, "0")) return false;
    const int path = gemm_path();
    return (path == 0 || path == 5) && use_x6(path, m, n, k, 1);
}

int gemm_f32_grouped(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, int groups, const float* const* a,
                     int64_t lda, const float* const* b, int64_t ldb, float* const* c, int64_t ldc, hipStream_t s,
                     PlaneCache* planes, const float* const* bias) {
    if (groups < 1 || groups > gemm16::Args::MAX_GROUPS)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: %d grouped products", groups);
    if (m < 0 || n < 0 || k < 0) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: negative size");
    for (int i = 0; i < groups; ++i)
        if (!a[i] || !b[i] || !c[i]) return fail(MLXHIP_ERR_NULL_PTR, "gemm: null operand in group %d", i);
    if (ldc < n || lda < (trans_a ? m : k) || ldb < (trans_b ? k : n))
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: leading dimension too small");
    // One launch only when the products' tiles together fill the chip
    // unsplit (224+ tiles of 256x128 or 256+ of 128x128): two 1024x1024x2048
    // weight gradients grouped (128 workgroups over K 2048) took 79 us,
    // against 35 us each split over K.
    const bool fills = ceil_div(m, 256) * ceil_div(n, 128) * groups >= 224 ||
                       ceil_div(m, 128) * ceil_div(n, 128) * groups >= 256;
    if (groups > 1 && fills && m > 0 && n > 0 && k > 0 && gemm_f32_groupable(m, n, k)) {
        bool ran = false;
        MLXHIP_TRY(gemm_x6(trans_a, trans_b, m, n, k, 1, groups, a, lda, 0, b, ldb, 0, c, ldc, 0, s, planes, nullptr,
                           &ran, bias));
        if (ran) return MLXHIP_OK;
    }
    for (int i = 0; i < groups; ++i)
        MLXHIP_TRY(gemm(MLXHIP_DTYPE_F32, MLXHIP_DTYPE_F32, trans_a, trans_b, m, n, k, 1, a[i], lda, 0, b[i], ldb, 0,
                        c[i], ldc, 0, s, planes, bias ? bias[i] : nullptr));
    return MLXHIP_OK;
}

int gemm(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
         int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
         int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s, PlaneCache* planes,
         const float* bias) {
    if (!bias)
        return gemm_impl(ab_dtype, c_dtype, trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, c,
                         ldc, stride_c, s, false, nullptr, planes);
    // C = op(A) op(B) + bias (row broadcast): the split-f32 kernel adds it as
    // it stores C (or its split-K sum does); any other path, one more launch.
    if (ab_dtype != MLXHIP_DTYPE_F32 || c_dtype != MLXHIP_DTYPE_F32 || batch != 1)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: a bias term needs f32 operands and C, batch 1");
    if (m > 0 && n > 0 && k > 0 && a && b && c && ldc >= n && lda >= (trans_a ? m : k) &&
        ldb >= (trans_b ? k : n) && use_x6(gemm_path(), m, n, k, 1)) {
        bool ran = false;
        const float* fa = static_cast<const float*>(a);
        const float* fb = static_cast<const float*>(b);
        float* fc = static_cast<float*>(c);
        MLXHIP_TRY(gemm_x6(trans_a, trans_b, m, n, k, 1, 1, &fa, lda, stride_a, &fb, ldb, stride_b, &fc, ldc, stride_c,
                           s, planes, nullptr, &ran, &bias));
        if (ran) return MLXHIP_OK;
    }
    MLXHIP_TRY(gemm_impl(ab_dtype, c_dtype, trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, c,
                         ldc, stride_c, s, false, nullptr, planes));
    return add_bias(static_cast<float*>(c), m, n, ldc, bias, s);
}

int gemm_noalloc(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                 int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
                 int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    ScratchState* st = nullptr;
    MLXHIP_TRY(fixed_scratch_locked(&st));
    // Overlapping calls share the scratch. A call on another stream than
    // the last one while the last one's kernels may still run is refused
    // (work on one stream runs in order, so same-stream calls never
    // overlap). Under graph capture the order of the replays is not known
    // here, so nothing is checked or recorded.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    MLXHIP_HIP(hipStreamIsCapturing(s, &cap));
    const bool capturing = cap != hipStreamCaptureStatusNone;
    if (!capturing && st->used && st->last != s) {
        const hipError_t q = hipEventQuery(st->done);
        if (q == hipErrorNotReady)
            return fail(MLXHIP_ERR_INVALID_ARGUMENT,
                        "gemm_noalloc: the fixed scratch is still in use by a call on another stream; calls that "
                        "may overlap on one device must be serialised (C is unchanged)");
        if (q != hipSuccess) return hip_fail(q, "hipEventQuery");
    }
    FixedScratch fs{static_cast<char*>(st->dev_ptr), GEMM_NOALLOC_SCRATCH_BYTES, 0};
    const int rc = gemm_impl(ab_dtype, c_dtype, trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb,
                             stride_b, c, ldc, stride_c, s, false, &fs);
    if (!capturing) {
        // Recorded whatever rc says: kernels enqueued before a failure
        // still use the scratch.
        MLXHIP_HIP(hipEventRecord(st->done, s));
        st->last = s;
        st->used = true;
    }
    return rc;
}

namespace {
// padded: the operands are the dispatcher's zero-padded copies (rows
// readable up to their leading dimension). fs: the fixed scratch of
// gemm_noalloc, or nullptr to take workspace from the device's pool.
int gemm_impl(int ab_dtype, int c_dtype, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
              int64_t batch, const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
              int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, hipStream_t s, bool padded,
              FixedScratch* fs, PlaneCache* cache) {
    if (ab_dtype != MLXHIP_DTYPE_F32 && ab_dtype != MLXHIP_DTYPE_BF16 && ab_dtype != MLXHIP_DTYPE_F16)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: input dtype %d unsupported", ab_dtype);
    if (c_dtype != MLXHIP_DTYPE_F32 && c_dtype != MLXHIP_DTYPE_BF16 && c_dtype != MLXHIP_DTYPE_F16)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: output dtype %d unsupported", c_dtype);
    if (m < 0 || n < 0 || k < 0 || batch < 0)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: negative size");
    if (m == 0 || n == 0 || batch == 0) return MLXHIP_OK;
    if (!c) return fail(MLXHIP_ERR_NULL_PTR, "gemm: C is null");
    if (ldc < n) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: ldc %lld < n %lld", (long long)ldc, (long long)n);
    if (batch > 65535) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: batch %lld > 65535", (long long)batch);
    if (k == 0) {
        const dim3 grid = elem_grid(m * n, batch);
        hipLaunchKernelGGL(zero_c_kernel, grid, dim3(256), 0, s, static_cast<char*>(c), ldc, stride_c,
                           m, n, elem_size(c_dtype));
        return launch_check("zero_c_kernel");
    }
    if (!a || !b) return fail(MLXHIP_ERR_NULL_PTR, "gemm: A or B is null");
    const int64_t a_cols = trans_a ? m : k, b_cols = trans_b ? k : n;
    if (lda < a_cols) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: lda %lld < %lld", (long long)lda, (long long)a_cols);
    if (ldb < b_cols) return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: ldb %lld < %lld", (long long)ldb, (long long)b_cols);
    if (ceil_div(m, 64) * ceil_div(n, 64) > INT32_MAX)
        return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: too many tiles");

    // Large f32 products: bf16 planes on the 16-bit matrix cores.
    if (ab_dtype == MLXHIP_DTYPE_F32 && c_dtype == MLXHIP_DTYPE_F32 && !padded &&
        use_x6(gemm_path(), m, n, k, batch)) {
        bool ran = false;
        const float* fa = static_cast<const float*>(a);
        const float* fb = static_cast<const float*>(b);
        float* fc = static_cast<float*>(c);
        MLXHIP_TRY(gemm_x6(trans_a, trans_b, m, n, k, batch, 1, &fa, lda, stride_a, &fb, ldb, stride_b, &fc, ldc,
                           stride_c, s, cache, fs, &ran));
        if (ran) return MLXHIP_OK;
    }

    // Small f32 products (config 1's 512^3): one launch of 32 x 32 tiles with
    // K split across the workgroup's waves, instead of split-K partials and
    // a reduction (measured 13.7 us per call for 512^3 that way, kernels
    // and launches included).
    if (ab_dtype == MLXHIP_DTYPE_F32 && c_dtype == MLXHIP_DTYPE_F32 && gemm_path() == 0 &&
        ceil_div(m, 64) * ceil_div(n, 64) * batch < 256 &&
        gemm_small_f32_fits(m, n, k, batch, lda, ldb, trans_a, trans_b))
        return gemm_small_f32(trans_a, trans_b, m, n, k, batch, static_cast<const float*>(a), lda, stride_a,
                              static_cast<const float*>(b), ldb, stride_b, static_cast<float*>(c), ldc, stride_c, s);

    // Many f32 products of attention over heads: short-K scores (C = A B^T,
    // bound by writing C) and head-dimension outputs (N = 64, bound by
    // reading A).
    if (ab_dtype == MLXHIP_DTYPE_F32 && c_dtype == MLXHIP_DTYPE_F32 && gemm_path() == 0 &&
        gemm_thin_f32_fits(trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c))
        return gemm_thin_f32(trans_a, trans_b, m, n, k, batch, static_cast<const float*>(a), lda, stride_a,
                             static_cast<const float*>(b), ldb, stride_b, static_cast<float*>(c), ldc, stride_c, s);

    const int ch = 16 / elem_size(ab_dtype);
    const bool aligned = reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(b) % 16 == 0 && lda % ch == 0 &&
                         ldb % ch == 0 && (batch == 1 || (stride_a % ch == 0 && stride_b % ch == 0));
    const int path = gemm_path();
    // 16-bit products the direct-to-LDS kernel cannot read as they are
    // (rows that are not whole 16-byte chunks) or that have too few 128 x 128
    // tiles to fill the chip: one launch of 64 x 64 tiles, no packed copies,
    // no K split. The odd 1000 x 777 x 1531 bf16 product: pack + split GEMM +
    // partial sums took ~25 us per call (three launches).
    if (ab_dtype != MLXHIP_DTYPE_F32 && (path == 6 || path == 0) && !padded &&
        gemm16_small_fits(m, n, k, batch, lda, ldb, trans_a, trans_b)) {
        const int64_t big_tiles = ceil_div(m, 256) * ceil_div(n, 256) * batch;
        const int64_t mid_tiles = ceil_div(m, 128) * ceil_div(n, 128) * batch;
        if (path == 6 || (big_tiles < 128 && (!aligned || mid_tiles < 16)))
            return gemm16_small(ab_dtype, c_dtype, trans_a, trans_b, m, n, k, batch, a, lda, stride_a, b, ldb,
                                stride_b, c, ldc, stride_c, s);
    }
    if (!aligned && path != 1) {
        // Unaligned operands (odd leading dimension, offset pointer): copy both
        // into zero-padded buffers whose rows are whole 16-byte chunks (K and
        // the contiguous extents rounded up to a multiple of 16 bytes) and run
        // the aligned kernels on those. The zero padding adds nothing to C.
        const int64_t kp = ceil_div(k, ch) * ch;
        const int64_t a_rows = trans_a ? k : m, a_cols = trans_a ? m : k;
        const int64_t a_rows_p = trans_a ? kp : m, a_cols_p = ceil_div(a_cols, ch) * ch;
        const int64_t b_rows = trans_b ? n : k, b_cols = trans_b ? k : n;
        const int64_t b_rows_p = trans_b ? n : kp, b_cols_p = ceil_div(b_cols, ch) * ch;
        const int es = elem_size(ab_dtype);
        // One stream-ordered allocation holds both copies (B at a 256-byte
        // boundary) and one launch fills both: the host work per call is
        // what such small products wait on.
        const size_t a_sz = (size_t)(a_rows_p * a_cols_p * batch * es);
        const size_t b_off = (a_sz + 255) & ~size_t(255);
        void* pa = nullptr;
        MLXHIP_TRY(take_workspace(fs, s, WS_PACK, b_off + (size_t)(b_rows_p * b_cols_p * batch * es), &pa));
        void* pb = static_cast<char*>(pa) + b_off;
        PackPair pp{{PackOp{a, lda, stride_a, a_rows, a_cols, pa, a_rows_p, a_cols_p},
                     PackOp{b, ldb, stride_b, b_rows, b_cols, pb, b_rows_p, b_cols_p}}};
        MLXHIP_TRY(pack2(ab_dtype, pp, batch, s));
        return gemm_impl(ab_dtype, c_dtype, trans_a, trans_b, m, n, kp, batch, pa, a_cols_p, a_rows_p * a_cols_p,
                         pb, b_cols_p, b_rows_p * b_cols_p, c, ldc, stride_c, s, true, fs);
    }

    gemm_detail::GemmArgs g{};
    g.m = m;
    g.n = n;
    g.k = k;
    g.a = a;
    g.lda = lda;
    g.sa = stride_a;
    g.b = b;
    g.ldb = ldb;
    g.sb = stride_b;
    g.c = c;
    g.ldc = ldc;
    g.sc = stride_c;
    const int ta = trans_a ? 1 : 0, tb = trans_b ? 1 : 0;
    // 16-bit operands go to the direct-to-LDS kernel when the operands meet
    // its layout requirements: 256x256 blocks from 128 tiles (one workgroup
    // per CU, so at least half the CUs busy), else 128x128 blocks (two per
    // CU) from 16 tiles. Even a partly idle chip runs it faster than the
    // general kernel split over K: the 1000x777x1531 bf16 product (56 tiles
    // of 128x128) took 41.6 us per call against 60-88 us (measured on
    // MI355X, operand packing and host work included). The general kernel
    // covers everything else.
    if (ab_dtype != MLXHIP_DTYPE_F32 && path != 1) {
        const int64_t big_tiles = ceil_div(m, 256) * ceil_div(n, 256) * batch;
        const int64_t mid_tiles = ceil_div(m, 128) * ceil_div(n, 128) * batch;
        const int cfg = path == 3 ? 0 : path == 4 ? 1 : big_tiles >= 128 ? 0 : 1;
        gemm16::Args h{};
        if ((path >= 2 || big_tiles >= 128 || mid_tiles >= 16) &&
            gemm16::supported(ta, tb, m, n, k, batch, a, lda, stride_a, b, ldb, stride_b, &h.a_bytes,
                              &h.b_bytes, padded)) {
            h.m = m;
            h.n = n;
            h.k = k;
            h.a = a;
            h.lda = lda;
            h.sa = stride_a;
            h.b = b;
            h.ldb = ldb;
            h.sb = stride_b;
            h.c = c;
            h.ldc = ldc;
            h.sc = stride_c;
            // Split over K when 128x128 tiles leave most CUs idle: the
            // smallest power of two giving one workgroup per CU, at most 8,
            // keeping at least 256 k (8 K tiles) per split. The 1000 x 777 x
            // 1531 product (56 tiles) runs 4 splits of 384 k on 224 CUs.
            int sp = 1;
            if (cfg == 1 && path == 0)
                while (sp < 8 && mid_tiles * sp < 256 && k / (2 * sp) >= 256) sp *= 2;
            // MLXHIP_GEMM16_SPLITS=s forces the split factor (1..8; tuning).
            if (const char* e = getenv("MLXHIP_GEMM16_SPLITS")) {
                const int v = atoi(e);
                if (v >= 1 && v <= 8) sp = v;
            }
            if (sp == 1)
                return ab_dtype == MLXHIP_DTYPE_BF16 ? gemm16_bf16(c_dtype, ta, tb, h, batch, cfg, s)
                                                     : gemm16_f16(c_dtype, ta, tb, h, batch, cfg, s);
            // f32 partials [batch][split][m][ldw] (rows padded to 16 bytes for
            // the vector stores), summed in split order into C.
            h.k_chunk = ceil_div(ceil_div(k, sp), 32) * 32;
            h.splits = (int)ceil_div(k, h.k_chunk);
            const int64_t ldw = ceil_div(n, 4) * 4;
            void* part = nullptr;
            MLXHIP_TRY(take_workspace(fs, s, WS_SPLITK, (size_t)(batch * h.splits * m * ldw) * sizeof(float), &part));
            h.c = part;
            h.ldc = ldw;
            h.sc = m * ldw;
            MLXHIP_TRY(ab_dtype == MLXHIP_DTYPE_BF16 ? gemm16_bf16(MLXHIP_DTYPE_F32, ta, tb, h, batch, cfg, s)
                                                     : gemm16_f16(MLXHIP_DTYPE_F32, ta, tb, h, batch, cfg, s));
            return splitk_reduce(c_dtype, static_cast<const float*>(part), c, m, n, ldw, ldc, stride_c, h.splits,
                                 batch, s);
        }
    }
    // General kernel. f32 operands (measured on MI355X): 256x256 blocks from
    // 256 tiles (one per CU); otherwise 128x128 blocks split over K by the
    // smallest power of two that gives at least 512 workgroups (two per CU),
    // keeping at least 256 k per split; below 64 such tiles, 64x64 blocks as for 16-bit operands.
    // 16-bit operands that reach this kernel (too small or unaligned for the
    // direct-to-LDS one): the largest block tile that still gives about one
    // workgroup per CU; below that 64x64 tiles, split over K until there are
    // about four workgroups per CU (the general kernel prefetches one K tile
    // ahead, so small tiles need several resident workgroups to hide load
    // latency), keeping at least four K tiles per split. The f32 partials are
    // summed in a fixed order (deterministic) by a second kernel.
    const int bk = ab_dtype == MLXHIP_DTYPE_F32 ? 32 : 64;
    auto tiles = [&](int w) { return ceil_div(m, 64 * w) * ceil_div(n, 64 * w) * batch; };
    auto limit = [&](int64_t sp) { return (int)(batch * sp > 65535 ? 1 : std::max<int64_t>(1, sp)); };
    // Fraction of the padded block tiles that holds C: a 128-wide tile over
    // N = 64 does twice the MFMA work it keeps.
    auto fill = [&](int w) {
        const int64_t e = 64 * w;
        return (double)(m * n) / ((double)(ceil_div(m, e) * e) * (double)(ceil_div(n, e) * e));
    };
    int wt = 2, splits = 1;
    if (ab_dtype == MLXHIP_DTYPE_F32 && tiles(4) >= 256 && fill(4) >= 0.75) {
        wt = 4;
    } else if (ab_dtype == MLXHIP_DTYPE_F32 && aligned && fill(2) < 0.75 && tiles(1) >= 256) {
        // Narrow products (config 4's 64 heads of P·V, [512, 512] x [512, 64]:
        // 34 us with 64x64 blocks against 56 us with 128x128 blocks split 2).
        wt = 1;
        int64_t want = 1;
        while (want < 8 && want * tiles(1) < 512) want *= 2;
        splits = limit(std::min<int64_t>(want, k / 256));
    } else if (ab_dtype == MLXHIP_DTYPE_F32 && tiles(2) >= 64 && aligned) {
        // A power of two: 192 tiles split 3 ways make 576 workgroups, one
        // round of 512 plus a tail of 64 (qkv dW of config 4 took ~40 % longer
        // than split 4 ways).
        int64_t want = 1;
        while (want < 8 && want * tiles(2) < 512) want *= 2;
        splits = limit(std::min<int64_t>(want, k / 256));
        if (tiles(2) * splits < 256) {
            // K too short to split far enough: fewer workgroups than CUs.
            // 64x64 blocks give four times as many (1024x1024x256: 12.9 us
            // against 25.6 us).
            wt = 1;
            splits = 1;
        }
    } else if (ab_dtype != MLXHIP_DTYPE_F32 && tiles(4) >= 240) {
        wt = 4;
    } else if (tiles(2) < 200) {
        wt = 1;
        const int64_t t = tiles(1);
        if (t < 768 && aligned) {
            const int64_t by_cus = std::max<int64_t>(1, 1024 / t);
            const int64_t by_k = k / (4 * bk);  // at least 4 K tiles per split
            splits = limit(std::min<int64_t>(8, std::min(by_cus, by_k)));
        }
    }
    if (aligned) {
        int w = 0, sp = 0;
        if (general_override(&w, &sp)) {
            wt = w;
            splits = limit(std::min<int64_t>(sp, ceil_div(k, bk)));
        }
    }
    auto run = [&](const gemm_detail::GemmArgs& ga, int ct) {
        switch (ab_dtype) {
            case MLXHIP_DTYPE_F32: return gemm_f32(ct, ta, tb, ga, batch, aligned, wt, s);
            case MLXHIP_DTYPE_BF16: return gemm_bf16(ct, ta, tb, ga, batch, aligned, wt, s);
            default: return gemm_f16(ct, ta, tb, ga, batch, aligned, wt, s);
        }
    };
    if (splits == 1) return run(g, c_dtype);
    g.k_chunk = ceil_div(ceil_div(k, splits), bk) * bk;
    g.splits = (int)ceil_div(k, g.k_chunk);
    void* part = nullptr;
    MLXHIP_TRY(take_workspace(fs, s, WS_SPLITK, (size_t)(batch * g.splits * m * n) * sizeof(float), &part));
    g.ws = static_cast<float*>(part);
    // Partials, then their sum in split order (deterministic). (Reducing in
    // the GEMM kernel's last workgroup per tile needs a device-scope release
    // per workgroup, which on this part writes back the whole L2 of the XCD:
    // measured 4-6x slower.)
    MLXHIP_TRY(run(g, c_dtype));
    return splitk_reduce(c_dtype, static_cast<const float*>(part), c, m, n, n, ldc, stride_c, g.splits, batch, s);
}
}  // namespace

}  // namespace mlxhip
