// Host side of the MI355X decode hot path: context, HBM weight store,
// resident layouts, and the C ABI declared in include/wohper_hip.h.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "libm_tables.inc"
#define WH_LIBM_TABLES_INCLUDED 1
#include "kernels.h"
#include "mhc.h"
#include "mla.h"
#include "moe_batch.h"
#include "moe_px.h"
#include "moe_tok.h"
#include "fp8_mm.h"
#include "fp8_tol.h"
#include "fp8_multi.h"
#include "moe_bmx.h"
#include "probe.h"
#include "quant_block.h"
#include "router.h"
#include "wohper_hip.h"

// Working memory of wh_routed_and_shared_experts_noalloc_async: one array on
// every GPU the library runs on, held until the process ends.  In host code
// this name is a stand-in for the device symbol, not a device address: the
// address on each GPU comes from hipGetSymbolAddress (noalloc_setup).
static __device__ __align__(256) uint8_t noalloc_scratch[WH_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kFp8 = 1, kFp4 = 2;

// Device address of noalloc_scratch on each GPU (null until wh_init ran on
// it with that GPU current).
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};

struct Tensor {
    int kind = 0;
    uint8_t* w = nullptr;  // device
    void* s = nullptr;     // device scales
    size_t rows = 0, cols = 0, scale_rows = 0, scale_cols = 0;
    int scale_fmt = WH_SCALE_UE8M0;
    bool fast = false;     // resident lane layout (else original row-major)
    bool special = false;  // FP8 codes 0x7F/0xFF present
    bool zero_scale = false;  // FP4: some UE8M0 scale byte is 0 (the MFMA kernels would read it as 2^-127)
    size_t bytes = 0;
    size_t w_alloc = 0, s_alloc = 0;  // arena bytes behind w and s
};

struct Expert {
    wh_tensor w1 = 0, w3 = 0, w2 = 0;
    bool owned = false;  // tensors created by a block store, released on replacement
};

// Outcome of one of the reference's router tensor lookups, kept for the
// route calls that would run it (the reference repeats the lookup per call).
struct LookupError {
    int status = WH_OK;
    std::string text;  // wh_last_error text when status != WH_OK
};

// A layer's router: the tensors route_experts_from_dense_block reads
// (E/compute.rs:2129-2237), resident.
struct Router {
    int gate = 0;                 // kGateBf16 (lane layout), kGateBf16Rows (row-major), kGateFp8
    uint16_t* bf16 = nullptr;     // device bf16 gate
    wh_tensor fp8 = 0;            // FP8 gate in the weight store
    size_t rows = 0, cols = 0;
    float* bias = nullptr;        // device f32 selection bias [rows], or null
    LookupError bias_err;         // router_bias_values failed (raised in sqrt-softplus math)
    bool has_table = false;       // a tid2eid table exists (hash layers)
    LookupError table_err;        // router_tid2eid_tensor failed (raised when hashing)
    int table_dtype = 0;          // dtype_original of the table
    size_t table_rows = 0, table_cols = 0;
    std::vector<uint8_t> table;   // its bytes, host side: one row is read per call
};
constexpr int kGateBf16 = 1, kGateBf16Rows = 2, kGateFp8 = 3;

// HBM of the weight store: large hipMalloc chunks (a 150 GB stack would
// otherwise need ~10^5 separate allocations), sub-allocated in 256-byte
// units.  Released ranges go back to a free list - best fit, split, merged
// with free neighbours of the same chunk - so replacing experts, or storing
// and releasing transient tensors, reuses the same bytes.
struct Arena {
    struct Range {
        size_t size;
        uint32_t chunk;
    };
    std::vector<void*> chunks;
    std::map<uintptr_t, Range> free_at;            // start -> free range
    std::multimap<size_t, uintptr_t> free_sizes;   // size -> start
    size_t total = 0;  // bytes of all chunks
    size_t live = 0;   // bytes handed out
    static constexpr size_t kChunk = size_t(4) << 30;

    static size_t round(size_t n) { return (n + 255) & ~size_t(255); }

    void insert(uintptr_t p, Range r) {
        free_at[p] = r;
        free_sizes.emplace(r.size, p);
    }
    void erase(std::map<uintptr_t, Range>::iterator it) {
        auto rng = free_sizes.equal_range(it->second.size);
        for (auto s = rng.first; s != rng.second; ++s)
            if (s->second == it->first) {
                free_sizes.erase(s);
                break;
            }
        free_at.erase(it);
    }
    // Returns [p, p + r.size) of chunk r.chunk to the list, merged with
    // free neighbours of the same chunk.
    void give_back(uintptr_t p, Range r) {
        auto next = free_at.lower_bound(p);
        if (next != free_at.end() && next->second.chunk == r.chunk && p + r.size == next->first) {
            r.size += next->second.size;
            erase(next);
        }
        auto it = free_at.lower_bound(p);
        if (it != free_at.begin()) {
            auto prev = std::prev(it);
            if (prev->second.chunk == r.chunk && prev->first + prev->second.size == p) {
                p = prev->first;
                r.size += prev->second.size;
                erase(prev);
            }
        }
        insert(p, r);
    }
    uint32_t chunk_of(uintptr_t p) const {
        // chunks are few (one per 4 GiB): a scan is enough
        for (size_t i = 0; i < chunk_sizes.size(); ++i) {
            const uintptr_t b = (uintptr_t)chunks[i];
            if (p >= b && p < b + chunk_sizes[i]) return (uint32_t)i;
        }
        return UINT32_MAX;
    }
    std::vector<size_t> chunk_sizes;

    hipError_t alloc(size_t n, void** out) {
        n = round(std::max<size_t>(n, 1));
        auto best = free_sizes.lower_bound(n);
        if (best == free_sizes.end()) {
            size_t sz = std::max(n, kChunk);
            void* p = nullptr;
            hipError_t e = hipMalloc(&p, sz);
            if (e != hipSuccess && sz != n) {  // retry with an exact-size chunk before giving up
                (void)hipGetLastError();
                sz = n;
                e = hipMalloc(&p, sz);
            }
            if (e != hipSuccess) return e;
            chunks.push_back(p);
            chunk_sizes.push_back(sz);
            total += sz;
            insert((uintptr_t)p, Range{sz, (uint32_t)(chunks.size() - 1)});
            best = free_sizes.lower_bound(n);
        }
        const uintptr_t p = best->second;
        auto it = free_at.find(p);
        const Range r = it->second;
        erase(it);
        if (r.size > n) insert(p + n, Range{r.size - n, r.chunk});
        live += n;
        *out = (void*)p;
        return hipSuccess;
    }
    // Returns a range alloc() handed out (n as passed to alloc).
    void free(void* ptr, size_t n) {
        if (!ptr) return;
        n = round(std::max<size_t>(n, 1));
        const uint32_t ch = chunk_of((uintptr_t)ptr);
        if (ch == UINT32_MAX) return;
        give_back((uintptr_t)ptr, Range{n, ch});
        live -= std::min(live, n);
    }
    void release_all() {
        for (void* p : chunks) (void)hipFree(p);
        chunks.clear();
        chunk_sizes.clear();
        free_at.clear();
        free_sizes.clear();
        total = live = 0;
    }
};

// Device scratch that grows on demand (allocation happens outside the
// steady state: the first call at a given size allocates, later calls reuse).
// While graphs captured from the context are alive, a buffer that has to
// grow is retired (freed with the last graph) rather than freed: the graphs
// keep its address.
struct Retire {
    size_t live = 0;             // captured graphs not yet released
    std::vector<void*> retired;  // device buffers replaced meanwhile
    void drop(void* q) {
        if (!q) return;
        if (live) retired.push_back(q);
        else (void)hipFree(q);
    }
};

struct Scratch {
    void* p = nullptr;
    size_t n = 0;
    Retire* retire = nullptr;  // set for the context's buffers
    hipError_t ensure(size_t bytes, bool zero) {
        if (bytes <= n) return hipSuccess;
        if (p) {
            if (retire) retire->drop(p);
            else (void)hipFree(p);
        }
        p = nullptr;
        n = 0;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return e;
        if (zero) {
            // the null-stream fill does not order against the library's
            // non-blocking stream: wait for it here
            e = hipMemset(p, 0, bytes);
            if (e == hipSuccess) e = hipDeviceSynchronize();
            if (e != hipSuccess) return e;
        }
        n = bytes;
        return hipSuccess;
    }
    template <class T>
    T* as() const { return (T*)p; }
};

// A layer's experts as a device array indexed by expert id, rebuilt after the
// layer's store entries change.
struct LayerTable {
    wh_expert_ptrs* dev = nullptr;
    uint32_t cap = 0;  // entries allocated
    uint32_t n = 0;    // ids < n
    bool valid = false;
    bool fast = false;  // every resident expert has one fast shape
    bool zero_scale = false;  // some resident expert has a UE8M0 scale byte 0
    uint32_t resident = 0;    // ids with a resident expert
    size_t hidden = 0, inter = 0;
};

struct HostBuf {
    void* p = nullptr;
    size_t n = 0;
    hipError_t ensure(size_t bytes) {
        if (bytes <= n) return hipSuccess;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
        hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocDefault);
        if (e != hipSuccess) return e;
        n = bytes;
        return hipSuccess;
    }
};

}  // namespace

struct wh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    Arena arena;
    std::unordered_map<wh_tensor, Tensor> tensors;
    std::map<std::pair<uint32_t, uint32_t>, Expert> experts;
    wh_tensor next_id = 1;
    uint32_t* status = nullptr;  // device status word
    uint32_t* status_host = nullptr;
    Scratch x_in, y_out, h, ybuf, cnt_y, tmp, batch, routes, bout, gu;
    Scratch relayout;  // raw FP4 rows on their way into the resident layout
    Scratch rtr;       // router: logits, available ids, outputs of the host-slice call
    Scratch rtr_cnt;   // router: arrival counter of the one-launch bf16 kernel (kept at 0)
    Scratch mla;       // MLA decode attention: activations between the projections
    Scratch hcs;       // mHC: chain sums and the internal pre weights
    std::map<std::string, float*> rope_tabs;  // device RoPE inverse frequencies by (dim, theta, YaRN)
    std::map<uint32_t, Router> routers;
    HostBuf stage_in, stage_out;
    HostBuf pack[2];   // experts-pack read buffers (one filling while the other uploads)
    std::map<uint32_t, LayerTable> tables;  // device expert tables of the batch path
    uint32_t moe_mfma_min = 1;              // batch experts with this many tokens use MFMA (0: never)
    uint32_t fp8_mm_min = 4;                // multi-input FP8 GEMVs with this many inputs use MFMA
    Scratch fp8mm_ws, fp8mm_cnt;            // their partial tiles and arrival counters
    Scratch moe_dyn;                        // a device route list resolved for the experts (wh_moe_dyn)
    Scratch layer;                          // the decode layer's state and activations between its steps
    bool exact = true;                      // routed experts in the reference's summation order
    int token_kernels = 1;                  // MFMA token kernels: bit 0 gate/up, bit 1 down on k_*_tok (else k_*_px)
    bool capture_gu = false;                // routed experts keep gate/up in `gu` (test support)
    size_t tok_last_n = 0, tok_last_tokens = 0, tok_last_hidden = 0, tok_last_inter = 0;
    size_t moe_last_slots = 0, moe_last_npos = 0;  // sizes of the last single-chunk batch call
    size_t moe_last_hidden = 0, moe_last_inter = 0;
    std::recursive_mutex mu;  // recursive: composite entry points call the others
    hipEvent_t timer[2] = {nullptr, nullptr};  // wh_timer_start / wh_timer_stop
    Retire retire;                                     // buffers kept for live graphs
    std::map<uint64_t, hipGraphExec_t> graphs;         // wh_graph_end handles
    uint64_t next_graph = 1;
    // Between wh_graph_begin and wh_graph_end `stream` is cap_stream, a
    // stream of its own in capture mode, so a call that breaks the capture
    // leaves the context's stream (base_stream) untouched.
    bool capturing = false;
    hipStream_t base_stream = nullptr, cap_stream = nullptr;
    std::vector<Scratch*> scratch() {
        return {&x_in, &y_out, &h, &ybuf, &cnt_y, &tmp, &batch, &routes, &bout, &gu, &relayout, &rtr, &rtr_cnt,
                &mla, &hcs, &fp8mm_ws, &fp8mm_cnt, &moe_dyn, &layer};
    }
};

namespace {

thread_local char g_last_error[256] = "";

int hip_status_at(hipError_t e, const char* what, int line) {
    if (e == hipSuccess) return WH_OK;
    std::snprintf(g_last_error, sizeof g_last_error, "%s (%d) at wohper_hip.hip:%d: %s",
                  hipGetErrorName(e), (int)e, line, what);
    if (e == hipErrorOutOfMemory) return WH_OUT_OF_MEMORY;
    return WH_HIP_ERROR;
}

#define hip_status(e) hip_status_at((e), "", __LINE__)

#define WH_HIP(expr)                                                   \
    do {                                                               \
        hipError_t _e = (expr);                                        \
        if (_e != hipSuccess) return hip_status_at(_e, #expr, __LINE__); \
    } while (0)

#define WH_TRY(expr)               \
    do {                           \
        int _s = (expr);           \
        if (_s != WH_OK) return _s; \
    } while (0)

int read_status(wh_ctx* c) {
    WH_HIP(hipMemcpyAsync(c->status_host, c->status, sizeof(uint32_t), hipMemcpyDeviceToHost,
                          c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    uint32_t st = *c->status_host;
    if (st) {
        WH_HIP(hipMemsetAsync(c->status, 0, sizeof(uint32_t), c->stream));
        WH_HIP(hipStreamSynchronize(c->stream));
    }
    if (st & WH_ST_NOT_RESIDENT) return WH_NOT_RESIDENT;
    if (st & WH_ST_NONFINITE_INPUT) return WH_NON_FINITE_INPUT;
    if (st & WH_ST_NONFINITE_OUTPUT) return WH_NON_FINITE_OUTPUT;
    return WH_OK;
}

Tensor* find_tensor(wh_ctx* c, wh_tensor t) {
    auto it = c->tensors.find(t);
    return it == c->tensors.end() ? nullptr : &it->second;
}

int alloc_device(wh_ctx* c, size_t n, void** out) {
    hipError_t e = c->arena.alloc(n, out);
    if (e != hipSuccess) return hip_status(e);
    return WH_OK;
}

// The weight and scale buffers of a new tensor, recorded for its release.
int alloc_tensor(wh_ctx* c, Tensor& t, size_t wbytes, size_t sbytes) {
    void* wd = nullptr;
    void* sd = nullptr;
    WH_TRY(alloc_device(c, wbytes, &wd));
    const int st = alloc_device(c, sbytes, &sd);
    if (st != WH_OK) {
        c->arena.free(wd, wbytes);
        return st;
    }
    t.w = (uint8_t*)wd;
    t.s = sd;
    t.w_alloc = wbytes;
    t.s_alloc = sbytes;
    return WH_OK;
}

// Drops a tensor handle and returns its HBM to the arena.  Work already
// queued on the library stream may still read the bytes; every later write
// to a reused range (uploads, fills) is queued behind it on the same stream.
void drop_tensor(wh_ctx* c, wh_tensor id) {
    auto it = c->tensors.find(id);
    if (it == c->tensors.end()) return;
    c->arena.free(it->second.w, it->second.w_alloc);
    c->arena.free(it->second.s, it->second.s_alloc);
    c->tensors.erase(it);
}

int upload(wh_ctx* c, void* dst, const void* src, size_t n) {
    if (n == 0) return WH_OK;
    WH_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    return WH_OK;
}

// FP8 resident permutation within each 128-col group (see kernels.h).
void fp8_permute_row(const uint8_t* src, uint8_t* dst, size_t cols) {
    for (size_t g = 0; g < cols / 128; ++g) {
        const uint8_t* s = src + g * 128;
        uint8_t* d = dst + g * 128;
        for (int l = 0; l < 8; ++l)
            for (int i = 0; i < 16; ++i) d[l * 16 + i] = s[(i & 7) * 16 + (i >> 3) * 8 + l];
    }
}

// Dynamic LDS a workgroup may use: the device's per-block limit (160 KB on
// gfx950) when the runtime accepts raising the kernels' attribute, else 64 KB.
size_t g_max_lds = 64 * 1024;

hipError_t kernel_setup_once(int device) {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [device] {
        int lds = 64 * 1024;
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > lds)
            lds = v;
        hipError_t e = hipSuccess;
        // leave room for the kernels' own static LDS (a few words each)
        lds -= 1024;
        auto set = [&](const void* f) {
            hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
            if (r != hipSuccess && e == hipSuccess) e = r;
        };
#define WH_SK_SET(G)                                                                              \
    for (const void* f : {(const void*)k_fp8_gemv_sk<false, false, G>, (const void*)k_fp8_gemv_sk<false, true, G>, \
                          (const void*)k_fp8_gemv_sk<true, false, G>, (const void*)k_fp8_gemv_sk<true, true, G>})    \
        set(f);
        WH_SK_SET(0)
        WH_SK_SET(1)
        WH_SK_SET(2)
        WH_SK_SET(4)
        WH_SK_SET(8)
#undef WH_SK_SET
        set((const void*)k_fp8_gemv<false, false>);
        set((const void*)k_fp8_gemv<false, true>);
        set((const void*)k_fp8_gemv<true, false>);
        set((const void*)k_fp8_gemv<true, true>);
        set((const void*)k_fp4_matvec<0>);
        set((const void*)k_fp4_matvec<8>);
        set((const void*)k_fp4_matvec<16>);
        set((const void*)k_moe_gateup<0>);
        set((const void*)k_moe_gateup<16>);
        set((const void*)k_moe_down<0>);
        set((const void*)k_moe_down<8>);
        set((const void*)k_moe_batch_gateup<0>);
        set((const void*)k_moe_batch_gateup<16>);
        set((const void*)k_moe_batch_down<0>);
        set((const void*)k_moe_batch_down<8>);
        set((const void*)k_moe_batch_mx<4096, true>);
        set((const void*)k_moe_batch_mx<2048, true>);
        set((const void*)k_moe_batch_mx<2048, false>);
#define WH_MM_SET(G_)                                    \
        set((const void*)k_fp8_mm<false, false, G_>);    \
        set((const void*)k_fp8_mm<false, true, G_>);     \
        set((const void*)k_fp8_mm<true, false, G_>);     \
        set((const void*)k_fp8_mm<true, true, G_>);
        WH_MM_SET(2)
        WH_MM_SET(4)
        WH_MM_SET(8)
#undef WH_MM_SET
        if (e == hipSuccess) {
            g_max_lds = (size_t)lds;
        } else {
            (void)hipGetLastError();  // keep the 64 KB default
        }
        err = hipSuccess;
    });
    return err;
}

// ------------------------------------------------------------ FP8 launch
// LDS of a split-K FP8 workgroup: staged x, the 8 rows x 8 lanes x groups
// partial sums and the 8 rows' group scales.
size_t fp8_sk_lds(size_t cols) { return sizeof(float) * (cols + 72 * (cols / 128)); }

// Whether launch_fp8 takes the split-K path for this tensor (which also
// supports per-row-group inputs).
bool is_pow2(size_t v) { return v && !(v & (v - 1)); }
uint32_t log2_of(size_t v) {
    uint32_t k = 0;
    while ((size_t(1) << k) < v) ++k;
    return k;
}
bool fp8_split_k(const Tensor& t) {
    return t.fast && (t.cols / 128) % 8 == 0 && fp8_sk_lds(t.cols) <= g_max_lds && is_pow2(t.rows / t.scale_rows);
}

// x_group_rows / x_group_stride: row groups with their own input (split-K
// path only; see wh_fp8_args).
// order_free: with exact numerics off the order-free kernel may run (the
// router's gate GEMV passes false: its top-k needs the reference's logits).
int launch_fp8(wh_ctx* c, const Tensor& t, size_t r0, size_t r1, const float* x, float* y,
               size_t n_batch, size_t x_stride, size_t y_stride, size_t x_group_rows = 0,
               size_t x_group_stride = 0, const Tensor* t2 = nullptr, size_t r0_2 = 0, size_t r1_2 = 0,
               float* y2 = nullptr, bool order_free = true) {
    wh_fp8_args a;
    std::memset(&a, 0, sizeof a);
    a.blocks1 = UINT32_MAX;
    a.w = t.w;
    a.scales = t.s;
    a.x = x;
    a.y = y;
    a.status = c->status;
    a.cols = (uint32_t)t.cols;
    a.scale_cols = (uint32_t)t.scale_cols;
    a.row_group = (uint32_t)(t.rows / t.scale_rows);
    a.row_group_shift = is_pow2(a.row_group) ? log2_of(a.row_group) : 32u;
    a.row_start = (uint32_t)r0;
    a.row_end = (uint32_t)r1;
    a.x_stride = (uint32_t)x_stride;
    a.y_stride = (uint32_t)y_stride;
    a.x_group_rows = (uint32_t)x_group_rows;
    a.x_group_stride = (uint32_t)x_group_stride;
    a.x_group_shift = x_group_rows ? log2_of(x_group_rows) : 32u;
    if (x_group_rows && (!fp8_split_k(t) || !is_pow2(x_group_rows) || x_group_rows < WH_FP8_SK_ROWS))
        return WH_UNSUPPORTED;
    bool u8 = t.scale_fmt == WH_SCALE_UE8M0;
    if (t2) {  // a second tensor on the same input: fp8_pair_ok
        a.blocks1 = (uint32_t)((r1 - r0 + WH_FP8_SK_ROWS - 1) / WH_FP8_SK_ROWS);
        a.w2 = t2->w;
        a.scales2 = t2->s;
        a.y2 = y2;
        a.scale_cols2 = (uint32_t)t2->scale_cols;
        a.row_group_shift2 = log2_of(t2->rows / t2->scale_rows);
        a.row_start2 = (uint32_t)r0_2;
        a.row_end2 = (uint32_t)r1_2;
    }
    // exact numerics off: the order-free kernel (fp8_tol.h) for lane-layout
    // tensors without the reference's +-480 codes, widths of 1, 2, 4 or 8
    // slices of 1024 columns and a power of two rows per scale row
    const size_t slices = t.cols / 1024;
    const bool tol_shape = order_free && !c->exact && t.fast && !t.special && t.cols % 1024 == 0 &&
                           (slices == 1 || slices == 2 || slices == 4 || slices == 8) &&
                           is_pow2(t.rows / t.scale_rows) &&
                           (!t2 || (t2->fast && !t2->special && t2->cols == t.cols));
    if (tol_shape) {
        // waves per workgroup: one per slice, at least 4; pairs (row,
        // slice) per wave: as many as keep >= 512 workgroups, up to 8
        const size_t kw = slices == 8 ? 8 : 4;
        const size_t pairs = ((r1 - r0) + (t2 ? r1_2 - r0_2 : 0)) * slices;
        size_t kp = pairs >= 8 * kw * 512 ? 8 : pairs >= 4 * kw * 512 ? 4 : 2;
#ifdef WH_TOL_KP
        kp = WH_TOL_KP;
#endif
        const size_t kr = kp * kw / slices;  // rows per workgroup
        const size_t rg = t.rows / t.scale_rows;
        // a workgroup stays inside one input's rows
        if (!x_group_rows || x_group_rows % kr == 0) {
            const bool one = rg % kr == 0 && r0 % kr == 0 &&
                             (!t2 || ((t2->rows / t2->scale_rows) % kr == 0 && r0_2 % kr == 0));
            const size_t b1 = (r1 - r0 + kr - 1) / kr;
            if (t2) a.blocks1 = (uint32_t)b1;
            dim3 grid((unsigned)(b1 + (t2 ? (r1_2 - r0_2 + kr - 1) / kr : 0)), (unsigned)n_batch);
            const unsigned threads = (unsigned)(64 * kw);
#define WH_TOL(W, S, P)                                                                      \
    do {                                                                                     \
        if (u8 && one) k_fp8_gemv_tol<W, S, P, true, true><<<grid, threads, 0, c->stream>>>(a);    \
        else if (u8) k_fp8_gemv_tol<W, S, P, true, false><<<grid, threads, 0, c->stream>>>(a);     \
        else if (one) k_fp8_gemv_tol<W, S, P, false, true><<<grid, threads, 0, c->stream>>>(a);    \
        else k_fp8_gemv_tol<W, S, P, false, false><<<grid, threads, 0, c->stream>>>(a);            \
    } while (0)
#define WH_TOL_S(P)                            \
    do {                                       \
        if (slices == 1) WH_TOL(4, 1, P);      \
        else if (slices == 2) WH_TOL(4, 2, P); \
        else if (slices == 4) WH_TOL(4, 4, P); \
        else WH_TOL(8, 8, P);                  \
    } while (0)
            if (kp == 2) WH_TOL_S(2);
            else if (kp == 4) WH_TOL_S(4);
#ifdef WH_TOL_KP
            else if (kp == 16) WH_TOL_S(16);
#endif
            else WH_TOL_S(8);
#undef WH_TOL_S
#undef WH_TOL
            WH_HIP(hipGetLastError());
            return WH_OK;
        }
    }
    // several inputs in the reference's order: each weight byte decoded
    // once for all of them (k_fp8_gemv_multi); the most inputs per
    // workgroup (16, 8, 4, 2) that keep about 1024 workgroups (two waves
    // per SIMD: every weight row is read once per block of inputs, and a
    // fuller device outweighs the re-reads)
    const size_t mrows = (r1 - r0) + (t2 ? r1_2 - r0_2 : 0);
    size_t mk = 16;
    while (mk > 2 && (mrows / WH_FP8_MULTI_ROWS) * ((n_batch + mk - 1) / mk) < 1024) mk /= 2;
    while (mk > 2 && mk / 2 >= n_batch) mk /= 2;  // no more slots than inputs
#ifdef WH_MULTI_MK
    mk = WH_MULTI_MK;
#endif
#ifndef WH_MULTI_MINROWS
#define WH_MULTI_MINROWS 4096
#endif
    // below WH_MULTI_MINROWS rows the per-input kernel's wider grid is
    // faster, and the weights are small enough to stay in cache across the
    // inputs
    if (n_batch >= 2 && mrows >= WH_MULTI_MINROWS && fp8_split_k(t) &&
        t.cols % (128 * (size_t)wh_fp8_multi_groups((int)mk)) == 0 &&
        (!t2 || (fp8_split_k(*t2) && t2->cols == t.cols && t2->special == t.special)) &&
        (!x_group_rows || (x_group_rows % WH_FP8_MULTI_ROWS == 0 && x_group_stride % 4 == 0)) && x_stride % 4 == 0) {
        const size_t b1 = (r1 - r0 + WH_FP8_MULTI_ROWS - 1) / WH_FP8_MULTI_ROWS;
        if (t2) a.blocks1 = (uint32_t)b1;
        dim3 grid((unsigned)(b1 + (t2 ? (r1_2 - r0_2 + WH_FP8_MULTI_ROWS - 1) / WH_FP8_MULTI_ROWS : 0)),
                  (unsigned)((n_batch + mk - 1) / mk));
        const uint32_t n_in = (uint32_t)n_batch;
#define WH_MULTI(N)                                                                               \
    do {                                                                                          \
        if (t.special) {                                                                          \
            if (u8) k_fp8_gemv_multi<N, true, true><<<grid, 128, 0, c->stream>>>(a, n_in);        \
            else k_fp8_gemv_multi<N, true, false><<<grid, 128, 0, c->stream>>>(a, n_in);          \
        } else {                                                                                  \
            if (u8) k_fp8_gemv_multi<N, false, true><<<grid, 128, 0, c->stream>>>(a, n_in);       \
            else k_fp8_gemv_multi<N, false, false><<<grid, 128, 0, c->stream>>>(a, n_in);         \
        }                                                                                         \
    } while (0)
        if (mk == 16) WH_MULTI(16);
        else if (mk == 8) WH_MULTI(8);
        else if (mk == 4) WH_MULTI(4);
        else WH_MULTI(2);
#undef WH_MULTI
        WH_HIP(hipGetLastError());
        return WH_OK;
    }
    if (fp8_split_k(t)) {
        const size_t blocks = (r1 - r0 + WH_FP8_SK_ROWS - 1) / WH_FP8_SK_ROWS +
                              (t2 ? (r1_2 - r0_2 + WH_FP8_SK_ROWS - 1) / WH_FP8_SK_ROWS : 0);
        dim3 grid((unsigned)blocks, (unsigned)n_batch);
        const size_t lds = fp8_sk_lds(t.cols);
        // groups per segment known at compile time for the common widths
        const size_t gps = t.cols / 128 / 8;
#define WH_SK(SP, U8)                                                                             \
    do {                                                                                          \
        if (gps == 1) k_fp8_gemv_sk<SP, U8, 1><<<grid, 256, lds, c->stream>>>(a);                 \
        else if (gps == 2) k_fp8_gemv_sk<SP, U8, 2><<<grid, 256, lds, c->stream>>>(a);            \
        else if (gps == 4) k_fp8_gemv_sk<SP, U8, 4><<<grid, 256, lds, c->stream>>>(a);            \
        else if (gps == 8) k_fp8_gemv_sk<SP, U8, 8><<<grid, 256, lds, c->stream>>>(a);            \
        else k_fp8_gemv_sk<SP, U8, 0><<<grid, 256, lds, c->stream>>>(a);                         \
    } while (0)
        if (t.special) {
            if (u8) WH_SK(true, true);
            else WH_SK(true, false);
        } else {
            if (u8) WH_SK(false, true);
            else WH_SK(false, false);
        }
#undef WH_SK
    } else if (t.fast) {
        dim3 grid((unsigned)((r1 - r0 + 31) / 32), (unsigned)n_batch);
        size_t lds = t.cols * sizeof(float);
        if (t.special) {
            if (u8) k_fp8_gemv<true, true><<<grid, 256, lds, c->stream>>>(a);
            else k_fp8_gemv<true, false><<<grid, 256, lds, c->stream>>>(a);
        } else {
            if (u8) k_fp8_gemv<false, true><<<grid, 256, lds, c->stream>>>(a);
            else k_fp8_gemv<false, false><<<grid, 256, lds, c->stream>>>(a);
        }
    } else {
        dim3 grid((unsigned)((r1 - r0 + 63) / 64), (unsigned)n_batch);
        uint32_t col_group = (uint32_t)(t.cols / t.scale_cols);
        if (u8) k_fp8_gemv_generic<true><<<grid, 64, 0, c->stream>>>(a, col_group);
        else k_fp8_gemv_generic<false><<<grid, 64, 0, c->stream>>>(a, col_group);
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// Multi-input GEMV on bf16 MFMA (fp8_mm.h): lane-layout tensors of a
// multiple of 256 columns whose scale rows span a power of two >= 16 rows, ranges starting on a
// 16-row boundary, and input groups (rows with their own input) of a power
// of two >= 128 rows.
bool fp8_mm_ok(const Tensor& t, size_t r0, size_t r1, size_t group_rows) {
    const size_t rg = t.rows / t.scale_rows;
    if (!t.fast || t.cols % 256 || !is_pow2(rg) || rg < 16 || r0 % 16) return false;
    if (group_rows && (!is_pow2(group_rows) || group_rows < 128 || (r1 - r0) % group_rows)) return false;
    return true;
}

// Groups per k split of a multi-input MFMA launch over `rows` rows and n
// inputs: 8, 4 or 2 (what divides the width and fits LDS), the most that
// still gives ~256 workgroups; 0 when none fits.
size_t fp8_mm_groups(const Tensor& t, size_t rows, size_t n) {
    const size_t rb = (rows + WH_FP8MM_ROWS - 1) / WH_FP8MM_ROWS, G = t.cols / 128;
    const size_t tbs = (n + WH_FP8MM_TOK - 1) / WH_FP8MM_TOK;
    size_t kg = 0;
    for (size_t g = WH_FP8MM_MAX_GROUPS; g >= 2; g /= 2) {
        if (G % g || wh_fp8mm_lds(g * 128) > g_max_lds) continue;
        kg = g;
        if (rb * tbs * (G / g) >= 256) break;
    }
    return kg;
}

// Rows [r0, r1) of a second tensor on the same inputs, for one launch.
struct Fp8MmSecond {
    const Tensor* t;
    size_t r0, r1;
    float* y;
    size_t y_stride;
};

// y_t = W x_t over rows [r0, r1) for n inputs; with group_rows, rows
// r0 + [g group_rows, (g + 1) group_rows) read input group g at
// x + g * xg_stride.  One launch over (row block, k split, token block); with
// `second`, its row blocks follow the first tensor's in the same launch
// (the caller checks that both take the same k split).
int launch_fp8_mm(wh_ctx* c, const Tensor& t, size_t r0, size_t r1, const float* x, size_t n, size_t x_stride,
                  float* y, size_t y_stride, size_t group_rows, size_t xg_stride,
                  const Fp8MmSecond* second = nullptr) {
    const size_t rows = r1 - r0, rb1 = (rows + WH_FP8MM_ROWS - 1) / WH_FP8MM_ROWS, G = t.cols / 128;
    const size_t rb2 = second ? (second->r1 - second->r0 + WH_FP8MM_ROWS - 1) / WH_FP8MM_ROWS : 0;
    const size_t rb = rb1 + rb2;
    const size_t tbs = (n + WH_FP8MM_TOK - 1) / WH_FP8MM_TOK;
    const size_t kg = fp8_mm_groups(t, rows, n);
    if (kg == 0) return WH_UNSUPPORTED;
    const size_t S = G / kg, kc = kg * 128;
    if (rb * S > 65535 || tbs > 65535) return WH_UNSUPPORTED;
    if (S > 1) {
        WH_HIP(c->fp8mm_ws.ensure(tbs * rb * S * WH_FP8MM_ROWS * 16 * sizeof(float), false));
        WH_HIP(c->fp8mm_cnt.ensure(tbs * rb * sizeof(uint32_t), true));
    }
    wh_fp8mm_args a;
    std::memset(&a, 0, sizeof a);
    a.w = t.w;
    a.scales = t.s;
    a.x = x;
    a.y = y;
    a.ws = c->fp8mm_ws.as<float>();
    a.cnt = c->fp8mm_cnt.as<uint32_t>();
    a.status = c->status;
    a.cols = (uint32_t)t.cols;
    a.scale_cols = (uint32_t)t.scale_cols;
    a.row_group_shift = log2_of(t.rows / t.scale_rows);
    a.row_start = (uint32_t)r0;
    a.row_end = (uint32_t)r1;
    a.n = (uint32_t)n;
    a.x_stride = (uint32_t)x_stride;
    a.y_stride = (uint32_t)y_stride;
    a.xg_shift = group_rows ? log2_of(group_rows) : 31u;
    a.xg_stride = (uint32_t)xg_stride;
    a.kc = (uint32_t)kc;
    a.splits = (uint32_t)S;
    a.row_blocks = (uint32_t)rb;
    a.rb_first = (uint32_t)rb1;
    if (second) {
        a.w2 = second->t->w;
        a.scales2 = second->t->s;
        a.y2 = second->y;
        a.row_start2 = (uint32_t)second->r0;
        a.row_end2 = (uint32_t)second->r1;
        a.y2_stride = (uint32_t)second->y_stride;
    }
    const dim3 grid((unsigned)rb, (unsigned)S, (unsigned)tbs);
    const size_t lds = wh_fp8mm_lds(kc);
    const bool u8 = t.scale_fmt == WH_SCALE_UE8M0;
    auto go = [&](auto kern) { kern<<<grid, 512, lds, c->stream>>>(a); };
#define WH_MM_GO(G_)                                        \
    if (kg == G_) {                                         \
        if (t.special) {                                    \
            if (u8) go(k_fp8_mm<true, true, G_>);           \
            else go(k_fp8_mm<true, false, G_>);             \
        } else {                                            \
            if (u8) go(k_fp8_mm<false, true, G_>);          \
            else go(k_fp8_mm<false, false, G_>);            \
        }                                                   \
    }
    WH_MM_GO(2)
    WH_MM_GO(4)
    WH_MM_GO(8)
#undef WH_MM_GO
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int launch_fp4(wh_ctx* c, const Tensor& t, const float* x, float* y) {
    wh_fp4_args a;
    a.w = t.w;
    a.s = (const uint8_t*)t.s;
    a.x = x;
    a.y = y;
    a.status = c->status;
    a.rows = (uint32_t)t.rows;
    a.cols = (uint32_t)t.cols;
    if (t.fast) {
        dim3 grid((unsigned)((t.rows + 31) / 32));
        size_t lds = wh_fp4_wg_lds(t.cols);
        if (t.cols == 4096) k_fp4_matvec<16><<<grid, 256, lds, c->stream>>>(a);
        else if (t.cols == 2048) k_fp4_matvec<8><<<grid, 256, lds, c->stream>>>(a);
        else k_fp4_matvec<0><<<grid, 256, lds, c->stream>>>(a);
    } else {
        k_fp4_matvec_generic<<<(unsigned)((t.rows + 63) / 64), 64, 0, c->stream>>>(a, (uint32_t)t.scale_cols);
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

__global__ void k_swiglu_generic(const float* g, const float* u, float* h, uint32_t n,
                                 uint32_t* status) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = wh_swiglu(g[i], u[i], kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
}

// Ordered routed sum (E/compute.rs:1948-2030) of the first n_experts -
// has_shared outputs; with has_shared the last output is the shared expert's
// and out = shared + routed (E/compute.rs:1929-1941).
__global__ void k_combine_generic(const float* y, const float* w, uint32_t n_experts, uint32_t has_shared,
                                  uint32_t hidden, float* out) {
    uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= hidden) return;
    const uint32_t nr = n_experts - has_shared;
    float o = 0.0f;
    if (nr == 1) {
        o = y[r];
    } else if (nr > 1) {
        float sum = 0.0f;
        bool valid = true;
        for (uint32_t i = 0; i < nr; ++i) {
            float wi = w[i];
            if (!(fabsf(wi) <= 3.4028235e38f && wi >= 0.0f)) valid = false;
            sum = sum + wi;
        }
        if (sum <= 1.1920929e-07f) valid = false;
        float uniform = 1.0f / (float)nr;
        for (uint32_t i = 0; i < nr; ++i) {
            float wi = valid ? w[i] / sum : uniform;
            float p = y[(size_t)i * hidden + r] * wi;
            o = o + p;
        }
    }
    if (has_shared) {
        const float sh = y[(size_t)nr * hidden + r];
        o = nr == 0 ? sh : sh + o;
    }
    out[r] = o;
}

struct ExpertView {
    const Tensor *w1, *w3, *w2;
};

int resolve_expert(wh_ctx* c, uint32_t layer, uint32_t expert, ExpertView* v) {
    auto it = c->experts.find({layer, expert});
    if (it == c->experts.end()) return WH_NOT_RESIDENT;
    v->w1 = find_tensor(c, it->second.w1);
    v->w3 = find_tensor(c, it->second.w3);
    v->w2 = find_tensor(c, it->second.w2);
    if (!v->w1 || !v->w3 || !v->w2) return WH_NOT_RESIDENT;
    return WH_OK;
}

// A UE8M0 scale byte 0 decodes to 0.0 (E/deepseek_v4.rs:166-172); the
// block-scaled MFMA reads it as 2^-127, so experts that have one run on the
// exact kernels.
bool expert_zero_scale(const ExpertView& v) { return v.w1->zero_scale || v.w3->zero_scale || v.w2->zero_scale; }

bool expert_fast(const ExpertView& v) {
    return v.w1->fast && v.w3->fast && v.w2->fast && v.w1->cols % 256 == 0 && v.w1->rows % 256 == 0 &&
           wh_moe_wg_lds(v.w1->cols) <= g_max_lds && wh_moe_wg_lds(v.w1->rows) <= g_max_lds;
}

// Working memory of the fast routed-expert kernels for one call.
struct MoeBufs {
    float* h = nullptr;       // [T][n][inter] SwiGLU outputs
    float* y = nullptr;       // [T][n][hidden] per-expert outputs
    uint32_t* cnt = nullptr;  // [T][hidden / 16] routed-sum arrivals (cleared by gate/up)
    float* gu = nullptr;      // test capture of gate and up, or null
};

// Compute units of the current device (cached).
int device_cus() {
    static std::mutex mu;
    static std::map<int, int> cache;
    std::lock_guard<std::mutex> lk(mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
    return cus;
}

// The MFMA token kernels (summation order freed) serve the model's shapes
// unless the context asks for the reference's order.
bool moe_mfma(const wh_ctx* c, size_t hidden, size_t inter) {
    return !c->exact && (hidden == 2048 || hidden == 4096) && inter == 2048;
}

// Bytes of each MoeBufs region (each rounded up to 256).
struct MoeSizes {
    size_t h, y, cnt;
    size_t total() const { return h + y + cnt; }
};
MoeSizes moe_sizes(size_t n, size_t n_tokens, size_t hidden, size_t inter) {
    auto r = [](size_t b) { return (b + 255) & ~size_t(255); };
    MoeSizes z;
    z.h = r(n_tokens * n * inter * sizeof(float));
    z.y = r(n_tokens * n * hidden * sizeof(float));
    z.cnt = r(n_tokens * (hidden / 16) * sizeof(uint32_t));
    return z;
}

// The context's own (growing) buffers.
int moe_bufs_ctx(wh_ctx* c, size_t n, size_t n_tokens, size_t hidden, size_t inter, MoeBufs* b) {
    const MoeSizes z = moe_sizes(n, n_tokens, hidden, inter);
    WH_HIP(c->h.ensure(z.h, false));
    WH_HIP(c->ybuf.ensure(z.y, false));
    WH_HIP(c->cnt_y.ensure(z.cnt, true));
    b->h = c->h.as<float>();
    b->y = c->ybuf.as<float>();
    b->cnt = c->cnt_y.as<uint32_t>();
    if (c->capture_gu) {
        WH_HIP(c->gu.ensure(n_tokens * n * 2 * inter * sizeof(float), false));
        b->gu = c->gu.as<float>();
    }
    return WH_OK;
}

// Launches the fast routed-expert kernels for n_tokens rows of x sharing one
// route list.  stages: bit 0 = gate/up + SwiGLU, bit 1 = down + routed sum.
// record: keep the call's sizes for the debug reads of the context buffers.
// A route list in device memory (wh_moe_dyn) instead of ev / route_w: the
// experts' shapes and whether any of them holds a UE8M0 scale byte 0.
struct MoeDyn {
    const wh_moe_dyn* p = nullptr;
    size_t hidden = 0, inter = 0;
    bool zero_scale = false;
};

int moe_launch_fast(wh_ctx* c, const ExpertView* ev, const float* route_w, size_t n, bool has_shared,
                    const void* x_dev, int x_bf16, size_t n_tokens, float* out_dev, unsigned stages,
                    const MoeBufs& bufs, bool record, const MoeDyn* dyn = nullptr) {
    const size_t hidden = dyn ? dyn->hidden : ev[0].w1->cols, inter = dyn ? dyn->inter : ev[0].w1->rows;
    if (((uintptr_t)x_dev & 15) || ((uintptr_t)out_dev & 3)) return WH_INVALID_ARGUMENT;
    wh_moe_args a;
    std::memset(&a, 0, sizeof a);
    if (dyn) a.dyn = dyn->p;
    for (size_t i = 0; i < n && !dyn; ++i) {
        a.ex[i].w1 = ev[i].w1->w;
        a.ex[i].s1 = (const uint8_t*)ev[i].w1->s;
        a.ex[i].w3 = ev[i].w3->w;
        a.ex[i].s3 = (const uint8_t*)ev[i].w3->s;
        a.ex[i].w2 = ev[i].w2->w;
        a.ex[i].s2 = (const uint8_t*)ev[i].w2->s;
        a.route_w[i] = route_w[i];
    }
    a.n_experts = (uint32_t)n;
    a.has_shared = has_shared ? 1u : 0u;
    a.hidden = (uint32_t)hidden;
    a.inter = (uint32_t)inter;
    a.n_tokens = (uint32_t)n_tokens;
    a.x = x_dev;
    a.x_is_bf16 = x_bf16 ? 1u : 0u;
    a.h = bufs.h;
    a.y = bufs.y;
    a.out = out_dev;
    a.cnt_y = bufs.cnt;
    a.status = c->status;
    a.gu = bufs.gu;
    if (record)
        c->tok_last_n = n, c->tok_last_tokens = n_tokens, c->tok_last_hidden = hidden, c->tok_last_inter = inter;
    bool sk = moe_mfma(c, hidden, inter);
    if (dyn) sk = sk && !dyn->zero_scale;
    for (size_t i = 0; i < n && sk && !dyn; ++i) sk = !expert_zero_scale(ev[i]);
    // the LDS-DMA kernels (moe_tok.h): hidden 4096, inter 2048, up to 8 experts
    const bool tk_shape = sk && hidden == 4096 && inter == 2048 && n <= 8;
    const bool tk = tk_shape && (c->token_kernels & 1), tkd = tk_shape && (c->token_kernels & 2);
    if (stages & 1) {
        if (tk) {
            const size_t tiles = n * inter / 16, cus = (size_t)device_cus();
            const size_t per = std::min<size_t>(4, std::max<size_t>(1, (tiles * n_tokens + cus - 1) / cus));
            dim3 ggrid((unsigned)((tiles + per - 1) / per), (unsigned)n_tokens);
#define WH_GU_TOK(P)                                                                                        \
    do {                                                                                                    \
        if (x_bf16) k_moe_gateup_tok<P, WH_TOK_SLOTS, true><<<ggrid, 512, 0, c->stream>>>(a);               \
        else k_moe_gateup_tok<P, WH_TOK_SLOTS, false><<<ggrid, 512, 0, c->stream>>>(a);                     \
    } while (0)
            if (per == 1) WH_GU_TOK(1);
            else if (per == 2) WH_GU_TOK(2);
            else if (per == 3) WH_GU_TOK(3);
            else WH_GU_TOK(4);
#undef WH_GU_TOK
        } else if (sk) {
            // block-scaled FP8 MFMA over the act-quantized x: persistent
            // workgroups of `per` 16-row tiles, about one per CU
            const size_t tiles = n * inter / 16, cus = (size_t)device_cus();
            const size_t per = std::min<size_t>(4, std::max<size_t>(1, (tiles * n_tokens + cus - 1) / cus));
            dim3 ggrid((unsigned)((tiles + per - 1) / per), (unsigned)n_tokens);
#define WH_GU_PX(C)                                                                      \
    do {                                                                                 \
        if (per == 1) k_moe_gateup_px<C, 1><<<ggrid, C / 8, 0, c->stream>>>(a);          \
        else if (per == 2) k_moe_gateup_px<C, 2><<<ggrid, C / 8, 0, c->stream>>>(a);     \
        else if (per == 3) k_moe_gateup_px<C, 3><<<ggrid, C / 8, 0, c->stream>>>(a);     \
        else k_moe_gateup_px<C, 4><<<ggrid, C / 8, 0, c->stream>>>(a);                   \
    } while (0)
            if (hidden == 4096) WH_GU_PX(4096);
            else WH_GU_PX(2048);
#undef WH_GU_PX
        } else if (hidden == 4096) {
            dim3 ggrid((unsigned)(n * inter / 16), (unsigned)n_tokens);
            k_moe_gateup<16><<<ggrid, 256, wh_moe_wg_lds(hidden), c->stream>>>(a);
        } else {
            dim3 ggrid((unsigned)(n * inter / 16), (unsigned)n_tokens);
            k_moe_gateup<0><<<ggrid, 256, wh_moe_wg_lds(hidden), c->stream>>>(a);
        }
    }
    if (stages & 2) {
        dim3 dgrid((unsigned)(n * hidden / 32), (unsigned)n_tokens);
        if (tkd) {
            // every expert of a 16-row output slice per workgroup, the
            // weights and h streamed into LDS
            dim3 pgrid((unsigned)(hidden / 16), (unsigned)n_tokens);
            switch ((n + 1) / 2) {
                case 1: k_moe_down_tok<1, WH_TOKD_SLOTS><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 2: k_moe_down_tok<2, WH_TOKD_SLOTS><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 3: k_moe_down_tok<3, WH_TOKD_SLOTS><<<pgrid, 512, 0, c->stream>>>(a); break;
                default: k_moe_down_tok<4, WH_TOKD_SLOTS><<<pgrid, 512, 0, c->stream>>>(a); break;
            }
        } else if (sk) {
            // every expert of a 16-row output slice per workgroup: the routed
            // sum stays in the workgroup
            dim3 pgrid((unsigned)(hidden / 16), (unsigned)n_tokens);
#ifndef WH_NO_DOWN_PB
            // an odd number of experts: one 256-column block per wave and
            // expert, every wave the same count
            if (n == 7) k_moe_down_pb<7><<<pgrid, 512, 0, c->stream>>>(a);
            else if (n == 5) k_moe_down_pb<5><<<pgrid, 512, 0, c->stream>>>(a);
            else if (n == 3) k_moe_down_pb<3><<<pgrid, 512, 0, c->stream>>>(a);
            else if (n == 1) k_moe_down_pb<1><<<pgrid, 512, 0, c->stream>>>(a);
            else
#endif
            switch ((n + 1) / 2) {
                case 1: k_moe_down_px<1><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 2: k_moe_down_px<2><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 3: k_moe_down_px<3><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 4: k_moe_down_px<4><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 5: k_moe_down_px<5><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 6: k_moe_down_px<6><<<pgrid, 512, 0, c->stream>>>(a); break;
                case 7: k_moe_down_px<7><<<pgrid, 512, 0, c->stream>>>(a); break;
                default: k_moe_down_px<8><<<pgrid, 512, 0, c->stream>>>(a); break;
            }
        } else if (inter == 2048) k_moe_down<8><<<dgrid, 256, wh_moe_wg_lds(inter), c->stream>>>(a);
        else k_moe_down<0><<<dgrid, 256, wh_moe_wg_lds(inter), c->stream>>>(a);
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// Shape rules shared by the routed-expert entry points; *fast: every expert
// takes the fast kernels.
int moe_shapes(const ExpertView* ev, size_t n, bool* fast) {
    const size_t hidden = ev[0].w1->cols, inter = ev[0].w1->rows, osz = ev[0].w2->rows;
    bool f = osz == hidden && n <= WH_MAX_EXPERTS;
    for (size_t i = 0; i < n; ++i) {
        if (ev[i].w1->cols != hidden || ev[i].w1->rows != inter || ev[i].w2->rows != osz) return WH_INVALID_SHAPE;
        f = f && expert_fast(ev[i]);
    }
    *fast = f;
    return WH_OK;
}

// Routed experts for n_tokens rows of x (all with the same route list).
// x_dev: device input (f32 or bf16).  out_dev: n_tokens x hidden f32.
// ev[0..n): the experts; with has_shared the last one is the shared expert
// (weights route_w cover the routed ones).
int moe_forward(wh_ctx* c, const ExpertView* ev, const float* route_w, size_t n, bool has_shared,
                const void* x_dev, int x_bf16, size_t n_tokens, float* out_dev) {
    const size_t hidden = ev[0].w1->cols, inter = ev[0].w1->rows, osz = ev[0].w2->rows;
    bool fast = false;
    WH_TRY(moe_shapes(ev, n, &fast));
    if (fast) {
        MoeBufs bufs;
        WH_TRY(moe_bufs_ctx(c, n, n_tokens, hidden, inter, &bufs));
        return moe_launch_fast(c, ev, route_w, n, has_shared, x_dev, x_bf16, n_tokens, out_dev, 3u, bufs, true);
    }
    // Generic composition (any shape the reference accepts), one token at a time.
    if (x_bf16) return WH_UNSUPPORTED;
    const size_t per = hidden + 3 * inter + n * osz + n;
    WH_HIP(c->tmp.ensure(per * sizeof(float), false));
    float* xq = c->tmp.as<float>();
    float* g = xq + hidden;
    float* u = g + inter;
    float* hh = u + inter;
    float* ys = hh + inter;
    float* wdev = ys + n * osz;
    WH_HIP(hipMemcpyAsync(wdev, route_w, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    for (size_t tok = 0; tok < n_tokens; ++tok) {
        const float* xt = (const float*)x_dev + tok * hidden;
        for (size_t i = 0; i < n; ++i) {
            WH_HIP(hipMemcpyAsync(xq, xt, hidden * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
            k_act_quant_inplace<<<(unsigned)((hidden + 63) / 64), 256, 0, c->stream>>>(xq, (uint32_t)hidden, 64);
            WH_TRY(launch_fp4(c, *ev[i].w1, xq, g));
            WH_TRY(launch_fp4(c, *ev[i].w3, xq, u));
            k_swiglu_generic<<<(unsigned)((inter + 255) / 256), 256, 0, c->stream>>>(g, u, hh, (uint32_t)inter, c->status);
            k_act_quant_inplace<<<(unsigned)((inter + 63) / 64), 256, 0, c->stream>>>(hh, (uint32_t)inter, 64);
            WH_TRY(launch_fp4(c, *ev[i].w2, hh, ys + i * osz));
        }
        k_combine_generic<<<(unsigned)((osz + 255) / 256), 256, 0, c->stream>>>(
            ys, wdev, (uint32_t)n, has_shared ? 1u : 0u, (uint32_t)osz, out_dev + tok * osz);
        WH_HIP(hipGetLastError());
    }
    return WH_OK;
}

// splitmix64 finaliser, the counter-based generator of the synthetic weights
__host__ __device__ inline uint64_t wh_mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__host__ __device__ inline uint8_t wh_synth_byte(uint64_t seed, uint64_t stream, uint64_t i) {
    uint64_t v = wh_mix64(seed ^ wh_mix64(stream * 0x100000001b3ull + (i >> 3)));
    return (uint8_t)(v >> (8 * (i & 7)));
}

// Resident dword (blk, l, d) of one FP4 row (layout described with the FP4
// kernels in kernels.h) from the row's original nibbles, nib(col).
template <class Nib>
__host__ __device__ inline uint32_t wh_fp4_resident_word(const Nib& nib, uint32_t blk, uint32_t l, uint32_t d) {
    const size_t g = (size_t)8 * blk + 2 * d;
    uint32_t a[4], b[4];
    for (uint32_t k = 0; k < 4; ++k) {
        a[k] = nib(32 * g + l + 8 * k);
        b[k] = nib(32 * (g + 1) + l + 8 * k);
    }
    return wh_fp4_encode_word(a, b);
}

// Raw FP4 rows (the reference's [row][cols/2] bytes, low nibble = even
// column) -> the resident layout: one thread per resident dword.  cols is a
// multiple of 256; raw and w both hold `rows` rows of cols/2 bytes.
__global__ void k_fp4_relayout(const uint8_t* __restrict__ raw, uint8_t* __restrict__ w, uint32_t rows,
                               uint32_t cols) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t blocks = cols / 256;
    if (id >= (size_t)rows * blocks * 32) return;
    const uint32_t d = id & 3, l = (id >> 2) & 7;
    const size_t rb = id >> 5;
    const uint32_t blk = rb % blocks;
    const size_t rowbase = (rb / blocks) * (cols / 2);
    const uint8_t* src = raw + rowbase;
    auto nib = [src](size_t col) -> uint32_t {
        const uint8_t b = src[col >> 1];
        return (col & 1) ? (b >> 4) : (b & 15);
    };
    ((uint32_t*)(w + rowbase + (size_t)blk * 128 + l * 16))[d] = wh_fp4_resident_word(nib, blk, l, d);
}

// Device synthetic FP4 tensor straight into the resident layout: each
// thread builds one weight dword (or one scale byte) from the generated
// original bytes.
__global__ void k_synth_fp4(uint8_t* w, uint8_t* s, uint32_t rows, uint32_t cols, uint64_t seed,
                            uint64_t stream, uint32_t slo, uint32_t shi) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t blocks = cols / 256, G = cols / 32;
    const size_t words = (size_t)rows * blocks * 32;
    if (id < words) {
        const uint32_t d = id & 3, l = (id >> 2) & 7;
        const size_t rb = id >> 5;
        const uint32_t blk = rb % blocks;
        const size_t row = rb / blocks;
        const size_t rowbase = row * (cols / 2);
        auto nib = [&](size_t col) -> uint32_t {
            uint8_t b = wh_synth_byte(seed, stream, rowbase + (col >> 1));
            return (col & 1) ? (b >> 4) : (b & 15);
        };
        ((uint32_t*)(w + rowbase + (size_t)blk * 128 + l * 16))[d] = wh_fp4_resident_word(nib, blk, l, d);
    }
    const size_t nscale = (size_t)rows * G;
    if (id < nscale) {
        uint32_t span = shi - slo + 1;
        s[id] = (uint8_t)(slo + wh_synth_byte(seed, stream ^ 0x5ca1e5ull, id) % span);
    }
}

// Synthetic FP8 byte: approximately uniform over the 254 finite E4M3 codes
// (0x7F and 0xFF excluded), from the same counter-based generator.
__host__ __device__ inline uint8_t wh_fp8_synth_code(uint64_t seed, uint64_t stream, uint64_t i) {
    const uint32_t r = wh_synth_byte(seed, stream, i) % 254u;
    return (uint8_t)(r < 127u ? r : r + 1u);
}

// Device synthetic FP8 tensor straight into the resident lane layout: one
// thread per resident byte, reading the generated byte of its original column.
__global__ void k_synth_fp8(uint8_t* w, uint32_t rows, uint32_t cols, uint64_t seed, uint64_t stream) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)rows * cols) return;
    const size_t row = id / cols;
    const uint32_t rc = (uint32_t)(id - row * cols);
    const uint32_t g = rc >> 7, l = (rc & 127) >> 4, i = rc & 15;
    const uint32_t col = g * 128 + (i & 7) * 16 + (i >> 3) * 8 + l;
    w[id] = wh_fp8_synth_code(seed, stream, row * cols + col);
}

// ------------------------------------------------------ batched routed experts
// Device table of a layer's experts (ids < n), rebuilt when the layer's store
// entries changed.  Experts of any shape may be resident; the fast batch
// path needs one fast shape for all of them.
int layer_table(wh_ctx* c, uint32_t layer, LayerTable** out) {
    LayerTable& t = c->tables[layer];
    *out = &t;
    if (t.valid) return WH_OK;
    auto lo = c->experts.lower_bound({layer, 0u});
    auto hi = c->experts.upper_bound({layer, 0xffffffffu});
    uint32_t n = 0;
    for (auto it = lo; it != hi; ++it) n = std::max(n, it->first.second + 1);
    std::vector<wh_expert_ptrs> host(n);
    std::memset(host.data(), 0, n * sizeof(wh_expert_ptrs));
    bool fast = n > 0 && n < WH_BATCH_MAX_TABLE;  // one id stays free for the shared expert
    bool zero_scale = false;
    uint32_t resident = 0;
    size_t hidden = 0, inter = 0;
    for (auto it = lo; it != hi; ++it) {
        ExpertView v;
        if (resolve_expert(c, layer, it->first.second, &v) != WH_OK) continue;  // released tensors
        ++resident;
        if (hidden == 0) {
            hidden = v.w1->cols;
            inter = v.w1->rows;
        }
        fast = fast && expert_fast(v) && v.w1->cols == hidden && v.w1->rows == inter && v.w2->rows == hidden;
        zero_scale = zero_scale || expert_zero_scale(v);
        wh_expert_ptrs& p = host[it->first.second];
        p.w1 = v.w1->w;
        p.s1 = (const uint8_t*)v.w1->s;
        p.w3 = v.w3->w;
        p.s3 = (const uint8_t*)v.w3->s;
        p.w2 = v.w2->w;
        p.s2 = (const uint8_t*)v.w2->s;
    }
    // kernels of earlier calls may still read the old table
    WH_HIP(hipStreamSynchronize(c->stream));
    if (n > t.cap) {
        c->retire.drop(t.dev);
        t.dev = nullptr;
        t.cap = 0;
        WH_HIP(hipMalloc((void**)&t.dev, n * sizeof(wh_expert_ptrs)));
        t.cap = n;
    }
    if (n) WH_HIP(hipMemcpy(t.dev, host.data(), n * sizeof(wh_expert_ptrs), hipMemcpyHostToDevice));
    t.n = n;
    t.fast = fast;
    t.zero_scale = zero_scale;
    t.resident = resident;
    t.hidden = hidden;
    t.inter = inter;
    t.valid = true;
    return WH_OK;
}

// Workgroups of a persistent kernel that fit on the device at once.
int persistent_grid(const void* kernel, size_t lds, unsigned* grid, int threads = 256) {
    static std::mutex mu;
    static std::map<std::pair<const void*, size_t>, unsigned> cache;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find({kernel, lds});
    if (it != cache.end()) {
        *grid = it->second;
        return WH_OK;
    }
    int dev = 0, cus = 0, per_cu = 0;
    WH_HIP(hipGetDevice(&dev));
    WH_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    WH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds));
    *grid = (unsigned)std::max(1, cus * std::max(1, per_cu));
    cache[{kernel, lds}] = *grid;
    return WH_OK;
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Device layout of one batch chunk inside c->batch.
struct BatchBufs {
    float* wgt;
    uint32_t *sorted, *uexp, *uoff, *uorder, *acc_order, *meta, *pos;
    wh_bmx_vt* vtab;
    float *xq, *g, *u, *hq, *y;
    uint8_t *xq8, *xs8, *hq8, *hs8;
};
int batch_bufs(wh_ctx* c, size_t npos, size_t slots, size_t hidden, size_t inter, BatchBufs* b) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += align256(bytes);
        return o;
    };
    // meta first: its flag word keeps its place whatever the sizes
    const size_t o_me = take(16 * 4), o_w = take(slots * 4), o_so = take(slots * 4), o_ue = take(slots * 4),
                 o_uo = take((slots + 1) * 4), o_ur = take(slots * 4), o_ac = take(slots * 4),
                 o_xq = take(npos * hidden * 4), o_g = take(slots * inter * 4), o_u = take(slots * inter * 4),
                 o_y = take(slots * hidden * 4),
                 o_hq = take(slots * inter * 4), o_xq8 = take(npos * hidden), o_xs8 = take(npos * hidden / 32),
                 o_hq8 = take(slots * inter), o_hs8 = take(slots * inter / 32),
                 o_vt = take(slots * sizeof(wh_bmx_vt)), o_pos = take(slots * 4);
    WH_HIP(c->batch.ensure(off, true));  // zeroed when (re)allocated: meta's flag starts clear
    uint8_t* base = c->batch.as<uint8_t>();
    b->wgt = (float*)(base + o_w);
    b->sorted = (uint32_t*)(base + o_so);
    b->uexp = (uint32_t*)(base + o_ue);
    b->uoff = (uint32_t*)(base + o_uo);
    b->uorder = (uint32_t*)(base + o_ur);
    b->acc_order = (uint32_t*)(base + o_ac);
    b->meta = (uint32_t*)(base + o_me);
    b->xq = (float*)(base + o_xq);
    b->g = (float*)(base + o_g);
    b->u = (float*)(base + o_u);
    b->y = (float*)(base + o_y);
    b->hq = (float*)(base + o_hq);
    b->xq8 = base + o_xq8;
    b->xs8 = base + o_xs8;
    b->hq8 = base + o_hq8;
    b->hs8 = base + o_hs8;
    b->vtab = (wh_bmx_vt*)(base + o_vt);
    b->pos = (uint32_t*)(base + o_pos);
    return WH_OK;
}

// Fast batch path over positions [0, npos) in chunks of at most
// WH_BATCH_MAX_ASSIGN slots; positions are independent, so chunking changes
// no result.  ids/scores/x/out are device pointers.
int moe_batch_fast(wh_ctx* c, const LayerTable& t, const uint32_t* ids, const float* scores, size_t npos,
                   size_t topk, const ExpertView* shared, const void* x, int x_bf16, float* out) {
    const size_t hidden = t.hidden, inter = t.inter;
    const size_t per_pos = topk + (shared ? 1 : 0);
    const size_t chunk = WH_BATCH_MAX_ASSIGN / per_pos;
    BatchBufs b;
    WH_TRY(batch_bufs(c, std::min(npos, chunk), std::min(npos, chunk) * per_pos, hidden, inter, &b));
    const void* kg = hidden == 4096 ? (const void*)k_moe_batch_gateup<16> : (const void*)k_moe_batch_gateup<0>;
    const void* kd = inter == 2048 ? (const void*)k_moe_batch_down<8> : (const void*)k_moe_batch_down<0>;
    const size_t lds_g = wh_batch_wg_lds(hidden), lds_d = wh_batch_wg_lds(inter);
    unsigned grid_g = 0, grid_d = 0;
    WH_TRY(persistent_grid(kg, lds_g, &grid_g));
    WH_TRY(persistent_grid(kd, lds_d, &grid_d));
    // With exact numerics off the MFMA experts run in k_moe_batch_mx (one
    // 512-thread workgroup per CU) and the other kernels keep the exact ones.
    // a UE8M0 scale byte 0 anywhere in the call's experts: every expert on
    // the exact items (the MFMA would read the byte as 2^-127)
    const bool zero_scale = t.zero_scale || (shared && expert_zero_scale(*shared));
    const bool mx = !c->exact && !zero_scale && c->moe_mfma_min && inter == 2048 && (hidden == 4096 || hidden == 2048) &&
                    wh_bmx_lds(hidden) <= g_max_lds;
    const void* kmg = hidden == 4096 ? (const void*)k_moe_batch_mx<4096, true> : (const void*)k_moe_batch_mx<2048, true>;
    const void* kmd = (const void*)k_moe_batch_mx<2048, false>;
    unsigned grid_mg = 0, grid_md = 0;
    if (mx) {
        WH_TRY(persistent_grid(kmg, wh_bmx_lds(hidden), &grid_mg, 512));
        WH_TRY(persistent_grid(kmd, wh_bmx_lds(inter), &grid_md, 512));
    }
    for (size_t p0 = 0; p0 < npos; p0 += chunk) {
        const size_t n = std::min(chunk, npos - p0), slots = n * per_pos;
        wh_batch_args a;
        std::memset(&a, 0, sizeof a);
        a.table = t.dev;
        a.n_table = t.n;
        a.route_ids = ids + p0 * topk;
        a.route_scores = scores + p0 * topk;
        a.npos = (uint32_t)n;
        a.topk = (uint32_t)topk;
        a.hidden = (uint32_t)hidden;
        a.inter = (uint32_t)inter;
        a.x = x_bf16 ? (const void*)((const uint16_t*)x + p0 * hidden) : (const void*)((const float*)x + p0 * hidden);
        a.x_is_bf16 = x_bf16 ? 1u : 0u;
        if (shared) {
            a.has_shared = 1;
            a.shared.w1 = shared->w1->w;
            a.shared.s1 = (const uint8_t*)shared->w1->s;
            a.shared.w3 = shared->w3->w;
            a.shared.s3 = (const uint8_t*)shared->w3->s;
            a.shared.w2 = shared->w2->w;
            a.shared.s2 = (const uint8_t*)shared->w2->s;
        }
        a.wgt = b.wgt;
        a.sorted = b.sorted;
        a.uexp = b.uexp;
        a.uoff = b.uoff;
        a.uorder = b.uorder;
        a.acc_order = b.acc_order;
        a.meta = b.meta;
        a.vtab = b.vtab;
        a.pos = b.pos;
        a.xq = b.xq;
        a.xq8 = b.xq8;
        a.xs8 = b.xs8;
        a.g = b.g;
        a.u = b.u;
        a.hq = b.hq;
        a.hq8 = b.hq8;
        a.hs8 = b.hs8;
        a.y = b.y;
        a.mfma_min = (c->exact || zero_scale) ? 0u : c->moe_mfma_min;  // exact numerics: every expert on the exact items
        a.mfma_external = mx ? 1u : 0u;
        // threshold 1: every used expert is an MFMA expert, so the exact-item
        // kernels would only run after an inf or NaN input; k_moe_batch_mx
        // covers that case and they are not launched
        const bool fb = mx && a.mfma_min == 1;
        a.mx_fallback = fb ? 1u : 0u;
        a.out = out + p0 * hidden;
        a.status = c->status;
        // the most items the queues can hold: used experts <= min(slots, ids),
        // and an expert has fewer MFMA items than exact ones
        const size_t max_used = std::min(slots, (size_t)t.n + (shared ? 1 : 0));
        const unsigned gg = (unsigned)std::min<size_t>(grid_g, max_used * (inter / 16));
        const unsigned gd = (unsigned)std::min<size_t>(grid_d, max_used * (hidden / 32));
        // workgroup 0 packs, the others act-quantize x
        k_moe_batch_pack<<<1 + (unsigned)((n * hidden / 16 + 255) / 256), 256, 0, c->stream>>>(a);
        if (mx) {
            if (hidden == 4096) k_moe_batch_mx<4096, true><<<grid_mg, 512, wh_bmx_lds(4096), c->stream>>>(a);
            else k_moe_batch_mx<2048, true><<<grid_mg, 512, wh_bmx_lds(2048), c->stream>>>(a);
        }
        if (!fb) {
            if (hidden == 4096) k_moe_batch_gateup<16><<<gg, 256, lds_g, c->stream>>>(a);
            else k_moe_batch_gateup<0><<<gg, 256, lds_g, c->stream>>>(a);
        }
        c->moe_last_slots = npos <= chunk ? slots : 0;
        c->moe_last_npos = n;
        c->moe_last_hidden = hidden;
        c->moe_last_inter = inter;
        k_moe_batch_swiglu_quant<<<(unsigned)((slots * inter / 4 + 255) / 256), 256, 0, c->stream>>>(
            a.g, a.u, (uint32_t)(slots * inter), a.hq, a.hq8, a.hs8);
        if (mx) k_moe_batch_mx<2048, false><<<grid_md, 512, wh_bmx_lds(2048), c->stream>>>(a);
        if (!fb) {
            if (inter == 2048) k_moe_batch_down<8><<<gd, 256, lds_d, c->stream>>>(a);
            else k_moe_batch_down<0><<<gd, 256, lds_d, c->stream>>>(a);
        }
        k_moe_batch_accumulate<<<dim3((unsigned)((hidden + 255) / 256), (unsigned)n), 256, 0, c->stream>>>(a);
        WH_HIP(hipGetLastError());
    }
    return WH_OK;
}

// acc[i] = acc[i] + y[i] * w, unfused (E/compute.rs:1804-1807)
__global__ void k_axpy_unfused(float* acc, const float* y, float w, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = y[i] * w;
        acc[i] = acc[i] + v;
    }
}
// out[i] = shared[i] + out[i] (E/compute.rs:1845-1848)
__global__ void k_add_shared(float* out, const float* sh, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = sh[i] + out[i];
}

// Per-position weights of the batch path (E/server/generation.rs:2495-2503).
void batch_weights(const float* sc, size_t topk, float* w) {
    float sum = 0.0f;
    bool finite = true;
    for (size_t k = 0; k < topk; ++k) {
        finite = finite && std::fabs(sc[k]) <= 3.4028235e38f;
        sum = sum + sc[k];
    }
    finite = finite && std::fabs(sum) <= 3.4028235e38f && sum > 0.0f;
    const float uniform = 1.0f / (float)topk;
    for (size_t k = 0; k < topk; ++k) w[k] = finite ? sc[k] / sum : uniform;
}

// Generic batch path (any shape the single-expert path accepts): the union
// is built on the host and each (expert, position) runs the expert forward.
// ids/scores are host arrays; x (f32) and out are device pointers.
int moe_batch_generic(wh_ctx* c, uint32_t layer, const uint32_t* ids, const float* scores, size_t npos,
                      size_t topk, const ExpertView* shared, const float* x, float* out) {
    std::map<uint32_t, std::vector<std::pair<size_t, float>>> uni;
    std::vector<float> w(topk);
    size_t hidden = 0, osz = 0;
    for (size_t p = 0; p < npos; ++p) {
        batch_weights(scores + p * topk, topk, w.data());
        for (size_t k = 0; k < topk; ++k) uni[ids[p * topk + k]].push_back({p, w[k]});
    }
    std::vector<std::pair<uint32_t, ExpertView>> ev;
    for (auto& kv : uni) {
        ExpertView v;
        WH_TRY(resolve_expert(c, layer, kv.first, &v));
        if (hidden == 0) {
            hidden = v.w1->cols;
            osz = v.w2->rows;
        }
        if (v.w1->cols != hidden || v.w2->rows != osz) return WH_INVALID_SHAPE;
        ev.push_back({kv.first, v});
    }
    if (shared && (shared->w1->cols != hidden || shared->w2->rows != osz)) return WH_INVALID_SHAPE;
    if (osz != hidden) return WH_INVALID_SHAPE;  // routed_acc rows are hidden wide
    WH_HIP(c->y_out.ensure(osz * sizeof(float), false));
    float* y = c->y_out.as<float>();
    WH_HIP(hipMemsetAsync(out, 0, npos * osz * sizeof(float), c->stream));
    const float one = 1.0f;
    const unsigned blocks = (unsigned)((osz + 255) / 256);
    for (auto& e : ev) {
        for (auto& tgt : uni[e.first]) {
            WH_TRY(moe_forward(c, &e.second, &one, 1, false, x + tgt.first * hidden, 0, 1, y));
            k_axpy_unfused<<<blocks, 256, 0, c->stream>>>(out + tgt.first * osz, y, tgt.second, (uint32_t)osz);
        }
    }
    if (shared) {
        for (size_t p = 0; p < npos; ++p) {
            WH_TRY(moe_forward(c, shared, &one, 1, false, x + p * hidden, 0, 1, y));
            k_add_shared<<<blocks, 256, 0, c->stream>>>(out + p * osz, y, (uint32_t)osz);
        }
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int store_tensor_common(wh_ctx* c, Tensor&& t, wh_tensor* out) {
    wh_tensor id = c->next_id++;
    c->tensors.emplace(id, std::move(t));
    *out = id;
    return WH_OK;
}

// Host -> device copy on the context stream.  A pinned source is queued; a
// pageable one goes through the pinned staging buffer in 64 MB pieces and
// has landed when the call returns.
int h2d(wh_ctx* c, void* dst, const uint8_t* src, size_t n, bool pinned) {
    if (n == 0) return WH_OK;
    if (pinned) {
        WH_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
        return WH_OK;
    }
    const size_t piece = size_t(64) << 20;
    WH_HIP(c->stage_in.ensure(std::min(n, piece)));
    for (size_t o = 0; o < n; o += piece) {
        const size_t k = std::min(piece, n - o);
        std::memcpy(c->stage_in.p, src + o, k);
        WH_HIP(hipMemcpyAsync((uint8_t*)dst + o, c->stage_in.p, k, hipMemcpyHostToDevice, c->stream));
        WH_HIP(hipStreamSynchronize(c->stream));
    }
    return WH_OK;
}

// One FP4 tensor from host bytes in the reference layout into a new
// resident tensor.  Shapes the fast kernels take (32 columns per scale,
// cols % 256 == 0) go up raw through the `relayout` scratch and
// k_fp4_relayout writes the lane layout; other shapes keep the row-major
// bytes.  With a pinned source the copies stay queued on the stream (the
// caller keeps the source alive until the stream passes them); otherwise the
// tensor is complete on return.  Shape rules are validate_fp4_matvec's
// (E/deepseek_v4.rs:434-462) minus the per-call input/output lengths.
int store_fp4_upload(wh_ctx* c, const uint8_t* packed, size_t packed_len, const uint8_t* scales, size_t scales_len,
                     size_t rows, size_t cols, size_t scale_cols, bool pinned, wh_tensor* out) {
    if (rows == 0 || cols == 0 || scale_cols == 0) return WH_EMPTY_SHAPE;
    if (cols % scale_cols != 0) return WH_INVALID_SHAPE;
    const size_t row_bytes = (cols + 1) / 2;
    if (rows > SIZE_MAX / row_bytes || rows > SIZE_MAX / scale_cols) return WH_INVALID_SHAPE;
    if (packed_len < rows * row_bytes) return WH_PACKED_WEIGHT_TOO_SMALL;
    if (scales_len < rows * scale_cols) return WH_SCALE_TOO_SMALL;
    Tensor t;
    t.kind = kFp4;
    t.rows = rows;
    t.cols = cols;
    t.scale_rows = rows;
    t.scale_cols = scale_cols;
    t.fast = (cols / scale_cols == 32) && cols % 256 == 0 && wh_fp4_wg_lds(cols) <= g_max_lds &&
             rows <= UINT32_MAX && cols <= UINT32_MAX;
    t.bytes = rows * row_bytes + rows * scale_cols;
    t.zero_scale = std::memchr(scales, 0, rows * scale_cols) != nullptr;
    WH_TRY(alloc_tensor(c, t, rows * row_bytes, rows * scale_cols));
    if (t.fast) {
        const size_t piece = size_t(64) << 20;
        const size_t chunk_rows = std::max<size_t>(1, piece / row_bytes);
        const size_t need = std::max(piece, row_bytes);
        if (need > c->relayout.n) WH_HIP(hipStreamSynchronize(c->stream));  // queued relayouts may read it
        WH_HIP(c->relayout.ensure(need, false));
        for (size_t r = 0; r < rows; r += chunk_rows) {
            const size_t nr = std::min(chunk_rows, rows - r);
            // stream order keeps this copy behind the previous piece's relayout
            WH_TRY(h2d(c, c->relayout.p, packed + r * row_bytes, nr * row_bytes, pinned));
            const size_t words = nr * (cols / 256) * 32;
            k_fp4_relayout<<<(unsigned)((words + 255) / 256), 256, 0, c->stream>>>(
                c->relayout.as<uint8_t>(), t.w + r * row_bytes, (uint32_t)nr, (uint32_t)cols);
            WH_HIP(hipGetLastError());
        }
    } else {
        WH_TRY(h2d(c, t.w, packed, rows * row_bytes, pinned));
    }
    WH_TRY(h2d(c, t.s, scales, rows * scale_cols, pinned));
    if (!pinned) WH_HIP(hipStreamSynchronize(c->stream));
    return store_tensor_common(c, std::move(t), out);
}

// Thread's error text: the reference's Display string of a block error,
// prefixed with `where` when given.
void set_block_error(const whqb::Error& e, const char* where) {
    char text[200];
    whqb::describe(e, text, sizeof text);
    if (where && *where)
        std::snprintf(g_last_error, sizeof g_last_error, "%s: %s", where, text);
    else
        std::snprintf(g_last_error, sizeof g_last_error, "%s", text);
}

int block_status(const whqb::Error& e) {
    switch (e.kind) {
        case whqb::Fail::None: return WH_OK;
        case whqb::Fail::Truncated: return WH_TRUNCATED_QUANT_BLOCK;
        case whqb::Fail::Magic: return WH_INVALID_QUANT_BLOCK_MAGIC;
        case whqb::Fail::Version: return WH_UNSUPPORTED_QUANT_BLOCK_VERSION;
        case whqb::Fail::Invalid: return WH_INVALID_QUANT_BLOCK;
        case whqb::Fail::Shape: return WH_INVALID_SHAPE;
    }
    return WH_INVALID_QUANT_BLOCK;
}

// Keys an expert whose tensors the library created; the tensors of an
// expert it replaces go with it if the library created those too.
void register_owned_expert(wh_ctx* c, uint32_t layer, uint32_t expert, const wh_tensor ids[3]) {
    auto it = c->experts.find({layer, expert});
    if (it != c->experts.end() && it->second.owned)
        for (wh_tensor old : {it->second.w1, it->second.w3, it->second.w2}) drop_tensor(c, old);
    c->experts[{layer, expert}] = Expert{ids[0], ids[1], ids[2], true};
    c->tables[layer].valid = false;
}

// ---------------------------------------------------------------- router

// The reference's InvalidShape(what) / InvalidQuantBlock(what) as a status
// and the Display text in the thread's error string.
int shape_error(const char* what) {
    std::snprintf(g_last_error, sizeof g_last_error, "invalid compute shape: %s", what);
    return WH_INVALID_SHAPE;
}

bool name_contains_ci(const whqb::Reader& r, const whqb::Tensor& t, const char* needle) {
    const size_t n = std::strlen(needle);
    const uint8_t* p = r.data() + t.name_off;
    for (size_t i = 0; i + n <= t.name_len; ++i) {
        size_t k = 0;
        while (k < n && std::tolower(p[i + k]) == needle[k]) ++k;
        if (k == n) return true;
    }
    return false;
}

constexpr uint32_t kRoleRouter = 9;  // TensorRole::Router, E/compute.rs:455-471

// bf16 row-major [rows][cols] -> the router kernel's layout (cols % 128 ==
// 0): per 128-column block, chain q = 8a + l (accumulator a, AVX lane l)
// holds its values of chunks 0..7 in 16 contiguous bytes.
void bf16_router_layout(const uint16_t* src, uint16_t* dst, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < cols / 128; ++b)
            for (size_t q = 0; q < 16; ++q)
                for (size_t j = 0; j < 8; ++j)
                    dst[r * cols + 128 * b + 8 * q + j] = src[r * cols + 128 * b + 16 * j + 8 * (q >> 3) + (q & 7)];
}

// router_bias_values (E/compute.rs:2335-2376): the first Router-role rank-1
// tensor named *bias* with at least `rows` values in f32 (dtype 12) or bf16
// (dtype 11), as f32.
int router_bias(const whqb::Reader& r, const whqb::Header& h, size_t rows, std::vector<float>* out, bool* found,
                LookupError* err) {
    *found = false;
    for (size_t i = 0; i < h.tensor_count; ++i) {
        whqb::Tensor t;
        whqb::Error e;
        if (!whqb::tensor_at(r, h, i, &t, &e)) {
            set_block_error(e, nullptr);
            err->status = block_status(e);
            err->text = g_last_error;
            return err->status;
        }
        if ((t.flags & 0xffff) != kRoleRouter || t.rank != 1 || !name_contains_ci(r, t, "bias")) continue;
        if ((size_t)t.dim(r, 0) < rows) continue;
        if (t.dtype_original != 12 && t.dtype_original != 11) continue;
        const size_t elem = t.dtype_original == 12 ? 4 : 2;
        if (t.data_len < rows * elem) {
            err->status = shape_error(elem == 4 ? "router bias out of range" : "BF16 tensor value out of range");
            err->text = g_last_error;
            return err->status;
        }
        out->resize(rows);
        const uint8_t* d = r.data() + t.data_off;
        for (size_t k = 0; k < rows; ++k) {
            if (elem == 4) {
                std::memcpy(&(*out)[k], d + 4 * k, 4);
            } else {
                uint16_t v;
                std::memcpy(&v, d + 2 * k, 2);
                const uint32_t bits = (uint32_t)v << 16;
                std::memcpy(&(*out)[k], &bits, 4);
            }
        }
        *found = true;
        return WH_OK;
    }
    return WH_OK;
}

// The token's tid2eid row (tid2eid_expert_ids, E/compute.rs:2287-2333).
int router_hash_row(const Router& rt, uint64_t token, uint32_t* ids, uint32_t* n) {
    size_t elem = 0;
    if (rt.table_dtype == 7) elem = 4;
    else if (rt.table_dtype == 9) elem = 8;
    else return shape_error("tid2eid table has unsupported dtype");
    if (token >= rt.table_rows) return shape_error("tid2eid token id out of range");
    const size_t top_k = rt.table_cols;
    const size_t row_bytes = top_k * elem, start = (size_t)token * row_bytes;
    if (start + row_bytes > rt.table.size()) return shape_error("tid2eid row out of range");
    if (top_k > WH_ROUTER_MAX_HASH) {
        std::snprintf(g_last_error, sizeof g_last_error, "tid2eid rows of %zu ids exceed %u", top_k, WH_ROUTER_MAX_HASH);
        return WH_UNSUPPORTED;
    }
    for (size_t k = 0; k < top_k; ++k) {
        int64_t v;
        if (elem == 4) {
            int32_t v32;
            std::memcpy(&v32, rt.table.data() + start + 4 * k, 4);
            v = v32;
        } else {
            std::memcpy(&v, rt.table.data() + start + 8 * k, 8);
        }
        if (v < 0) return shape_error("tid2eid negative expert id");
        ids[k] = (uint32_t)v;
    }
    *n = (uint32_t)top_k;
    return WH_OK;
}

// Everything of route_experts_from_dense_block that runs on the host before
// the kernels: the argument checks in the reference's order, the hash row,
// the bias lookup's outcome.  Fills the selection arguments except the
// pointers.
int router_prepare(const Router& rt, const wh_route_options& o, size_t hidden_len, size_t active, size_t n_avail,
                   wh_router_sel* sa) {
    if (hidden_len < rt.cols) return shape_error("router input too small");
    std::memset(sa, 0, sizeof *sa);
    sa->rows = (uint32_t)rt.rows;
    sa->active = (uint32_t)active;
    sa->n_avail = (uint32_t)n_avail;
    sa->math = o.math == WH_ROUTER_SQRT_SOFTPLUS ? 1u : 0u;
    sa->route_scale = o.route_scale;
    if (o.hash_token_id >= 0 && rt.has_table) {
        if (rt.table_err.status != WH_OK) {
            std::snprintf(g_last_error, sizeof g_last_error, "%s", rt.table_err.text.c_str());
            return rt.table_err.status;
        }
        WH_TRY(router_hash_row(rt, (uint64_t)o.hash_token_id, sa->hash, &sa->n_hash));
        if (sa->n_hash == 0) sa->active = 0;  // an empty row routes nowhere
        return WH_OK;
    }
    if (sa->math && rt.bias_err.status != WH_OK) {
        std::snprintf(g_last_error, sizeof g_last_error, "%s", rt.bias_err.text.c_str());
        return rt.bias_err.status;
    }
    return WH_OK;
}

// What the experts of one token with a device route list need from the
// host: the layer's expert table, the shared expert, the one fast shape.
struct MoeDevPrep {
    LayerTable* t = nullptr;
    wh_expert_ptrs shp = {};
    bool has_shared = false, zero_scale = false;
    size_t n_slots = 0, hidden = 0, inter = 0;
    wh_moe_dyn* dyn = nullptr;
};

// Gate GEMV then selection, on the context stream.  x: device f32 [cols];
// avail: device ids or null; logits: device scratch [rows].
int router_launch(wh_ctx* c, const Router& rt, wh_router_sel sa, const float* x, const uint32_t* avail,
                  float* logits, uint32_t* ids, float* scores, uint32_t* count, const MoeDevPrep* rs = nullptr,
                  bool* resolved = nullptr) {
    const unsigned rows = (unsigned)rt.rows, cols = (unsigned)rt.cols;
    sa.logits = logits;
    sa.bias = sa.math ? rt.bias : nullptr;
    sa.avail = avail;
    sa.out_ids = ids;
    sa.out_scores = scores;
    sa.out_count = count;
    if (rt.gate == kGateBf16) {  // one launch: the last workgroup selects
        // each workgroup's 4 candidates published in selection order where
        // the candidates are exactly the rows (the scratch holds 3 words a row)
        sa.sorted = (!avail && sa.n_hash == 0 && rows % 4 == 0 && rows <= 256) ? 1u : 0u;
        if (sa.sorted && rs && rs->n_slots <= 64) {  // the last arriver also resolves the routes
            sa.rs_out = rs->dyn;
            sa.rs_table = rs->t->dev;
            sa.rs_table_n = (uint32_t)rs->t->n;
            sa.rs_slots = (uint32_t)rs->n_slots;
            sa.rs_has_shared = rs->has_shared ? 1u : 0u;
            sa.rs_status = c->status;
            sa.rs_shared = rs->shp;
            *resolved = true;
        }
        WH_HIP(c->rtr_cnt.ensure(sizeof(uint32_t), true));
        auto kern = sa.rs_out ? k_router_bf16<true> : k_router_bf16<false>;
        kern<<<(rows + 3) / 4, 64, cols * sizeof(float), c->stream>>>(rt.bf16, x, cols, sa, c->rtr_cnt.as<uint32_t>(),
                                                                      0, 0);
        WH_HIP(hipGetLastError());
        return WH_OK;
    }
    if (rt.gate == kGateBf16Rows) {
        k_router_gemv_bf16_generic<<<(rows + 63) / 64, 64, 0, c->stream>>>(rt.bf16, x, rows, cols, logits);
    } else {
        Tensor* t = find_tensor(c, rt.fp8);
        if (!t) return WH_NOT_RESIDENT;
        WH_TRY(launch_fp8(c, *t, 0, t->rows, x, logits, 1, 0, 0, 0, 0, nullptr, 0, 0, nullptr, false));
    }
    k_router_select<<<1, 256, 0, c->stream>>>(sa);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// The router of npos inputs (x: npos rows x_ld floats apart; ids and scores
// npos x active, count npos), each as wh_route_experts_async routes it: one
// launch for a bf16 gate of at most 256 rows (a multiple of 4) without an
// available list or a hash row, else one call per input.  token_ids: each
// input's hash token, or null for opts->hash_token_id.  The caller holds
// c->mu.
int route_batch(wh_ctx* c, uint32_t layer, const float* x, size_t x_ld, size_t hidden_len, size_t npos,
                size_t active, const uint32_t* avail, size_t n_avail, const wh_route_options& opts,
                const int64_t* token_ids, uint32_t* ids, float* scores, uint32_t* count) {
    auto it = c->routers.find(layer);
    if (it == c->routers.end()) return WH_NOT_RESIDENT;
    const Router& rt = it->second;
    bool hashed = false;
    for (size_t i = 0; i < npos; ++i) hashed = hashed || (token_ids ? token_ids[i] : opts.hash_token_id) >= 0;
    hashed = hashed && rt.has_table;
    const bool one = rt.gate == kGateBf16 && !avail && !hashed && active > 0 && rt.rows % 4 == 0 &&
                     rt.rows <= 256 && npos <= 65535 && x_ld <= 0xffffffffu && ((uintptr_t)x & 15) == 0 &&
                     (x_ld & 3) == 0;
    if (!one) {
        for (size_t i = 0; i < npos; ++i) {
            wh_route_options o = opts;
            if (token_ids) o.hash_token_id = token_ids[i];
            WH_TRY(wh_route_experts_async(c, layer, x + i * x_ld, hidden_len, active, avail, n_avail, &o,
                                          ids + i * active, scores + i * active, count + i));
        }
        return WH_OK;
    }
    if (active > WH_ROUTER_MAX_ACTIVE) return WH_UNSUPPORTED;
    wh_route_options o = opts;
    o.hash_token_id = -1;
    wh_router_sel sa;
    WH_TRY(router_prepare(rt, o, hidden_len, active, rt.rows, &sa));
    const size_t pub_ld = 3 * rt.rows;  // (key, score) u64 and the row id per row, a multiple of 2 words
    WH_HIP(c->rtr.ensure((rt.cols + npos * pub_ld) * 4, false));
    WH_HIP(c->rtr_cnt.ensure(npos * sizeof(uint32_t), true));
    sa.logits = c->rtr.as<float>() + rt.cols;
    sa.bias = sa.math ? rt.bias : nullptr;
    sa.out_ids = ids;
    sa.out_scores = scores;
    sa.out_count = count;
    sa.sorted = 1;
    k_router_bf16<false><<<dim3((unsigned)(rt.rows / 4), (unsigned)npos), 64, rt.cols * sizeof(float), c->stream>>>(
        rt.bf16, x, (uint32_t)rt.cols, sa, c->rtr_cnt.as<uint32_t>(), (uint32_t)x_ld, (uint32_t)pub_ld);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// Once per GPU, with that GPU current: the device address of its copy of
// noalloc_scratch.
int noalloc_setup(int device) {
    if (device >= kMaxDevices) return WH_OK;  // the allocation-free entry point then reports Unsupported
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return WH_OK;
    void* p = nullptr;
    WH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch)));
    g_noalloc_ptr[device] = p;
    return WH_OK;
}

// Drops a layer's router and returns its HBM to the arena.
void drop_router(wh_ctx* c, uint32_t layer) {
    auto it = c->routers.find(layer);
    if (it == c->routers.end()) return;
    if (it->second.fp8) drop_tensor(c, it->second.fp8);
    c->arena.free(it->second.bf16, it->second.rows * it->second.cols * 2);
    c->arena.free(it->second.bias, it->second.rows * sizeof(float));
    c->routers.erase(it);
}

// Parses a ZCBLK01 expert block and makes its three FP4 projections
// resident under (layer, expert).  The caller holds c->mu.
int store_block_locked(wh_ctx* c, uint32_t layer, uint32_t expert, const uint8_t* block, size_t len, bool pinned,
                       const char* where) {
    whqb::Fp4 p[3];
    whqb::Error err;
    if (!whqb::fp4_expert(block, len, p, &err)) {
        set_block_error(err, where);
        return block_status(err);
    }
    wh_tensor ids[3] = {0, 0, 0};
    for (int m = 0; m < 3; ++m) {
        int st = store_fp4_upload(c, block + p[m].weight_off, p[m].weight_len, block + p[m].scale_off,
                                  p[m].scale_len, p[m].rows, p[m].cols, p[m].scale_cols, pinned, &ids[m]);
        if (st != WH_OK) {
            for (int k = 0; k < m; ++k) drop_tensor(c, ids[k]);
            return st;
        }
    }
    register_owned_expert(c, layer, expert, ids);
    return WH_OK;
}

}  // namespace

// ===================================================================== ABI
extern "C" {

const char* wh_status_string(int s) {
    switch (s) {
        case WH_OK: return "ok";
        case WH_EMPTY_SHAPE: return "EmptyShape";
        case WH_INVALID_SHAPE: return "InvalidShape";
        case WH_PACKED_WEIGHT_TOO_SMALL: return "PackedWeightTooSmall";
        case WH_SCALE_TOO_SMALL: return "ScaleTooSmall";
        case WH_INPUT_TOO_SMALL: return "InputTooSmall";
        case WH_OUTPUT_TOO_SMALL: return "OutputTooSmall";
        case WH_SCRATCH_TOO_SMALL: return "ScratchTooSmall";
        case WH_NON_FINITE_OUTPUT: return "NonFiniteOutput";
        case WH_INVALID_QUANT_FORMAT: return "InvalidQuantFormat";
        case WH_NOT_RESIDENT: return "NotResident";
        case WH_OUT_OF_MEMORY: return "OutOfMemory";
        case WH_HIP_ERROR: return "HipError";
        case WH_INVALID_ARGUMENT: return "InvalidArgument";
        case WH_NON_FINITE_INPUT: return "NonFiniteInput";
        case WH_UNSUPPORTED: return "Unsupported";
        case WH_TRUNCATED_QUANT_BLOCK: return "TruncatedQuantBlock";
        case WH_INVALID_QUANT_BLOCK_MAGIC: return "InvalidQuantBlockMagic";
        case WH_UNSUPPORTED_QUANT_BLOCK_VERSION: return "UnsupportedQuantBlockVersion";
        case WH_INVALID_QUANT_BLOCK: return "InvalidQuantBlock";
        case WH_TENSOR_INDEX_OUT_OF_RANGE: return "TensorIndexOutOfRange";
        case WH_UNALIGNED: return "Unaligned";
        case WH_IO_ERROR: return "Io";
        default: return "unknown";
    }
}

const char* wh_last_error(void) { return g_last_error; }

const char* wh_build_info(void) {
    static char buf[160];
    std::snprintf(buf, sizeof buf, "wohper_hip gfx950; expf exceptions %u; max experts %d; lds %zu",
                  (unsigned)WH_EXPF_EXC_COUNT, WH_MAX_EXPERTS, g_max_lds);
    return buf;
}

int wh_init(int device, wh_ctx** out) {
    if (!out) return WH_INVALID_ARGUMENT;
    *out = nullptr;
    int n = 0;
    WH_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return WH_INVALID_ARGUMENT;
    WH_HIP(hipSetDevice(device));
    WH_HIP(kernel_setup_once(device));
    WH_TRY(noalloc_setup(device));
    wh_ctx* c = new wh_ctx();
    c->device = device;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    c->base_stream = c->stream;
    if (e == hipSuccess) e = hipMalloc(&c->status, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c->status, 0, sizeof(uint32_t));
    if (e == hipSuccess) e = hipHostMalloc((void**)&c->status_host, sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreate(&c->timer[0]);
    if (e == hipSuccess) e = hipEventCreate(&c->timer[1]);
    if (e != hipSuccess) {
        delete c;
        return hip_status(e);
    }
    for (Scratch* sp : c->scratch()) sp->retire = &c->retire;
    *out = c;
    return WH_OK;
}

int wh_shutdown(wh_ctx* c) {
    if (!c) return WH_INVALID_ARGUMENT;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (c->capturing) {
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(c->cap_stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        c->stream = c->base_stream;
    }
    if (c->cap_stream) (void)hipStreamDestroy(c->cap_stream);
    for (auto& kv : c->graphs) (void)hipGraphExecDestroy(kv.second);
    (void)hipStreamSynchronize(c->stream);
    c->arena.release_all();
    for (Scratch* s : c->scratch())
        if (s->p) (void)hipFree(s->p);
    for (void* q : c->retire.retired) (void)hipFree(q);
    for (auto& kv : c->rope_tabs) (void)hipFree(kv.second);
    for (auto& kv : c->tables)
        if (kv.second.dev) (void)hipFree(kv.second.dev);
    for (HostBuf* h : {&c->stage_in, &c->stage_out, &c->pack[0], &c->pack[1]})
        if (h->p) (void)hipHostFree(h->p);
    for (hipEvent_t e : c->timer)
        if (e) (void)hipEventDestroy(e);
    (void)hipFree(c->status);
    (void)hipHostFree(c->status_host);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return WH_OK;
}

int wh_synchronize(wh_ctx* c) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    return read_status(c);
}

int wh_stream_status(wh_ctx* c) { return wh_synchronize(c); }

int wh_graph_begin(wh_ctx* c) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    if (c->capturing) return WH_INVALID_ARGUMENT;
    WH_HIP(hipSetDevice(c->device));
    if (!c->cap_stream) WH_HIP(hipStreamCreateWithFlags(&c->cap_stream, hipStreamNonBlocking));
    // thread-local: calls of this thread that would synchronize fail (and
    // invalidate the capture) instead of running
    WH_HIP(hipStreamBeginCapture(c->cap_stream, hipStreamCaptureModeThreadLocal));
    c->stream = c->cap_stream;
    c->capturing = true;
    return WH_OK;
}

int wh_graph_end(wh_ctx* c, wh_graph* out) {
    if (!c || !out) return WH_INVALID_ARGUMENT;
    *out = 0;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    if (!c->capturing) return WH_INVALID_ARGUMENT;
    (void)hipSetDevice(c->device);
    hipGraph_t g = nullptr;
    const hipError_t ce = hipStreamEndCapture(c->cap_stream, &g);
    c->stream = c->base_stream;
    c->capturing = false;
    if (ce != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        // a broken capture can leave its stream in capture mode: the next
        // capture gets a fresh one
        (void)hipStreamDestroy(c->cap_stream);
        c->cap_stream = nullptr;
        const int st = hip_status(ce);
        (void)hipGetLastError();  // the thread's sticky error is this capture's, reported here
        return st;
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    WH_HIP(e);
    const wh_graph id = c->next_graph++;
    c->graphs[id] = exec;
    ++c->retire.live;
    *out = id;
    return WH_OK;
}

int wh_graph_launch(wh_ctx* c, wh_graph g) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    auto it = c->graphs.find(g);
    if (it == c->graphs.end() || c->capturing) return WH_INVALID_ARGUMENT;
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(hipGraphLaunch(it->second, c->stream));
    return WH_OK;
}

int wh_graph_release(wh_ctx* c, wh_graph g) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    auto it = c->graphs.find(g);
    if (it == c->graphs.end()) return WH_INVALID_ARGUMENT;
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(hipStreamSynchronize(c->stream));  // replays still queued use the buffers
    (void)hipGraphExecDestroy(it->second);
    c->graphs.erase(it);
    if (--c->retire.live == 0) {
        for (void* q : c->retire.retired) (void)hipFree(q);
        c->retire.retired.clear();
    }
    return WH_OK;
}

void* wh_stream(wh_ctx* c) { return c ? (void*)c->stream : nullptr; }

int wh_store_fp8(wh_ctx* c, const uint8_t* weight, size_t weight_len, size_t rows, size_t cols,
                 const void* scales, size_t scales_len, int scale_format, size_t scale_rows,
                 size_t scale_cols, wh_tensor* out) {
    if (!c || !out || !weight || !scales) return WH_INVALID_ARGUMENT;
    if (scale_format != WH_SCALE_UE8M0 && scale_format != WH_SCALE_F32) return WH_INVALID_QUANT_FORMAT;
    // E/compute.rs:6184-6215
    if (rows == 0 || cols == 0 || scale_rows == 0 || scale_cols == 0 || rows % scale_rows ||
        cols % scale_cols)
        return WH_INVALID_SHAPE;
    if (weight_len < rows * cols) return WH_PACKED_WEIGHT_TOO_SMALL;
    size_t sbytes = scale_rows * scale_cols * (scale_format == WH_SCALE_F32 ? 4 : 1);
    if (scales_len < sbytes) return WH_SCALE_TOO_SMALL;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    Tensor t;
    t.kind = kFp8;
    t.rows = rows;
    t.cols = cols;
    t.scale_rows = scale_rows;
    t.scale_cols = scale_cols;
    t.scale_fmt = scale_format;
    t.fast = (cols / scale_cols == 128) && cols * 4 <= g_max_lds;
    for (size_t i = 0; i < rows * cols && !t.special; ++i) t.special = (weight[i] & 0x7f) == 0x7f;
    t.bytes = rows * cols + sbytes;
    WH_TRY(alloc_tensor(c, t, rows * cols, sbytes));
    const size_t chunk_rows = std::max<size_t>(1, (size_t(64) << 20) / cols);
    WH_HIP(c->stage_in.ensure(std::min(rows, chunk_rows) * cols));
    for (size_t r = 0; r < rows; r += chunk_rows) {
        size_t nr = std::min(chunk_rows, rows - r);
        uint8_t* st = (uint8_t*)c->stage_in.p;
        if (t.fast)
            for (size_t i = 0; i < nr; ++i) fp8_permute_row(weight + (r + i) * cols, st + i * cols, cols);
        else
            std::memcpy(st, weight + r * cols, nr * cols);
        WH_TRY(upload(c, t.w + r * cols, st, nr * cols));
    }
    WH_TRY(upload(c, t.s, scales, sbytes));
    return store_tensor_common(c, std::move(t), out);
}

int wh_store_fp4(wh_ctx* c, const uint8_t* packed, size_t packed_len, const uint8_t* scales,
                 size_t scales_len, size_t rows, size_t cols, size_t scale_cols, wh_tensor* out) {
    if (!c || !out || !packed || !scales) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    return store_fp4_upload(c, packed, packed_len, scales, scales_len, rows, cols, scale_cols, false, out);
}

int wh_store_expert(wh_ctx* c, uint32_t layer, uint32_t expert, wh_tensor w1, wh_tensor w3,
                    wh_tensor w2) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    Tensor *t1 = find_tensor(c, w1), *t3 = find_tensor(c, w3), *t2 = find_tensor(c, w2);
    if (!t1 || !t3 || !t2) return WH_NOT_RESIDENT;
    if (t1->kind != kFp4 || t3->kind != kFp4 || t2->kind != kFp4) return WH_INVALID_QUANT_FORMAT;
    // E/compute.rs:1263-1265
    if (t1->cols != t3->cols || t1->rows != t3->rows || t2->cols != t1->rows) return WH_INVALID_SHAPE;
    auto it = c->experts.find({layer, expert});
    if (it != c->experts.end() && it->second.owned)
        for (wh_tensor old : {it->second.w1, it->second.w3, it->second.w2})
            if (old != w1 && old != w3 && old != w2) drop_tensor(c, old);
    c->experts[{layer, expert}] = Expert{w1, w3, w2};
    c->tables[layer].valid = false;
    return WH_OK;
}

void wh_synth_fp4_host(uint64_t seed, uint64_t stream, uint8_t* packed, size_t packed_len,
                       uint8_t* scales, size_t scales_len, uint32_t slo, uint32_t shi) {
    for (size_t i = 0; i < packed_len; ++i) packed[i] = wh_synth_byte(seed, stream, i);
    uint32_t span = shi - slo + 1;
    for (size_t i = 0; i < scales_len; ++i)
        scales[i] = (uint8_t)(slo + wh_synth_byte(seed, stream ^ 0x5ca1e5ull, i) % span);
}

int wh_store_expert_synthetic(wh_ctx* c, uint32_t layer, uint32_t expert, size_t hidden,
                              size_t inter, uint64_t seed, uint32_t slo, uint32_t shi) {
    if (!c || slo > shi || shi > 255) return WH_INVALID_ARGUMENT;
    if (hidden % 256 || inter % 256 || hidden == 0 || inter == 0) return WH_INVALID_SHAPE;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    wh_tensor ids[3];
    const size_t shapes[3][2] = {{inter, hidden}, {inter, hidden}, {hidden, inter}};
    for (int m = 0; m < 3; ++m) {
        Tensor t;
        t.kind = kFp4;
        t.rows = shapes[m][0];
        t.cols = shapes[m][1];
        t.scale_rows = t.rows;
        t.scale_cols = t.cols / 32;
        t.fast = true;
        t.zero_scale = slo == 0;  // bytes uniform in [slo, shi]
        t.bytes = t.rows * t.cols / 2 + t.rows * t.scale_cols;
        const int st = alloc_tensor(c, t, t.rows * t.cols / 2, t.rows * t.scale_cols);
        if (st != WH_OK) {
            for (int k = 0; k < m; ++k) drop_tensor(c, ids[k]);
            return st;
        }
        uint64_t stream = ((uint64_t)layer << 40) ^ ((uint64_t)expert << 8) ^ (uint64_t)m;
        size_t words = t.rows * (t.cols / 256) * 32;
        size_t work = std::max(words, t.rows * t.scale_cols);
        k_synth_fp4<<<(unsigned)((work + 255) / 256), 256, 0, c->stream>>>(
            t.w, (uint8_t*)t.s, (uint32_t)t.rows, (uint32_t)t.cols, seed, stream, slo, shi);
        WH_HIP(hipGetLastError());
        WH_TRY(store_tensor_common(c, std::move(t), &ids[m]));
    }
    WH_HIP(hipStreamSynchronize(c->stream));
    register_owned_expert(c, layer, expert, ids);
    return WH_OK;
}

int wh_quant_block_header(const uint8_t* block, size_t block_len, uint32_t* tensor_count, uint32_t* quant_format,
                          uint32_t* flags) {
    if (!block && block_len) return WH_INVALID_ARGUMENT;
    whqb::Reader r(block, block_len);
    whqb::Header h;
    whqb::Error err;
    if (!whqb::parse_header(r, &h, &err)) {
        set_block_error(err, nullptr);
        return block_status(err);
    }
    if (tensor_count) *tensor_count = h.tensor_count;
    if (quant_format) *quant_format = h.quant_format;
    if (flags) *flags = h.flags;
    return WH_OK;
}

int wh_quant_block_tensor(const uint8_t* block, size_t block_len, size_t index, wh_quant_tensor* out) {
    if ((!block && block_len) || !out) return WH_INVALID_ARGUMENT;
    whqb::Reader r(block, block_len);
    whqb::Header h;
    whqb::Error err;
    whqb::Tensor t;
    if (!whqb::parse_header(r, &h, &err) || (index < h.tensor_count && !whqb::tensor_at(r, h, index, &t, &err))) {
        set_block_error(err, nullptr);
        return block_status(err);
    }
    if (index >= h.tensor_count) {
        // TensorIndexOutOfRange, E/compute.rs:546-550
        std::snprintf(g_last_error, sizeof g_last_error, "tensor index out of range: index=%zu, count=%u", index,
                      h.tensor_count);
        return WH_TENSOR_INDEX_OUT_OF_RANGE;
    }
    *out = wh_quant_tensor{};
    out->dtype_original = t.dtype_original;
    out->quant_format = t.quant_format;
    out->rank = t.rank;
    out->flags = t.flags;
    out->scale = t.scale;
    out->zero_point = t.zero_point;
    out->name_offset = t.name_off;
    out->name_len = t.name_len;
    out->shape_offset = t.shape_off;
    out->data_offset = t.data_off;
    out->data_bytes = t.data_len;
    return WH_OK;
}

int wh_quant_block_fp4_expert(const uint8_t* block, size_t block_len, wh_fp4_view out[3]) {
    if ((!block && block_len) || !out) return WH_INVALID_ARGUMENT;
    whqb::Fp4 p[3];
    whqb::Error err;
    if (!whqb::fp4_expert(block, block_len, p, &err)) {
        set_block_error(err, nullptr);
        return block_status(err);
    }
    for (int m = 0; m < 3; ++m)
        out[m] = wh_fp4_view{p[m].rows,       p[m].cols,      p[m].scale_cols, p[m].weight_off,
                             p[m].weight_len, p[m].scale_off, p[m].scale_len};
    return WH_OK;
}

int wh_store_expert_block(wh_ctx* c, uint32_t layer, uint32_t expert, const uint8_t* block, size_t block_len) {
    if (!c || (!block && block_len)) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    return store_block_locked(c, layer, expert, block, block_len, false, nullptr);
}

int wh_store_expert_pack(wh_ctx* c, const char* pack_path, const wh_expert_pack_entry* entries, size_t n,
                         size_t* stored) {
    if (stored) *stored = 0;
    if (!c || !pack_path || (!entries && n)) return WH_INVALID_ARGUMENT;
    // the index checks of load_optional_expert_pack (E/model_format.rs:488-491)
    constexpr uint64_t kAlign = uint64_t(2) << 20;
    for (size_t i = 0; i < n; ++i) {
        const wh_expert_pack_entry& e = entries[i];
        const char* field = e.offset % kAlign ? "expert_pack.offset" : e.disk_bytes % kAlign ? "expert_pack.disk_bytes" : nullptr;
        if (field) {
            std::snprintf(g_last_error, sizeof g_last_error, "unaligned field %s: value=%llu, required=%llu", field,
                          (unsigned long long)(e.offset % kAlign ? e.offset : e.disk_bytes),
                          (unsigned long long)kAlign);
            return WH_UNALIGNED;
        }
        // the reader hands compute the first payload_bytes of the disk_bytes it read
        if (e.payload_bytes > e.disk_bytes) {
            std::snprintf(g_last_error, sizeof g_last_error,
                          "layer %u expert %u: payload_bytes %llu exceeds disk_bytes %llu", e.layer_id, e.expert_id,
                          (unsigned long long)e.payload_bytes, (unsigned long long)e.disk_bytes);
            return WH_INVALID_ARGUMENT;
        }
    }
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const int fd = open(pack_path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        std::snprintf(g_last_error, sizeof g_last_error, "experts pack file %s: %s", pack_path, std::strerror(errno));
        return WH_IO_ERROR;
    }
    struct Guard {
        int fd;
        hipStream_t stream;
        hipEvent_t ev[2] = {nullptr, nullptr};
        ~Guard() {
            (void)hipStreamSynchronize(stream);  // no copy from the read buffers outlives the call
            for (hipEvent_t e : ev)
                if (e) (void)hipEventDestroy(e);
            close(fd);
        }
    } g{fd, c->stream};
    for (hipEvent_t& e : g.ev) WH_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (size_t i = 0; i < n; ++i) {
        const wh_expert_pack_entry& e = entries[i];
        HostBuf& buf = c->pack[i & 1];
        // the uploads queued from this buffer two experts ago must have left it
        if (i >= 2) WH_HIP(hipEventSynchronize(g.ev[i & 1]));
        WH_HIP(buf.ensure(std::max<size_t>((size_t)e.payload_bytes, 1)));
        uint8_t* p = (uint8_t*)buf.p;
        for (size_t got = 0; got < e.payload_bytes;) {
            const ssize_t k = pread(fd, p + got, (size_t)e.payload_bytes - got, (off_t)(e.offset + got));
            if (k < 0 && errno == EINTR) continue;
            if (k <= 0) {
                std::snprintf(g_last_error, sizeof g_last_error, "experts pack read (layer %u expert %u at %llu): %s",
                              e.layer_id, e.expert_id, (unsigned long long)e.offset,
                              k < 0 ? std::strerror(errno) : "unexpected end of file");
                return WH_IO_ERROR;
            }
            got += (size_t)k;
        }
        char where[64];
        std::snprintf(where, sizeof where, "layer %u expert %u", e.layer_id, e.expert_id);
        WH_TRY(store_block_locked(c, e.layer_id, e.expert_id, p, (size_t)e.payload_bytes, true, where));
        WH_HIP(hipEventRecord(g.ev[i & 1], c->stream));
        if (stored) ++*stored;
    }
    WH_HIP(hipStreamSynchronize(c->stream));
    return WH_OK;
}

int wh_store_router(wh_ctx* c, uint32_t layer, const uint8_t* block, size_t block_len, size_t hidden_len,
                    int* found) {
    if (found) *found = 0;
    if (!c || (!block && block_len)) return WH_INVALID_ARGUMENT;
    whqb::Reader r(block, block_len);
    whqb::Header h;
    whqb::Error e;
    auto fail = [&]() {
        set_block_error(e, nullptr);
        return block_status(e);
    };
    if (!whqb::parse_header(r, &h, &e)) return fail();
    // router_gate_tensor (E/compute.rs:2444-2467): the Router-role matrix
    // whose cols match the hidden size, else the first one; never tid2eid
    whqb::Tensor gate;
    bool have_gate = false, exact = false;
    for (size_t i = 0; i < h.tensor_count && !exact; ++i) {
        whqb::Tensor t;
        if (!whqb::tensor_at(r, h, i, &t, &e)) return fail();
        if ((t.flags & 0xffff) != kRoleRouter || t.rank != 2 || name_contains_ci(r, t, "tid2eid")) continue;
        if ((size_t)t.dim(r, 1) == hidden_len) {
            gate = t;
            have_gate = exact = true;
        } else if (!have_gate) {
            gate = t;
            have_gate = true;
        }
    }
    if (!have_gate) {  // Ok(None): the engine falls back to its own routing
        std::lock_guard<std::recursive_mutex> lk(c->mu);
        drop_router(c, layer);
        return WH_OK;
    }
    Router rt;
    rt.rows = (size_t)gate.dim(r, 0);
    rt.cols = (size_t)gate.dim(r, 1);
    if (rt.rows == 0 || rt.rows > WH_ROUTER_MAX_ROWS) {
        std::snprintf(g_last_error, sizeof g_last_error, "router of %zu experts (1..%u supported)", rt.rows,
                      WH_ROUTER_MAX_ROWS);
        return WH_UNSUPPORTED;
    }
    const bool fp8 = gate.quant_format == 2401;
    const bool bf16 = gate.quant_format == 2404 && gate.dtype_original == 11;
    if (!fp8 && !bf16) {
        std::snprintf(g_last_error, sizeof g_last_error, "router gate quant format %u (dtype %u) is not on the GPU path",
                      gate.quant_format, gate.dtype_original);
        return WH_UNSUPPORTED;
    }
    if (bf16 && gate.data_len / 2 / rt.cols < rt.rows) return shape_error("BF16 GEMV tensor data too small");
    wh_tensor fp8_handle = 0;
    if (fp8) {
        // fp8_scale_for_weight (E/compute.rs:1184-1199), then the checks of
        // gemv_fp8_e4m3_ue8m0_tensorwise (E/compute.rs:6174-6215)
        static const char kW[] = ".weight";
        if (gate.name_len < 7 || std::memcmp(r.data() + gate.name_off + gate.name_len - 7, kW, 7) != 0) {
            whqb::Reader::fail(&e, whqb::Fail::Invalid, "DeepSeek FP8 weight name does not end with .weight");
            return fail();
        }
        const size_t stem = gate.name_len - 7;
        whqb::Tensor sc;
        bool have_scale = false;
        for (size_t i = 0; i < h.tensor_count && !have_scale; ++i) {
            whqb::Tensor t;
            if (!whqb::tensor_at(r, h, i, &t, &e)) return fail();
            have_scale = t.name_len == stem + 6 &&
                         std::memcmp(r.data() + t.name_off, r.data() + gate.name_off, stem) == 0 &&
                         std::memcmp(r.data() + t.name_off + stem, ".scale", 6) == 0;
            if (have_scale) sc = t;
        }
        if (!have_scale) {
            whqb::Reader::fail(&e, whqb::Fail::Invalid, "missing DeepSeek FP8 scale tensor");
            return fail();
        }
        if (sc.quant_format != whqb::kQuantUe8m0) {
            whqb::Reader::fail(&e, whqb::Fail::Invalid, "DeepSeek FP8 scale is not UE8M0");
            return fail();
        }
        if (sc.rank != 2) return shape_error("DeepSeek FP8 scale rank");
        const size_t srows = (size_t)sc.dim(r, 0), scols = (size_t)sc.dim(r, 1);
        if (srows == 0 || scols == 0 || rt.rows % srows || rt.cols % scols) return shape_error("DeepSeek FP8 scale shape");
        if (gate.data_len / rt.cols < rt.rows) return shape_error("DeepSeek FP8 weight data too small");
        if (sc.data_len < srows * scols) return shape_error("DeepSeek FP8 scale data too small");
        WH_TRY(wh_store_fp8(c, r.data() + gate.data_off, gate.data_len, rt.rows, rt.cols, r.data() + sc.data_off,
                            sc.data_len, WH_SCALE_UE8M0, srows, scols, &fp8_handle));
    }
    // the bias and tid2eid lookups run per route call in the reference;
    // their outcome is the same every time, so it is kept
    std::vector<float> bias;
    bool have_bias = false;
    router_bias(r, h, rt.rows, &bias, &have_bias, &rt.bias_err);
    for (size_t i = 0; i < h.tensor_count; ++i) {  // router_tid2eid_tensor, E/compute.rs:2270-2285
        whqb::Tensor t;
        if (!whqb::tensor_at(r, h, i, &t, &e)) {
            rt.has_table = true;
            set_block_error(e, nullptr);
            rt.table_err.status = block_status(e);
            rt.table_err.text = g_last_error;
            break;
        }
        if ((t.flags & 0xffff) != kRoleRouter || t.rank != 2 || !name_contains_ci(r, t, "tid2eid")) continue;
        rt.has_table = true;
        rt.table_dtype = t.dtype_original;
        rt.table_rows = (size_t)t.dim(r, 0);
        rt.table_cols = (size_t)t.dim(r, 1);
        rt.table.assign(r.data() + t.data_off, r.data() + t.data_off + t.data_len);
        break;
    }
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    if (fp8) {
        rt.gate = kGateFp8;
        rt.fp8 = fp8_handle;
    } else {
        const size_t n = rt.rows * rt.cols;
        void* d = nullptr;
        WH_TRY(alloc_device(c, n * 2, &d));
        rt.bf16 = (uint16_t*)d;
        std::vector<uint16_t> tmp(n);  // the block's bytes need not be 2-byte aligned
        std::memcpy(tmp.data(), r.data() + gate.data_off, n * 2);
        if (rt.cols % 128 == 0 && rt.cols * sizeof(float) <= g_max_lds) {
            std::vector<uint16_t> lane(n);
            bf16_router_layout(tmp.data(), lane.data(), rt.rows, rt.cols);
            tmp.swap(lane);
            rt.gate = kGateBf16;
        } else {
            rt.gate = kGateBf16Rows;
        }
        WH_TRY(h2d(c, rt.bf16, reinterpret_cast<const uint8_t*>(tmp.data()), n * 2, false));
    }
    if (have_bias) {
        void* d = nullptr;
        WH_TRY(alloc_device(c, rt.rows * sizeof(float), &d));
        rt.bias = (float*)d;
        WH_TRY(h2d(c, rt.bias, reinterpret_cast<const uint8_t*>(bias.data()), rt.rows * sizeof(float), false));
    }
    auto old = c->routers.find(layer);
    drop_router(c, layer);
    c->routers[layer] = std::move(rt);
    if (found) *found = 1;
    return WH_OK;
}

int wh_route_experts(wh_ctx* c, uint32_t layer, const float* hidden, size_t hidden_len, size_t active,
                     const uint32_t* available, size_t n_available, const wh_route_options* opts, uint32_t* expert_ids,
                     float* scores, size_t out_cap, size_t* n_out) {
    if (n_out) *n_out = 0;
    if (!c || !opts || !n_out || (!hidden && hidden_len)) return WH_INVALID_ARGUMENT;
    if (active == 0 || (available && n_available == 0)) return WH_OK;  // E/compute.rs:2138-2140
    if (!expert_ids || !scores) return WH_INVALID_ARGUMENT;
    if (out_cap < active) return WH_OUTPUT_TOO_SMALL;
    if (active > WH_ROUTER_MAX_ACTIVE || n_available > WH_ROUTER_MAX_ROWS) return WH_UNSUPPORTED;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    auto it = c->routers.find(layer);
    if (it == c->routers.end()) return WH_NOT_RESIDENT;
    const Router& rt = it->second;
    wh_router_sel sa;
    WH_TRY(router_prepare(rt, *opts, hidden_len, active, available ? n_available : rt.rows, &sa));
    // scratch: x [cols], logits [rows], available ids, then the outputs
    const size_t nav = available ? n_available : 0;
    const size_t words = rt.cols + 3 * rt.rows + nav + 2 * WH_ROUTER_MAX_ACTIVE + 1;
    WH_HIP(c->rtr.ensure(words * 4, false));
    float* x = c->rtr.as<float>();
    float* logits = x + rt.cols;  // [3 * rows]: scores and selection keys, or (score, key) pairs and ids
    uint32_t* av = reinterpret_cast<uint32_t*>(logits + 3 * rt.rows);
    uint32_t* ids = av + nav;
    float* sc = reinterpret_cast<float*>(ids + WH_ROUTER_MAX_ACTIVE);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(sc + WH_ROUTER_MAX_ACTIVE);
    WH_TRY(h2d(c, x, reinterpret_cast<const uint8_t*>(hidden), rt.cols * sizeof(float), false));
    if (nav) WH_TRY(h2d(c, av, reinterpret_cast<const uint8_t*>(available), nav * 4, false));
    WH_TRY(router_launch(c, rt, sa, x, nav ? av : nullptr, logits, ids, sc, cnt));
    const size_t back = (2 * WH_ROUTER_MAX_ACTIVE + 1) * 4;
    WH_HIP(c->stage_out.ensure(back));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, ids, back, hipMemcpyDeviceToHost, c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    const uint32_t* hb = (const uint32_t*)c->stage_out.p;
    const uint32_t n = hb[2 * WH_ROUTER_MAX_ACTIVE];
    std::memcpy(expert_ids, hb, n * 4);
    std::memcpy(scores, hb + WH_ROUTER_MAX_ACTIVE, n * 4);
    *n_out = n;
    return read_status(c);
}

// wh_route_experts_async; with rs, the router's last workgroup also
// resolves the selected routes into rs->dyn where the one-launch sorted
// selection applies (*resolved then true).  The caller holds c->mu.
int route_experts(wh_ctx* c, uint32_t layer, const float* x_dev, size_t hidden_len, size_t active,
                  const uint32_t* available_dev, size_t n_available, const wh_route_options* opts,
                  uint32_t* ids_dev, float* scores_dev, uint32_t* count_dev, const MoeDevPrep* rs, bool* resolved) {
    if (resolved) *resolved = false;
    if (!c || !opts || !x_dev || !ids_dev || !scores_dev || !count_dev) return WH_INVALID_ARGUMENT;
    if ((uintptr_t)x_dev & 15) return WH_INVALID_ARGUMENT;  // x is read in 16-byte pieces
    if (active > WH_ROUTER_MAX_ACTIVE || n_available > WH_ROUTER_MAX_ROWS) return WH_UNSUPPORTED;
    WH_HIP(hipSetDevice(c->device));
    auto it = c->routers.find(layer);
    if (it == c->routers.end()) return WH_NOT_RESIDENT;
    const Router& rt = it->second;
    wh_router_sel sa;
    if (active == 0 || (available_dev && n_available == 0)) {
        // no routes: the selection kernel only writes the zero count
        std::memset(&sa, 0, sizeof sa);
        sa.out_ids = ids_dev;
        sa.out_scores = scores_dev;
        sa.out_count = count_dev;
        k_router_select<<<1, 256, 0, c->stream>>>(sa);
        WH_HIP(hipGetLastError());
        return WH_OK;
    }
    WH_TRY(router_prepare(rt, *opts, hidden_len, active, available_dev ? n_available : rt.rows, &sa));
    WH_HIP(c->rtr.ensure((rt.cols + 3 * rt.rows + 2 * WH_ROUTER_MAX_ACTIVE + 1) * 4, false));
    float* logits = c->rtr.as<float>() + rt.cols;
    return router_launch(c, rt, sa, x_dev, available_dev, logits, ids_dev, scores_dev, count_dev, rs, resolved);
}

int wh_route_experts_async(wh_ctx* c, uint32_t layer, const float* x_dev, size_t hidden_len, size_t active,
                           const uint32_t* available_dev, size_t n_available, const wh_route_options* opts,
                           uint32_t* ids_dev, float* scores_dev, uint32_t* count_dev) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    return route_experts(c, layer, x_dev, hidden_len, active, available_dev, n_available, opts, ids_dev, scores_dev,
                         count_dev, nullptr, nullptr);
}

void wh_synth_fp8_host(uint64_t seed, uint64_t stream, uint8_t* weight, size_t n) {
    for (size_t i = 0; i < n; ++i) weight[i] = wh_fp8_synth_code(seed, stream, i);
}

int wh_store_fp8_synthetic(wh_ctx* c, size_t rows, size_t cols, uint64_t seed, uint64_t stream,
                           const float* scales, size_t scale_rows, size_t scale_cols, wh_tensor* out) {
    if (!c || !out || !scales) return WH_INVALID_ARGUMENT;
    if (rows == 0 || cols == 0 || scale_rows == 0 || scale_cols == 0 || rows % scale_rows || cols % scale_cols ||
        cols / scale_cols != 128)
        return WH_INVALID_SHAPE;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    Tensor t;
    t.kind = kFp8;
    t.rows = rows;
    t.cols = cols;
    t.scale_rows = scale_rows;
    t.scale_cols = scale_cols;
    t.scale_fmt = WH_SCALE_F32;
    t.fast = cols * 4 <= g_max_lds;
    if (!t.fast) return WH_UNSUPPORTED;
    const size_t sbytes = scale_rows * scale_cols * sizeof(float);
    t.bytes = rows * cols + sbytes;
    WH_TRY(alloc_tensor(c, t, rows * cols, sbytes));
    const size_t n = rows * cols;
    k_synth_fp8<<<(unsigned)((n + 255) / 256), 256, 0, c->stream>>>(t.w, (uint32_t)rows, (uint32_t)cols, seed, stream);
    WH_HIP(hipGetLastError());
    WH_TRY(upload(c, t.s, scales, sbytes));
    return store_tensor_common(c, std::move(t), out);
}

int wh_store_release(wh_ctx* c, wh_tensor t) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    auto it = c->tensors.find(t);
    if (it == c->tensors.end()) return WH_NOT_RESIDENT;
    drop_tensor(c, t);
    for (auto& kv : c->tables) kv.second.valid = false;
    return WH_OK;
}

int wh_store_usage(wh_ctx* c, size_t* bytes, size_t* tensors, size_t* experts) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    if (bytes) *bytes = c->arena.live;
    if (tensors) *tensors = c->tensors.size();
    if (experts) *experts = c->experts.size();
    return WH_OK;
}

int wh_tensor_dequant(wh_ctx* c, wh_tensor th, float* out, size_t out_len) {
    if (!c || !out) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    Tensor* t = find_tensor(c, th);
    if (!t) return WH_NOT_RESIDENT;
    if (!t->fast) return WH_UNSUPPORTED;
    size_t n = t->rows * t->cols;
    if (out_len < n) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(c->y_out.ensure(n * sizeof(float), false));
    float* d = c->y_out.as<float>();
    if (t->kind == kFp4) {
        size_t th_n = t->rows * (t->cols / 256) * 8;
        k_fp4_dequant<<<(unsigned)((th_n + 255) / 256), 256, 0, c->stream>>>(
            t->w, (const uint8_t*)t->s, (uint32_t)t->rows, (uint32_t)t->cols, d);
    } else {
        size_t th_n = t->rows * (t->cols / 128) * 8;
        if (t->special)
            k_fp8_dequant<true><<<(unsigned)((th_n + 255) / 256), 256, 0, c->stream>>>(t->w, (uint32_t)t->rows, (uint32_t)t->cols, d);
        else
            k_fp8_dequant<false><<<(unsigned)((th_n + 255) / 256), 256, 0, c->stream>>>(t->w, (uint32_t)t->rows, (uint32_t)t->cols, d);
    }
    WH_HIP(hipGetLastError());
    WH_HIP(hipMemcpyAsync(out, d, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    return WH_OK;
}

int wh_fp8_gemv_multi(wh_ctx* c, wh_tensor w, size_t row_start, size_t row_end,
                      const float* inputs, size_t n, size_t input_stride, float* outputs,
                      size_t output_stride, size_t* values_out) {
    if (!c || !inputs || !outputs) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    Tensor* t = find_tensor(c, w);
    if (!t) return WH_NOT_RESIDENT;
    if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    if (n == 0) return WH_INVALID_SHAPE;
    // E/compute.rs:6400-6430
    if (row_start >= row_end || row_end > t->rows) return WH_INVALID_SHAPE;
    if (input_stride < t->cols) return WH_INPUT_TOO_SMALL;
    const size_t rows = row_end - row_start;
    if (output_stride < rows) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(c->x_in.ensure(n * t->cols * sizeof(float), false));
    WH_HIP(c->y_out.ensure(n * rows * sizeof(float), false));
    WH_HIP(c->stage_in.ensure(n * t->cols * sizeof(float)));
    WH_HIP(c->stage_out.ensure(n * rows * sizeof(float)));
    float* si = (float*)c->stage_in.p;
    for (size_t b = 0; b < n; ++b) std::memcpy(si + b * t->cols, inputs + b * input_stride, t->cols * sizeof(float));
    WH_HIP(hipMemcpyAsync(c->x_in.p, si, n * t->cols * sizeof(float), hipMemcpyHostToDevice, c->stream));
    if (!c->exact && n >= c->fp8_mm_min && fp8_mm_ok(*t, row_start, row_end, 0))
        WH_TRY(launch_fp8_mm(c, *t, row_start, row_end, c->x_in.as<float>(), n, t->cols, c->y_out.as<float>(), rows, 0, 0));
    else
        WH_TRY(launch_fp8(c, *t, row_start, row_end, c->x_in.as<float>(), c->y_out.as<float>(), n, t->cols, rows));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->y_out.p, n * rows * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    int st = read_status(c);
    if (st != WH_OK) return st;
    float* so = (float*)c->stage_out.p;
    for (size_t b = 0; b < n; ++b) std::memcpy(outputs + b * output_stride, so + b * rows, rows * sizeof(float));
    if (values_out) *values_out = rows * t->cols;
    return WH_OK;
}

int wh_fp8_gemv(wh_ctx* c, wh_tensor w, size_t row_start, size_t row_end, const float* input,
                size_t input_len, float* output, size_t output_len, size_t* values_out) {
    if (!c || !input || !output) return WH_INVALID_ARGUMENT;
    {
        std::lock_guard<std::recursive_mutex> lk(c->mu);
        Tensor* t = find_tensor(c, w);
        if (!t) return WH_NOT_RESIDENT;
        if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
        if (row_start >= row_end || row_end > t->rows) return WH_INVALID_SHAPE;
        if (input_len < t->cols) return WH_INPUT_TOO_SMALL;
        if (output_len < row_end - row_start) return WH_OUTPUT_TOO_SMALL;
    }
    return wh_fp8_gemv_multi(c, w, row_start, row_end, input, 1, input_len, output, output_len,
                             values_out);
}

// Pointer rules of the device-pointer FP8 entry points: the lane-layout
// kernels stage x with 16-byte loads, so x must be 16-byte aligned for them
// (any float alignment for the generic row-major kernel); y takes floats.
static int fp8_ptr_check(const Tensor& t, const float* x, const float* y) {
    if (t.fast && ((uintptr_t)x & 15)) return WH_INVALID_ARGUMENT;
    if (((uintptr_t)x & 3) || ((uintptr_t)y & 3)) return WH_INVALID_ARGUMENT;
    return WH_OK;
}

int wh_fp8_gemv_async(wh_ctx* c, wh_tensor w, size_t row_start, size_t row_end,
                      const float* x_dev, float* y_dev) {
    if (!c || !x_dev || !y_dev) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    Tensor* t = find_tensor(c, w);
    if (!t) return WH_NOT_RESIDENT;
    if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    if (row_start >= row_end || row_end > t->rows) return WH_INVALID_SHAPE;
    WH_TRY(fp8_ptr_check(*t, x_dev, y_dev));
    WH_HIP(hipSetDevice(c->device));
    return launch_fp8(c, *t, row_start, row_end, x_dev, y_dev, 1, t->cols, row_end - row_start);
}

int wh_fp8_gemv_multi_async(wh_ctx* c, wh_tensor w, size_t row_start, size_t row_end, const float* x_dev, size_t n,
                            size_t x_stride, float* y_dev, size_t y_stride) {
    if (!c || !x_dev || !y_dev) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    Tensor* t = find_tensor(c, w);
    if (!t) return WH_NOT_RESIDENT;
    if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    if (n == 0 || row_start >= row_end || row_end > t->rows) return WH_INVALID_SHAPE;  // E/compute.rs:6400-6430
    if (x_stride < t->cols) return WH_INPUT_TOO_SMALL;
    if (y_stride < row_end - row_start) return WH_OUTPUT_TOO_SMALL;
    // the kernels take 32-bit strides and the inputs on grid.y
    if (x_stride > UINT32_MAX || y_stride > UINT32_MAX || n > 65535) return WH_UNSUPPORTED;
    WH_TRY(fp8_ptr_check(*t, x_dev, y_dev));
    if (t->fast && (x_stride & 3)) return WH_INVALID_ARGUMENT;  // every input 16-byte aligned
    WH_HIP(hipSetDevice(c->device));
    if (!c->exact && n >= c->fp8_mm_min && fp8_mm_ok(*t, row_start, row_end, 0))
        return launch_fp8_mm(c, *t, row_start, row_end, x_dev, n, x_stride, y_dev, y_stride, 0, 0);
    return launch_fp8(c, *t, row_start, row_end, x_dev, y_dev, n, x_stride, y_stride);
}

// Checks of wh_fp8_gemv_multi_async's arguments.
static int fp8_multi_check(const Tensor* t, size_t row_start, size_t row_end, const float* x_dev, size_t n,
                           size_t x_stride, float* y_dev, size_t y_stride) {
    if (!t) return WH_NOT_RESIDENT;
    if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    if (n == 0 || row_start >= row_end || row_end > t->rows) return WH_INVALID_SHAPE;  // E/compute.rs:6400-6430
    if (x_stride < t->cols) return WH_INPUT_TOO_SMALL;
    if (y_stride < row_end - row_start) return WH_OUTPUT_TOO_SMALL;
    if (x_stride > UINT32_MAX || y_stride > UINT32_MAX || n > 65535) return WH_UNSUPPORTED;
    WH_TRY(fp8_ptr_check(*t, x_dev, y_dev));
    if (t->fast && (x_stride & 3)) return WH_INVALID_ARGUMENT;
    return WH_OK;
}

int wh_fp8_gemv_multi_pair_async(wh_ctx* c, wh_tensor w0, size_t row_start0, size_t row_end0, float* y0_dev,
                                 size_t y0_stride, wh_tensor w1, size_t row_start1, size_t row_end1, float* y1_dev,
                                 size_t y1_stride, const float* x_dev, size_t n, size_t x_stride) {
    if (!c || !x_dev || !y0_dev || !y1_dev) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    Tensor* t0 = find_tensor(c, w0);
    Tensor* t1 = find_tensor(c, w1);
    WH_TRY(fp8_multi_check(t0, row_start0, row_end0, x_dev, n, x_stride, y0_dev, y0_stride));
    WH_TRY(fp8_multi_check(t1, row_start1, row_end1, x_dev, n, x_stride, y1_dev, y1_stride));
    WH_HIP(hipSetDevice(c->device));
    const bool mm0 = !c->exact && n >= c->fp8_mm_min && fp8_mm_ok(*t0, row_start0, row_end0, 0);
    const bool mm1 = !c->exact && n >= c->fp8_mm_min && fp8_mm_ok(*t1, row_start1, row_end1, 0);
    // one launch when both take the MFMA path with the same k split, the
    // tensors agree in width, scale format, rows per scale row and special
    // codes, and neither output overlaps the inputs or the other output
    // (the two calls are ordered; where the order could show, they stay two)
    if (mm0 && mm1 && t0->cols == t1->cols && t0->scale_fmt == t1->scale_fmt && t0->special == t1->special &&
        t0->rows / t0->scale_rows == t1->rows / t1->scale_rows && t0->scale_cols == t1->scale_cols &&
        fp8_mm_groups(*t0, row_end0 - row_start0, n) == fp8_mm_groups(*t1, row_end1 - row_start1, n)) {
        const uintptr_t x_lo = (uintptr_t)x_dev, x_hi = (uintptr_t)(x_dev + (n - 1) * x_stride + t0->cols);
        const uintptr_t a_lo = (uintptr_t)y0_dev, a_hi = (uintptr_t)(y0_dev + (n - 1) * y0_stride + (row_end0 - row_start0));
        const uintptr_t b_lo = (uintptr_t)y1_dev, b_hi = (uintptr_t)(y1_dev + (n - 1) * y1_stride + (row_end1 - row_start1));
        if (!(a_lo < x_hi && x_lo < a_hi) && !(b_lo < x_hi && x_lo < b_hi) && !(a_lo < b_hi && b_lo < a_hi)) {
            const Fp8MmSecond sec{t1, row_start1, row_end1, y1_dev, y1_stride};
            return launch_fp8_mm(c, *t0, row_start0, row_end0, x_dev, n, x_stride, y0_dev, y0_stride, 0, 0, &sec);
        }
    }
    if (mm0) WH_TRY(launch_fp8_mm(c, *t0, row_start0, row_end0, x_dev, n, x_stride, y0_dev, y0_stride, 0, 0));
    else WH_TRY(launch_fp8(c, *t0, row_start0, row_end0, x_dev, y0_dev, n, x_stride, y0_stride));
    if (mm1) return launch_fp8_mm(c, *t1, row_start1, row_end1, x_dev, n, x_stride, y1_dev, y1_stride, 0, 0);
    return launch_fp8(c, *t1, row_start1, row_end1, x_dev, y1_dev, n, x_stride, y1_stride);
}

int wh_fp8_gemv_multi_groups_async(wh_ctx* c, wh_tensor w, size_t row_start, size_t row_end, size_t group_rows,
                                   const float* x_dev, size_t x_group_stride, size_t n, size_t x_stride, float* y_dev,
                                   size_t y_stride) {
    if (!c || !x_dev || !y_dev || group_rows == 0) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    Tensor* t = find_tensor(c, w);
    if (!t) return WH_NOT_RESIDENT;
    if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    if (n == 0 || row_start >= row_end || row_end > t->rows || (row_end - row_start) % group_rows)
        return WH_INVALID_SHAPE;
    if (x_stride < t->cols) return WH_INPUT_TOO_SMALL;
    if (y_stride < row_end - row_start) return WH_OUTPUT_TOO_SMALL;
    if (x_stride > UINT32_MAX || y_stride > UINT32_MAX || x_group_stride > UINT32_MAX || n > 65535)
        return WH_UNSUPPORTED;
    WH_TRY(fp8_ptr_check(*t, x_dev, y_dev));
    if (t->fast && ((x_stride | x_group_stride) & 3)) return WH_INVALID_ARGUMENT;  // every input 16-byte aligned
    WH_HIP(hipSetDevice(c->device));
    if (!c->exact && n >= c->fp8_mm_min && fp8_mm_ok(*t, row_start, row_end, group_rows))
        return launch_fp8_mm(c, *t, row_start, row_end, x_dev, n, x_stride, y_dev, y_stride, group_rows,
                             x_group_stride);
    // one launch over every group where the kernels take row groups
    if (fp8_split_k(*t) && is_pow2(group_rows) && group_rows >= WH_FP8_SK_ROWS)
        return launch_fp8(c, *t, row_start, row_end, x_dev, y_dev, n, x_stride, y_stride, group_rows, x_group_stride);
    for (size_t r = row_start, g = 0; r < row_end; r += group_rows, ++g)
        WH_TRY(launch_fp8(c, *t, r, r + group_rows, x_dev + g * x_group_stride, y_dev + (r - row_start), n, x_stride,
                          y_stride));
    return WH_OK;
}

int wh_set_fp8_mfma_min(wh_ctx* c, uint32_t min_inputs) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    c->fp8_mm_min = min_inputs ? min_inputs : UINT32_MAX;
    return WH_OK;
}

// Two projections of one input (wq_a and wkv of a decode layer) as one
// launch: both split-K tensors of the same width, special-code set and
// scale format, single row runs, one input, neither output overlapping that
// input or the other output (the descriptors are ordered: where the order
// could show, the pair stays two launches).
bool fp8_pair_ok(const Tensor& t1, const wh_gemv_desc& d1, const Tensor& t2, const wh_gemv_desc& d2) {
    if (d1.x_dev != d2.x_dev || !fp8_split_k(t1) || !fp8_split_k(t2) || t1.cols != t2.cols ||
        t1.special != t2.special || t1.scale_fmt != t2.scale_fmt)
        return false;
    const uintptr_t x_lo = (uintptr_t)d1.x_dev, x_hi = (uintptr_t)(d1.x_dev + t1.cols);
    const uintptr_t a_lo = (uintptr_t)d1.y_dev, a_hi = (uintptr_t)(d1.y_dev + (d1.row_end - d1.row_start));
    const uintptr_t b_lo = (uintptr_t)d2.y_dev, b_hi = (uintptr_t)(d2.y_dev + (d2.row_end - d2.row_start));
    if (a_lo < x_hi && x_lo < a_hi) return false;
    if (b_lo < x_hi && x_lo < b_hi) return false;
    return !(a_lo < b_hi && b_lo < a_hi);  // the second's output must not land on the first's
}

int wh_fp8_gemv_batch_async(wh_ctx* c, const wh_gemv_desc* descs, size_t n) {
    if (!c || (n && !descs)) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    // validate everything before launching anything
    for (size_t i = 0; i < n; ++i) {
        const wh_gemv_desc& d = descs[i];
        Tensor* t = find_tensor(c, d.weight);
        if (!t) return WH_NOT_RESIDENT;
        if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
        if (!d.x_dev || !d.y_dev) return WH_INVALID_ARGUMENT;
        if (d.row_start >= d.row_end || d.row_end > t->rows) return WH_INVALID_SHAPE;
        WH_TRY(fp8_ptr_check(*t, d.x_dev, d.y_dev));
    }
    for (size_t i = 0; i < n;) {
        const wh_gemv_desc& d = descs[i];
        const Tensor* t = find_tensor(c, d.weight);
        const size_t rows = d.row_end - d.row_start;
        // A run of equal, consecutive row groups of one tensor with evenly
        // spaced inputs and back-to-back outputs goes out as one launch.  The
        // kernel takes the input step as a 32-bit count of floats, and the
        // run's outputs must not overlap its inputs: the descriptors are
        // ordered, so an output that feeds a later input keeps its own launch.
        size_t j = i + 1;
        ptrdiff_t xs = 0;
        if (j < n && fp8_split_k(*t) && is_pow2(rows) && rows >= WH_FP8_SK_ROWS) {
            xs = descs[j].x_dev - d.x_dev;
            if (xs >= 0 && (uint64_t)xs <= UINT32_MAX) {
                while (j < n && descs[j].weight == d.weight && descs[j].row_start == descs[j - 1].row_end &&
                       descs[j].row_end - descs[j].row_start == rows && descs[j].x_dev - descs[j - 1].x_dev == xs &&
                       descs[j].y_dev == descs[j - 1].y_dev + rows)
                    ++j;
                const uintptr_t x_lo = (uintptr_t)d.x_dev, x_hi = (uintptr_t)(descs[j - 1].x_dev + t->cols);
                const uintptr_t y_lo = (uintptr_t)d.y_dev, y_hi = (uintptr_t)(descs[j - 1].y_dev + rows);
                if (j - i > 1 && y_lo < x_hi && x_lo < y_hi) j = i + 1;
            }
        }
        if (j - i > 1) {
            WH_TRY(launch_fp8(c, *t, d.row_start, descs[j - 1].row_end, d.x_dev, d.y_dev, 1, t->cols,
                              descs[j - 1].row_end - d.row_start, rows, (size_t)xs));
        } else if (i + 1 < n && descs[i + 1].weight != d.weight &&
                   fp8_pair_ok(*t, d, *find_tensor(c, descs[i + 1].weight), descs[i + 1])) {
            const wh_gemv_desc& e = descs[i + 1];
            WH_TRY(launch_fp8(c, *t, d.row_start, d.row_end, d.x_dev, d.y_dev, 1, t->cols, rows, 0, 0,
                              find_tensor(c, e.weight), e.row_start, e.row_end, e.y_dev));
            j = i + 2;
        } else {
            WH_TRY(launch_fp8(c, *t, d.row_start, d.row_end, d.x_dev, d.y_dev, 1, t->cols, rows));
        }
        i = j;
    }
    return WH_OK;
}

int wh_fp4_matvec(wh_ctx* c, wh_tensor w, const float* input, size_t input_len, float* output,
                  size_t output_len) {
    if (!c || !input || !output) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    Tensor* t = find_tensor(c, w);
    if (!t) return WH_NOT_RESIDENT;
    if (t->kind != kFp4) return WH_INVALID_QUANT_FORMAT;
    if (input_len < t->cols) return WH_INPUT_TOO_SMALL;
    if (output_len < t->rows) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(c->x_in.ensure(t->cols * sizeof(float), false));
    WH_HIP(c->y_out.ensure(t->rows * sizeof(float), false));
    WH_HIP(c->stage_out.ensure(t->rows * sizeof(float)));
    WH_HIP(hipMemcpyAsync(c->x_in.p, input, t->cols * sizeof(float), hipMemcpyHostToDevice, c->stream));
    WH_TRY(launch_fp4(c, *t, c->x_in.as<float>(), c->y_out.as<float>()));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->y_out.p, t->rows * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    int st = read_status(c);
    if (st != WH_OK) return st;
    std::memcpy(output, c->stage_out.p, t->rows * sizeof(float));
    return WH_OK;
}

int wh_act_quant_dequant(wh_ctx* c, float* values, size_t n, size_t block) {
    if (!c) return WH_INVALID_ARGUMENT;
    if (block == 0 || n == 0) return WH_OK;  // E/compute.rs:2505-2507
    if (!values) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(c->x_in.ensure(n * sizeof(float), false));
    WH_HIP(hipMemcpyAsync(c->x_in.p, values, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    k_act_quant_inplace<<<(unsigned)((n + block - 1) / block), 256, 0, c->stream>>>(
        c->x_in.as<float>(), (uint32_t)n, (uint32_t)block);
    WH_HIP(hipGetLastError());
    WH_HIP(hipMemcpyAsync(values, c->x_in.p, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    return WH_OK;
}

static int routed_common(wh_ctx* c, const wh_expert_route* routes, size_t n, ExpertView* ev,
                         float* wts) {
    if (n > WH_MAX_EXPERTS) return WH_UNSUPPORTED;
    for (size_t i = 0; i < n; ++i) {
        WH_TRY(resolve_expert(c, routes[i].layer_id, routes[i].expert_id, &ev[i]));
        wts[i] = routes[i].route_weight;
    }
    return WH_OK;
}

int wh_routed_experts(wh_ctx* c, const wh_expert_route* routes, size_t n, float* hidden,
                      size_t hidden_len) {
    if (!c) return WH_INVALID_ARGUMENT;
    if (n == 0) return WH_OK;  // E/compute.rs:1956-1958
    if (!routes || !hidden) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    ExpertView ev[WH_MAX_EXPERTS];
    float wts[WH_MAX_EXPERTS];
    WH_TRY(routed_common(c, routes, n, ev, wts));
    const size_t hsz = ev[0].w1->cols, osz = ev[0].w2->rows;
    if (hidden_len < hsz) return WH_INVALID_SHAPE;  // "DeepSeek FP4 expert input dim"
    if (osz > hidden_len) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(c->x_in.ensure(hsz * sizeof(float), false));
    WH_HIP(c->y_out.ensure(osz * sizeof(float), false));
    WH_HIP(c->stage_out.ensure(osz * sizeof(float)));
    WH_HIP(hipMemcpyAsync(c->x_in.p, hidden, hsz * sizeof(float), hipMemcpyHostToDevice, c->stream));
    WH_TRY(moe_forward(c, ev, wts, n, false, c->x_in.p, 0, 1, c->y_out.as<float>()));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->y_out.p, osz * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    int st = read_status(c);
    if (st != WH_OK) return st;
    std::memcpy(hidden, c->stage_out.p, osz * sizeof(float));
    return WH_OK;
}

int wh_routed_experts_async(wh_ctx* c, const wh_expert_route* routes, size_t n, const void* x_dev,
                            int x_bf16, size_t n_tokens, float* out_dev) {
    if (!c || !routes || !x_dev || !out_dev || n == 0 || n_tokens == 0) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    ExpertView ev[WH_MAX_EXPERTS];
    float wts[WH_MAX_EXPERTS];
    WH_TRY(routed_common(c, routes, n, ev, wts));
    return moe_forward(c, ev, wts, n, false, x_dev, x_bf16, n_tokens, out_dev);
}

// Routed experts plus the shared expert keyed (shared_layer, shared_expert).
static int routed_shared_common(wh_ctx* c, const wh_expert_route* routes, size_t n, uint32_t shared_layer,
                                uint32_t shared_expert, ExpertView* ev, float* wts) {
    if (n + 1 > WH_MAX_EXPERTS) return WH_UNSUPPORTED;
    if (n) WH_TRY(routed_common(c, routes, n, ev, wts));
    return resolve_expert(c, shared_layer, shared_expert, &ev[n]);
}

int wh_routed_and_shared_experts(wh_ctx* c, const wh_expert_route* routes, size_t n, uint32_t shared_layer,
                                 uint32_t shared_expert, float* hidden, size_t hidden_len) {
    if (!c || !hidden || (n && !routes)) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    ExpertView ev[WH_MAX_EXPERTS];
    float wts[WH_MAX_EXPERTS];
    WH_TRY(routed_shared_common(c, routes, n, shared_layer, shared_expert, ev, wts));
    const size_t hsz = ev[n].w1->cols, osz = ev[n].w2->rows;
    if (hidden_len < hsz) return WH_INVALID_SHAPE;  // "hidden_states is empty" / input dim
    if (osz > hidden_len) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(c->x_in.ensure(hsz * sizeof(float), false));
    WH_HIP(c->y_out.ensure(osz * sizeof(float), false));
    WH_HIP(c->stage_out.ensure(osz * sizeof(float)));
    WH_HIP(hipMemcpyAsync(c->x_in.p, hidden, hsz * sizeof(float), hipMemcpyHostToDevice, c->stream));
    WH_TRY(moe_forward(c, ev, wts, n + 1, true, c->x_in.p, 0, 1, c->y_out.as<float>()));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->y_out.p, osz * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    int st = read_status(c);
    if (st != WH_OK) return st;
    std::memcpy(hidden, c->stage_out.p, osz * sizeof(float));
    return WH_OK;
}

int wh_routed_and_shared_experts_async(wh_ctx* c, const wh_expert_route* routes, size_t n, uint32_t shared_layer,
                                       uint32_t shared_expert, const void* x_dev, int x_bf16, size_t n_tokens,
                                       float* out_dev) {
    if (!c || !x_dev || !out_dev || n_tokens == 0 || (n && !routes)) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    ExpertView ev[WH_MAX_EXPERTS];
    float wts[WH_MAX_EXPERTS];
    WH_TRY(routed_shared_common(c, routes, n, shared_layer, shared_expert, ev, wts));
    return moe_forward(c, ev, wts, n + 1, true, x_dev, x_bf16, n_tokens, out_dev);
}

int moe_dev_prepare(wh_ctx* c, uint32_t layer_id, size_t n_slots, uint32_t shared_layer, uint32_t shared_expert,
                    MoeDevPrep* m) {
    LayerTable* t = nullptr;
    WH_TRY(layer_table(c, layer_id, &t));
    const bool has_shared = shared_expert != WH_NO_SHARED_EXPERT;
    ExpertView sh;
    if (has_shared) WH_TRY(resolve_expert(c, shared_layer, shared_expert, &sh));
    if (t->resident == 0 && !has_shared) return WH_NOT_RESIDENT;
    if (n_slots == 0 || n_slots + (has_shared ? 1 : 0) > WH_MAX_EXPERTS) return WH_INVALID_ARGUMENT;
    // every resident expert (and the shared one) on one fast shape
    size_t hidden = t->hidden, inter = t->inter;
    bool fast = t->resident ? t->fast : true;
    if (has_shared) {
        if (!t->resident) hidden = sh.w1->cols, inter = sh.w1->rows;
        fast = fast && expert_fast(sh) && sh.w1->cols == hidden && sh.w1->rows == inter && sh.w2->rows == hidden;
    }
    if (!fast) return WH_UNSUPPORTED;
    WH_HIP(c->moe_dyn.ensure(sizeof(wh_moe_dyn), false));
    m->t = t;
    m->dyn = c->moe_dyn.as<wh_moe_dyn>();
    m->shp = {};
    if (has_shared) {
        m->shp.w1 = sh.w1->w;
        m->shp.s1 = (const uint8_t*)sh.w1->s;
        m->shp.w3 = sh.w3->w;
        m->shp.s3 = (const uint8_t*)sh.w3->s;
        m->shp.w2 = sh.w2->w;
        m->shp.s2 = (const uint8_t*)sh.w2->s;
    }
    m->has_shared = has_shared;
    m->n_slots = n_slots;
    m->hidden = hidden;
    m->inter = inter;
    m->zero_scale = t->zero_scale || (has_shared && expert_zero_scale(sh));
    return WH_OK;
}

// The route-list resolve as its own launch (k_moe_resolve).
int moe_dev_resolve(wh_ctx* c, const MoeDevPrep& m, const uint32_t* ids_dev, const float* w_dev,
                    const uint32_t* count_dev) {
    k_moe_resolve<<<1, 64, 0, c->stream>>>(ids_dev, w_dev, count_dev, m.t->dev, m.t->n, m.shp,
                                          m.has_shared ? 1u : 0u, (uint32_t)m.n_slots, m.dyn, c->status);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// The fast expert kernels on the resolved list (m.dyn).
int moe_dev_experts(wh_ctx* c, const MoeDevPrep& m, const void* x_dev, int x_bf16, float* out_dev) {
    const size_t n = m.n_slots + (m.has_shared ? 1 : 0);
    MoeBufs bufs;
    WH_TRY(moe_bufs_ctx(c, n, 1, m.hidden, m.inter, &bufs));
    MoeDyn md;
    md.p = m.dyn;
    md.hidden = m.hidden;
    md.inter = m.inter;
    md.zero_scale = m.zero_scale;
    return moe_launch_fast(c, nullptr, nullptr, n, m.has_shared, x_dev, x_bf16, 1, out_dev, 3u, bufs, true, &md);
}

// The experts of one token whose route list is in device memory: resolved
// on the device (k_moe_resolve), then the fast kernels with the list as
// their wh_moe_dyn.
int moe_dev_routes(wh_ctx* c, uint32_t layer_id, const uint32_t* ids_dev, const float* w_dev,
                   const uint32_t* count_dev, size_t n_slots, uint32_t shared_layer, uint32_t shared_expert,
                   const void* x_dev, int x_bf16, float* out_dev) {
    MoeDevPrep m;
    WH_TRY(moe_dev_prepare(c, layer_id, n_slots, shared_layer, shared_expert, &m));
    WH_TRY(moe_dev_resolve(c, m, ids_dev, w_dev, count_dev));
    return moe_dev_experts(c, m, x_dev, x_bf16, out_dev);
}

int wh_routed_and_shared_experts_dev_async(wh_ctx* c, uint32_t layer_id, const uint32_t* ids_dev,
                                           const float* weights_dev, const uint32_t* count_dev, size_t n_slots,
                                           uint32_t shared_layer, uint32_t shared_expert, const void* x_dev,
                                           int x_is_bf16, float* out_dev) {
    if (!c || !ids_dev || !weights_dev || !count_dev || !x_dev || !out_dev) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    return moe_dev_routes(c, layer_id, ids_dev, weights_dev, count_dev, n_slots, shared_layer, shared_expert, x_dev,
                          x_is_bf16, out_dev);
}

int wh_routed_and_shared_experts_noalloc_async(wh_ctx* c, const wh_expert_route* routes, size_t n,
                                               uint32_t shared_layer, uint32_t shared_expert, const void* x_dev,
                                               int x_bf16, size_t n_tokens, float* out_dev) {
    if (!c || !x_dev || !out_dev || n_tokens == 0 || (n && !routes)) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    ExpertView ev[WH_MAX_EXPERTS];
    float wts[WH_MAX_EXPERTS];
    WH_TRY(routed_shared_common(c, routes, n, shared_layer, shared_expert, ev, wts));
    bool fast = false;
    WH_TRY(moe_shapes(ev, n + 1, &fast));
    if (!fast) {
        std::snprintf(g_last_error, sizeof g_last_error,
                      "allocation-free routed experts: the experts are not on the fast kernels' shapes");
        return WH_UNSUPPORTED;
    }
    const size_t hidden = ev[0].w1->cols, inter = ev[0].w1->rows;
    const MoeSizes z = moe_sizes(n + 1, n_tokens, hidden, inter);
    if (z.total() > WH_NOALLOC_SCRATCH_BYTES) {
        std::snprintf(g_last_error, sizeof g_last_error,
                      "allocation-free routed experts: %zu tokens x %zu experts need %zu bytes of working memory, "
                      "the fixed array holds %zu",
                      n_tokens, n + 1, z.total(), (size_t)WH_NOALLOC_SCRATCH_BYTES);
        return WH_SCRATCH_TOO_SMALL;
    }
    uint8_t* base = nullptr;
    {
        std::lock_guard<std::mutex> g(g_noalloc_mu);
        if (c->device < kMaxDevices) base = (uint8_t*)g_noalloc_ptr[c->device];
    }
    if (!base) {
        std::snprintf(g_last_error, sizeof g_last_error, "allocation-free routed experts: no working memory on device %d",
                      c->device);
        return WH_UNSUPPORTED;
    }
    MoeBufs b;
    b.h = (float*)base;
    b.y = (float*)(base + z.h);
    b.cnt = (uint32_t*)(base + z.h + z.y);
    return moe_launch_fast(c, ev, wts, n + 1, true, x_dev, x_bf16, n_tokens, out_dev, 3u, b, false);
}

// ------------------------------------------------------ batched routed experts
// Shared lookups of both batch entry points: the layer table, the shared
// expert, and whether the fast path applies.
static int batch_setup(wh_ctx* c, uint32_t layer, size_t npos, size_t topk, uint32_t shared_layer,
                       uint32_t shared_expert, LayerTable** t, ExpertView* shared, bool* has_shared, bool* fast) {
    if (npos == 0 || topk == 0) return WH_INVALID_ARGUMENT;
    WH_TRY(layer_table(c, layer, t));
    if ((*t)->n == 0) return WH_NOT_RESIDENT;
    *has_shared = shared_expert != WH_NO_SHARED_EXPERT;
    if (*has_shared) WH_TRY(resolve_expert(c, shared_layer, shared_expert, shared));
    *fast = (*t)->fast && topk <= WH_BATCH_MAX_TOPK && topk + (*has_shared ? 1 : 0) <= WH_BATCH_MAX_ASSIGN &&
            wh_batch_wg_lds((*t)->hidden) <= g_max_lds && wh_batch_wg_lds((*t)->inter) <= g_max_lds;
    if (*has_shared)
        *fast = *fast && expert_fast(*shared) && shared->w1->cols == (*t)->hidden &&
                shared->w1->rows == (*t)->inter && shared->w2->rows == (*t)->hidden;
    return WH_OK;
}

int wh_debug_moe_batch_read(wh_ctx* c, int which, void* out, size_t bytes) {
    if (!c || !out) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const size_t S = c->moe_last_slots, P = c->moe_last_npos, hidden = c->moe_last_hidden, inter = c->moe_last_inter;
    if (S == 0) return WH_INVALID_ARGUMENT;
    BatchBufs b;
    WH_TRY(batch_bufs(c, P, S, hidden, inter, &b));
    const void* src = nullptr;
    size_t n = 0;
    switch (which) {
        case 0: src = b.sorted; n = S * 4; break;
        case 1: src = b.g; n = S * inter * 4; break;
        case 2: src = b.u; n = S * inter * 4; break;
        case 8: src = b.hq; n = S * inter * 4; break;
        case 3: src = b.y; n = S * hidden * 4; break;
        case 4: src = b.meta; n = 8 * 4; break;
        case 5: src = b.uoff; n = (S + 1) * 4; break;
        case 6: src = b.uexp; n = S * 4; break;
        case 7: src = b.uorder; n = S * 4; break;
        default: return WH_INVALID_ARGUMENT;
    }
    if (bytes < n) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(hipStreamSynchronize(c->stream));
    WH_HIP(hipMemcpy(out, src, n, hipMemcpyDeviceToHost));
    return WH_OK;
}

int wh_set_exact_numerics(wh_ctx* c, int on) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    c->exact = on != 0;
    return WH_OK;
}

int wh_debug_token_kernels(wh_ctx* c, int mask) {
    if (!c || mask < 0 || mask > 3) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    c->token_kernels = mask;
    return WH_OK;
}

int wh_debug_moe_token_capture(wh_ctx* c, int on) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    c->capture_gu = on != 0;
    return WH_OK;
}

int wh_debug_moe_token_read(wh_ctx* c, int which, void* out, size_t bytes) {
    if (!c || !out) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const size_t T = c->tok_last_tokens, n = c->tok_last_n, hidden = c->tok_last_hidden, inter = c->tok_last_inter;
    if (T == 0) return WH_INVALID_ARGUMENT;
    const void* src = nullptr;
    size_t len = 0;
    switch (which) {
        case 0:
            if (!c->capture_gu || c->gu.n < T * n * 2 * inter * sizeof(float)) return WH_INVALID_ARGUMENT;
            src = c->gu.p, len = T * n * 2 * inter * sizeof(float);
            break;
        case 1: src = c->h.p, len = T * n * inter * sizeof(float); break;
        case 2: src = c->ybuf.p, len = T * n * hidden * sizeof(float); break;
        default: return WH_INVALID_ARGUMENT;
    }
    if (bytes < len) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(hipStreamSynchronize(c->stream));
    WH_HIP(hipMemcpy(out, src, len, hipMemcpyDeviceToHost));
    return WH_OK;
}

int wh_set_moe_mfma_min(wh_ctx* c, uint32_t min_tokens) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    c->moe_mfma_min = min_tokens;
    return WH_OK;
}

int wh_moe_batch(wh_ctx* c, uint32_t layer_id, const uint32_t* route_ids, const float* route_scores, size_t npos,
                 size_t topk, uint32_t shared_layer, uint32_t shared_expert, const float* x, size_t x_len,
                 float* out, size_t out_len) {
    if (!c || !route_ids || !route_scores || !x || !out) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    LayerTable* t = nullptr;
    ExpertView sh;
    bool has_shared = false, fast = false;
    WH_TRY(batch_setup(c, layer_id, npos, topk, shared_layer, shared_expert, &t, &sh, &has_shared, &fast));
    for (size_t i = 0; i < npos * topk; ++i)
        if (!c->experts.count({layer_id, route_ids[i]})) return WH_NOT_RESIDENT;
    size_t hidden = t->hidden;
    if (!fast) {
        ExpertView v;
        WH_TRY(resolve_expert(c, layer_id, route_ids[0], &v));
        hidden = v.w1->cols;
    }
    if (x_len < npos * hidden) return WH_INPUT_TOO_SMALL;
    if (out_len < npos * hidden) return WH_OUTPUT_TOO_SMALL;
    WH_HIP(c->x_in.ensure(npos * hidden * sizeof(float), false));
    WH_HIP(c->bout.ensure(npos * hidden * sizeof(float), false));
    WH_HIP(c->stage_out.ensure(npos * hidden * sizeof(float)));
    WH_HIP(hipMemcpyAsync(c->x_in.p, x, npos * hidden * sizeof(float), hipMemcpyHostToDevice, c->stream));
    if (fast) {
        WH_HIP(c->routes.ensure(npos * topk * 8, false));
        uint32_t* ids_dev = c->routes.as<uint32_t>();
        float* sc_dev = (float*)(ids_dev + npos * topk);
        WH_HIP(hipMemcpyAsync(ids_dev, route_ids, npos * topk * 4, hipMemcpyHostToDevice, c->stream));
        WH_HIP(hipMemcpyAsync(sc_dev, route_scores, npos * topk * 4, hipMemcpyHostToDevice, c->stream));
        WH_TRY(moe_batch_fast(c, *t, ids_dev, sc_dev, npos, topk, has_shared ? &sh : nullptr, c->x_in.p, 0,
                              c->bout.as<float>()));
    } else {
        WH_TRY(moe_batch_generic(c, layer_id, route_ids, route_scores, npos, topk, has_shared ? &sh : nullptr,
                                 c->x_in.as<float>(), c->bout.as<float>()));
    }
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->bout.p, npos * hidden * sizeof(float), hipMemcpyDeviceToHost,
                          c->stream));
    int st = read_status(c);
    if (st != WH_OK) return st;
    std::memcpy(out, c->stage_out.p, npos * hidden * sizeof(float));
    return WH_OK;
}

int wh_moe_batch_async(wh_ctx* c, uint32_t layer_id, const uint32_t* route_ids_dev, const float* route_scores_dev,
                       size_t npos, size_t topk, uint32_t shared_layer, uint32_t shared_expert, const void* x_dev,
                       int x_is_bf16, float* out_dev) {
    if (!c || !route_ids_dev || !route_scores_dev || !x_dev || !out_dev) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    LayerTable* t = nullptr;
    ExpertView sh;
    bool has_shared = false, fast = false;
    WH_TRY(batch_setup(c, layer_id, npos, topk, shared_layer, shared_expert, &t, &sh, &has_shared, &fast));
    if (fast) {
        if (((uintptr_t)x_dev & 15) || ((uintptr_t)out_dev & 3) || ((uintptr_t)route_ids_dev & 3) ||
            ((uintptr_t)route_scores_dev & 3))
            return WH_INVALID_ARGUMENT;
        return moe_batch_fast(c, *t, route_ids_dev, route_scores_dev, npos, topk, has_shared ? &sh : nullptr, x_dev,
                              x_is_bf16, out_dev);
    }
    // generic shapes: the union is built on the host
    if (x_is_bf16) return WH_UNSUPPORTED;
    std::vector<uint32_t> ids(npos * topk);
    std::vector<float> sc(npos * topk);
    WH_HIP(hipMemcpyAsync(ids.data(), route_ids_dev, ids.size() * 4, hipMemcpyDeviceToHost, c->stream));
    WH_HIP(hipMemcpyAsync(sc.data(), route_scores_dev, sc.size() * 4, hipMemcpyDeviceToHost, c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    return moe_batch_generic(c, layer_id, ids.data(), sc.data(), npos, topk, has_shared ? &sh : nullptr,
                             (const float*)x_dev, out_dev);
}

int wh_fp4_expert_forward(wh_ctx* c, uint32_t layer, uint32_t expert, const float* input,
                          size_t input_len, float* output, size_t output_len, size_t scratch_len) {
    if (!c || !input || !output) return WH_INVALID_ARGUMENT;
    ExpertView ev;
    {
        std::lock_guard<std::recursive_mutex> lk(c->mu);
        WH_TRY(resolve_expert(c, layer, expert, &ev));
    }
    // E/deepseek_v4.rs:567-580
    if (ev.w1->cols != input_len || ev.w3->cols != input_len || ev.w1->rows != ev.w3->rows ||
        ev.w2->cols != ev.w1->rows)
        return WH_INVALID_SHAPE;
    if (output_len < ev.w2->rows) return WH_OUTPUT_TOO_SMALL;
    if (scratch_len < ev.w1->rows * 2) return WH_SCRATCH_TOO_SMALL;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const size_t hsz = ev.w1->cols, osz = ev.w2->rows;
    WH_HIP(c->x_in.ensure(hsz * sizeof(float), false));
    WH_HIP(c->y_out.ensure(osz * sizeof(float), false));
    WH_HIP(c->stage_out.ensure(osz * sizeof(float)));
    WH_HIP(hipMemcpyAsync(c->x_in.p, input, hsz * sizeof(float), hipMemcpyHostToDevice, c->stream));
    float one = 1.0f;
    WH_TRY(moe_forward(c, &ev, &one, 1, false, c->x_in.p, 0, 1, c->y_out.as<float>()));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->y_out.p, osz * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    int st = read_status(c);
    if (st != WH_OK) return st;
    std::memcpy(output, c->stage_out.p, osz * sizeof(float));
    return WH_OK;
}

namespace {
// compute_deepseek_fp8_shared_expert_into_hidden (E/compute.rs:5545-5614) on
// device pointers: xq = act_quant(x); gate = W1 xq; up = W3 xq;
// h = act_quant(swiglu(gate, up)); y = W2 h.  Every stage is the bit-exact
// kernel of its own entry point.  x and y may alias (the reference works in
// place): x is copied to scratch first.
int fp8_shared_launch(wh_ctx* c, const Tensor& w1, const Tensor& w3, const Tensor& w2, const float* x_dev,
                      float* y_dev) {
    const size_t hidden = w1.cols, inter = w1.rows;
    WH_HIP(c->tmp.ensure((hidden + 3 * inter) * sizeof(float), false));
    float* xq = c->tmp.as<float>();
    float* gate = xq + hidden;
    float* up = gate + inter;
    float* h = up + inter;
    WH_HIP(hipMemcpyAsync(xq, x_dev, hidden * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    k_act_quant_inplace<<<(unsigned)((hidden + 63) / 64), 256, 0, c->stream>>>(xq, (uint32_t)hidden, 64);
    WH_TRY(launch_fp8(c, w1, 0, inter, xq, gate, 1, hidden, inter));
    WH_TRY(launch_fp8(c, w3, 0, inter, xq, up, 1, hidden, inter));
    k_swiglu_generic<<<(unsigned)((inter + 255) / 256), 256, 0, c->stream>>>(gate, up, h, (uint32_t)inter, c->status);
    k_act_quant_inplace<<<(unsigned)((inter + 63) / 64), 256, 0, c->stream>>>(h, (uint32_t)inter, 64);
    WH_TRY(launch_fp8(c, w2, 0, w2.rows, h, y_dev, 1, inter, w2.rows));
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// Shape rules of E/compute.rs:5558-5570.
int fp8_shared_check(wh_ctx* c, wh_tensor h1, wh_tensor h3, wh_tensor h2, const Tensor** w1, const Tensor** w3,
                     const Tensor** w2) {
    *w1 = find_tensor(c, h1);
    *w3 = find_tensor(c, h3);
    *w2 = find_tensor(c, h2);
    if (!*w1 || !*w3 || !*w2) return WH_NOT_RESIDENT;
    if ((*w1)->kind != kFp8 || (*w3)->kind != kFp8 || (*w2)->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    if ((*w3)->cols != (*w1)->cols) return WH_INVALID_SHAPE;  // "DeepSeek shared expert input dim"
    if ((*w1)->rows != (*w3)->rows || (*w2)->cols != (*w1)->rows)
        return WH_INVALID_SHAPE;  // "DeepSeek shared expert projection shape"
    return WH_OK;
}
}  // namespace

int wh_fp8_shared_expert(wh_ctx* c, wh_tensor w1, wh_tensor w3, wh_tensor w2, const float* input, size_t input_len,
                         float* output, size_t output_len) {
    if (!c || !input || !output) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const Tensor *t1, *t3, *t2;
    WH_TRY(fp8_shared_check(c, w1, w3, w2, &t1, &t3, &t2));
    if (t1->cols != input_len) return WH_INVALID_SHAPE;  // "DeepSeek shared expert input dim"
    if (t2->rows > output_len) return WH_OUTPUT_TOO_SMALL;
    const size_t hidden = t1->cols, osz = t2->rows;
    WH_HIP(c->x_in.ensure(hidden * sizeof(float), false));
    WH_HIP(c->y_out.ensure(osz * sizeof(float), false));
    WH_HIP(c->stage_out.ensure(osz * sizeof(float)));
    WH_HIP(hipMemcpyAsync(c->x_in.p, input, hidden * sizeof(float), hipMemcpyHostToDevice, c->stream));
    WH_TRY(fp8_shared_launch(c, *t1, *t3, *t2, c->x_in.as<float>(), c->y_out.as<float>()));
    WH_HIP(hipMemcpyAsync(c->stage_out.p, c->y_out.p, osz * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    const int st = read_status(c);
    if (st != WH_OK) return st;
    std::memcpy(output, c->stage_out.p, osz * sizeof(float));
    return WH_OK;
}

int wh_fp8_shared_expert_async(wh_ctx* c, wh_tensor w1, wh_tensor w3, wh_tensor w2, const float* x_dev,
                               float* y_dev) {
    if (!c || !x_dev || !y_dev) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const Tensor *t1, *t3, *t2;
    WH_TRY(fp8_shared_check(c, w1, w3, w2, &t1, &t3, &t2));
    return fp8_shared_launch(c, *t1, *t3, *t2, x_dev, y_dev);
}

int wh_device_alloc(wh_ctx* c, size_t bytes, void** out) {
    if (!c || !out) return WH_INVALID_ARGUMENT;
    *out = nullptr;
    if (bytes == 0) return WH_OK;
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(hipMalloc(out, bytes));
    return WH_OK;
}

int wh_device_free(wh_ctx* c, void* p) {
    if (!c) return WH_INVALID_ARGUMENT;
    if (!p) return WH_OK;
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(hipStreamSynchronize(c->stream));
    WH_HIP(hipFree(p));
    return WH_OK;
}

int wh_memcpy(wh_ctx* c, void* dst, const void* src, size_t bytes, int kind) {
    if (!c || (bytes && (!dst || !src)) || kind < 0 || kind > 2) return WH_INVALID_ARGUMENT;
    if (bytes == 0) return WH_OK;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const hipMemcpyKind kinds[3] = {hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice};
    WH_HIP(hipMemcpyAsync(dst, src, bytes, kinds[kind], c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    return WH_OK;
}

int wh_timer_start(wh_ctx* c) {
    if (!c) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(hipEventRecord(c->timer[0], c->stream));
    return WH_OK;
}

int wh_timer_stop(wh_ctx* c, double* elapsed_us) {
    if (!c || !elapsed_us) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(hipEventRecord(c->timer[1], c->stream));
    WH_HIP(hipEventSynchronize(c->timer[1]));
    float ms = 0.0f;
    WH_HIP(hipEventElapsedTime(&ms, c->timer[0], c->timer[1]));
    *elapsed_us = (double)ms * 1000.0;
    return WH_OK;
}

int wh_probe_read_floor(wh_ctx* c, const void* buf_dev, size_t buf_bytes, size_t bytes, size_t reps,
                        double* best_us, uint32_t* best_grid, uint32_t* best_depth, double* empty_us) {
    if (!c || !buf_dev || !best_us || !best_grid || !best_depth || !empty_us || reps == 0 || bytes < 16 ||
        bytes % 16 || ((uintptr_t)buf_dev & 15))
        return WH_INVALID_ARGUMENT;
    const size_t stride = (bytes + 4095) & ~(size_t)4095;  // window pitch
    if (buf_bytes < stride) return WH_INVALID_SHAPE;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(c->y_out.ensure(8192 * sizeof(uint32_t), false));
    uint32_t* out = c->y_out.as<uint32_t>();
    const size_t windows = std::min<size_t>(buf_bytes / stride, 300);
    const size_t total16 = bytes / 16;
    auto time_it = [&](auto&& launch, size_t n, double* us) -> int {
        for (size_t i = 0; i < 5; ++i) launch(i);
        WH_HIP(hipEventRecord(c->timer[0], c->stream));
        for (size_t i = 0; i < n; ++i) launch(i + 7);
        WH_HIP(hipEventRecord(c->timer[1], c->stream));
        WH_HIP(hipEventSynchronize(c->timer[1]));
        float ms = 0.0f;
        WH_HIP(hipEventElapsedTime(&ms, c->timer[0], c->timer[1]));
        *us = (double)ms * 1000.0 / (double)n;
        return WH_OK;
    };
    WH_TRY(time_it([&](size_t) { k_empty_launch<<<1024, 256, 0, c->stream>>>(out); }, 200, empty_us));
    *best_us = 0.0;
    for (uint32_t grid : {256u, 512u, 1024u, 2048u, 4096u, 8192u}) {
        const size_t chunk16 = (total16 + grid - 1) / grid;  // every unit in [0, total16) is read once
        for (uint32_t depth : {4u, 8u, 16u}) {
            auto launch = [&](size_t i) {
                const uint4* b = (const uint4*)((const uint8_t*)buf_dev + (i % windows) * stride);
                if (depth == 4) k_read_floor<4><<<grid, 256, 0, c->stream>>>(b, chunk16, total16, out);
                else if (depth == 8) k_read_floor<8><<<grid, 256, 0, c->stream>>>(b, chunk16, total16, out);
                else k_read_floor<16><<<grid, 256, 0, c->stream>>>(b, chunk16, total16, out);
            };
            double us = 0.0;
            WH_TRY(time_it(launch, reps, &us));
            if (*best_us == 0.0 || us < *best_us) {
                *best_us = us;
                *best_grid = grid;
                *best_depth = depth;
            }
        }
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int wh_profile_routed(wh_ctx* c, const wh_expert_route* routes, size_t n_routes, size_t n_sets,
                      const void* x_dev, int x_bf16, float* out_dev, size_t iters, double* us_per_launch) {
    if (!c || !routes || !x_dev || !out_dev || !us_per_launch || n_routes == 0 || n_sets == 0 || iters == 0 ||
        n_routes > WH_MAX_EXPERTS)
        return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    std::vector<ExpertView> ev(n_sets * n_routes);
    std::vector<float> wts(n_sets * n_routes);
    for (size_t s = 0; s < n_sets; ++s) {
        WH_TRY(routed_common(c, routes + s * n_routes, n_routes, &ev[s * n_routes], &wts[s * n_routes]));
        const ExpertView* e = &ev[s * n_routes];
        for (size_t i = 0; i < n_routes; ++i)
            if (!expert_fast(e[i]) || e[i].w1->cols != e[0].w1->cols || e[i].w1->rows != e[0].w1->rows ||
                e[i].w2->rows != e[0].w1->cols)
                return WH_UNSUPPORTED;
    }
    MoeBufs bufs;
    WH_TRY(moe_bufs_ctx(c, n_routes, 1, ev[0].w1->cols, ev[0].w1->rows, &bufs));
    for (unsigned stage = 1; stage <= 2; ++stage) {
        WH_HIP(hipEventRecord(c->timer[0], c->stream));
        for (size_t it = 0; it < iters; ++it) {
            const size_t s = it % n_sets;
            WH_TRY(moe_launch_fast(c, &ev[s * n_routes], &wts[s * n_routes], n_routes, false, x_dev, x_bf16, 1,
                                   out_dev, stage, bufs, true));
        }
        WH_HIP(hipEventRecord(c->timer[1], c->stream));
        WH_HIP(hipEventSynchronize(c->timer[1]));
        float ms = 0.0f;
        WH_HIP(hipEventElapsedTime(&ms, c->timer[0], c->timer[1]));
        us_per_launch[stage - 1] = (double)ms * 1000.0 / (double)iters;
    }
    return read_status(c);
}

int wh_profile_token_pipeline(wh_ctx* c, const wh_expert_route* routes, size_t n_routes, size_t n_sets,
                              const void* x_dev, int x_bf16, size_t x_stride, float* out_dev, size_t iters, int mode,
                              double* us_per_token) {
    if (!c || !routes || !x_dev || !out_dev || !us_per_token || n_routes == 0 || n_sets == 0 || iters == 0 ||
        n_routes > WH_MAX_EXPERTS || mode < 0 || mode > 1 || (x_stride & 15))
        return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    std::vector<ExpertView> ev(n_sets * n_routes);
    std::vector<float> wts(n_sets * n_routes);
    for (size_t s = 0; s < n_sets; ++s) {
        WH_TRY(routed_common(c, routes + s * n_routes, n_routes, &ev[s * n_routes], &wts[s * n_routes]));
        const ExpertView* e = &ev[s * n_routes];
        for (size_t i = 0; i < n_routes; ++i)
            if (!expert_fast(e[i]) || e[i].w1->cols != e[0].w1->cols || e[i].w1->rows != e[0].w1->rows ||
                e[i].w2->rows != e[0].w1->cols)
                return WH_UNSUPPORTED;
    }
    const size_t hidden = ev[0].w1->cols;
    MoeBufs bufs;
    WH_TRY(moe_bufs_ctx(c, n_routes, 1, hidden, ev[0].w1->rows, &bufs));
    auto enqueue = [&]() -> int {
        for (size_t it = 0; it < iters; ++it) {
            const size_t s = it % n_sets;
            WH_TRY(moe_launch_fast(c, &ev[s * n_routes], &wts[s * n_routes], n_routes, false,
                                   (const uint8_t*)x_dev + s * x_stride, x_bf16, 1, out_dev + s * hidden, 3, bufs,
                                   true));
        }
        return WH_OK;
    };
    float ms = 0.0f;
    if (mode == 0) {
        WH_HIP(hipEventRecord(c->timer[0], c->stream));
        WH_TRY(enqueue());
        WH_HIP(hipEventRecord(c->timer[1], c->stream));
        WH_HIP(hipEventSynchronize(c->timer[1]));
        WH_HIP(hipEventElapsedTime(&ms, c->timer[0], c->timer[1]));
    } else {
        // the same launches captured once into a graph (kernel nodes only),
        // replayed once untimed and once between the events
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        WH_HIP(hipStreamSynchronize(c->stream));
        WH_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue();
        const hipError_t ce = hipStreamEndCapture(c->stream, &graph);
        if (rc != WH_OK || ce != hipSuccess) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc != WH_OK ? rc : hip_status(ce);
        }
        hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e == hipSuccess) e = hipGraphLaunch(exec, c->stream);
        if (e == hipSuccess) e = hipEventRecord(c->timer[0], c->stream);
        if (e == hipSuccess) e = hipGraphLaunch(exec, c->stream);
        if (e == hipSuccess) e = hipEventRecord(c->timer[1], c->stream);
        if (e == hipSuccess) e = hipEventSynchronize(c->timer[1]);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, c->timer[0], c->timer[1]);
        if (exec) (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        WH_HIP(e);
    }
    *us_per_token = (double)ms * 1000.0 / (double)iters;
    return read_status(c);
}

#ifdef WH_TIMELINE
// Timeline of the last persistent token kernels (builds with -DWH_TIMELINE
// only): which = 0 gate/up, 1 down; n <= 512 * 16 * WH_TL_POINTS stamps.
int wh_debug_timeline(int which, uint64_t* out, size_t n) {
    constexpr size_t kStamps = 512 * 16 * WH_TL_POINTS;
    if (which < 0 || which > 1 || n > kStamps) return WH_INVALID_ARGUMENT;
    WH_HIP(hipDeviceSynchronize());
    if (!out) {  // clears the kernel's stamps
        void* p = nullptr;
        WH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(wh_tl_buf)));
        WH_HIP(hipMemset((uint64_t*)p + (size_t)which * kStamps, 0, kStamps * sizeof(uint64_t)));
        WH_HIP(hipDeviceSynchronize());
        return WH_OK;
    }
    WH_HIP(hipMemcpyFromSymbol(out, HIP_SYMBOL(wh_tl_buf), n * sizeof(uint64_t), (size_t)which * kStamps * sizeof(uint64_t)));
    return WH_OK;
}
#endif

int wh_debug_eval(wh_ctx* c, int fn, const float* in, float* out, size_t n) {
    if (!c || !in || !out || fn < 0 || fn > 8) return WH_INVALID_ARGUMENT;
    if ((fn == 3 && n % 4) || (fn >= 7 && n % 64)) return WH_INVALID_ARGUMENT;
    if (n == 0) return WH_OK;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    WH_HIP(c->x_in.ensure(n * sizeof(float), false));
    WH_HIP(c->y_out.ensure(n * sizeof(float), false));
    WH_HIP(hipMemcpyAsync(c->x_in.p, in, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    if (fn == 3)
        k_copy_f32x4<<<(unsigned)std::min<size_t>((n / 4 + 255) / 256, 8192), 256, 0, c->stream>>>(
            reinterpret_cast<const float4*>(c->x_in.p), reinterpret_cast<float4*>(c->y_out.p), (uint32_t)(n / 4));
    else if (fn == 7)
        k_debug_tok_quant<true><<<(unsigned)((n / 8 + 255) / 256), 256, 0, c->stream>>>(c->x_in.as<float>(),
                                                                                    c->y_out.as<float>(), (uint32_t)n);
    else if (fn == 8)
        k_debug_tok_quant<false><<<(unsigned)((n / 8 + 255) / 256), 256, 0, c->stream>>>(c->x_in.as<float>(),
                                                                                     c->y_out.as<float>(), (uint32_t)n);
    else if (fn >= 4)
        k_debug_eval_router<<<(unsigned)((n + 255) / 256), 256, 0, c->stream>>>(fn, c->x_in.as<float>(),
                                                                               c->y_out.as<float>(), (uint32_t)n);
    else
        k_debug_eval<<<(unsigned)((n + 255) / 256), 256, 0, c->stream>>>(fn, c->x_in.as<float>(), c->y_out.as<float>(), (uint32_t)n);
    WH_HIP(hipGetLastError());
    WH_HIP(hipMemcpyAsync(out, c->y_out.p, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    WH_HIP(hipStreamSynchronize(c->stream));
    return WH_OK;
}

}  // extern "C"

// ------------------------------------------------------------- MLA glue
namespace {
// rope_inv_freqs (E/compute.rs:2591-2620) in the reference's f32 arithmetic
// with the platform libm (powf, logf), on the host: a per-layer constant.
void rope_inv_freqs_host(size_t rope_dim, float theta, const wh_yarn* yarn, float* out) {
    const size_t pairs = rope_dim / 2;
    for (size_t p = 0; p < pairs; ++p) out[p] = powf(theta, -(float)(2 * p) / (float)rope_dim);
    if (!yarn || yarn->original_seq_len == 0) return;
    const float dim = (float)rope_dim;
    const float base_ln = logf(theta);
    const float pi = 3.14159265358979323846f;
    auto correction_dim = [&](float rotations) {
        return dim * logf((float)yarn->original_seq_len / (rotations * 2.0f * pi)) / (2.0f * base_ln);
    };
    const float low = fmaxf(floorf(correction_dim(yarn->beta_fast)), 0.0f);
    float high = fminf(ceilf(correction_dim(yarn->beta_slow)), dim - 1.0f);
    if (fabsf(low - high) < 1.1920929e-7f) high = low + 0.001f;
    for (size_t p = 0; p < pairs; ++p) {
        float ramp = ((float)p - low) / (high - low);
        ramp = ramp < 0.0f ? 0.0f : (ramp > 1.0f ? 1.0f : ramp);
        const float smooth = 1.0f - ramp;
        out[p] = out[p] / yarn->factor * (1.0f - smooth) + out[p] * smooth;
    }
}

// DEEPSEEK_V4_COMPRESS_RATIOS (E/compute.rs:2552-2555): 0 = sliding window only.
const uint32_t kCompressRatios[44] = {0, 0, 4, 128, 4, 128, 4, 128, 4, 128, 4, 128, 4, 128, 4,
                                      128, 4, 128, 4, 128, 4, 128, 4, 128, 4, 128, 4, 128, 4, 128,
                                      4, 128, 4, 128, 4, 128, 4, 128, 4, 128, 4, 128, 4, 0};

// The device copy of a layer type's inverse frequencies, made once.
int rope_table(wh_ctx* c, size_t rope_dim, float theta, const wh_yarn* yarn, const float** out) {
    char key[128];
    snprintf(key, sizeof key, "%zu/%08x/%d/%08x/%08x/%08x/%zu", rope_dim, wh_float_to_bits(theta), yarn != nullptr,
             yarn ? wh_float_to_bits(yarn->factor) : 0u, yarn ? wh_float_to_bits(yarn->beta_fast) : 0u,
             yarn ? wh_float_to_bits(yarn->beta_slow) : 0u, yarn ? yarn->original_seq_len : (size_t)0);
    auto it = c->rope_tabs.find(key);
    if (it == c->rope_tabs.end()) {
        std::vector<float> host(rope_dim / 2 + 1);
        rope_inv_freqs_host(rope_dim, theta, yarn, host.data());
        float* dev = nullptr;
        WH_HIP(hipMalloc(&dev, host.size() * sizeof(float)));
        const hipError_t e = hipMemcpy(dev, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(dev);
            return WH_HIP_ERROR;
        }
        it = c->rope_tabs.emplace(key, dev).first;
    }
    *out = it->second;
    return WH_OK;
}

int rowpost_launch(wh_ctx* c, const wh_rowpost_args& args) {
    if (args.rows == 0) return WH_OK;
    wh_rowpost_args a = args;
    a.tree = c->exact ? 0u : 1u;  // exact numerics off: the norms' sums of squares in a fixed tree
    // a lone row gets 1024 threads (the act-quant's 64-value blocks and the
    // norm's terms spread over 16 waves), many rows 256 each
    if (a.rows < 16) k_rowpost<1024><<<a.rows, 1024, 0, c->stream>>>(a);
    else k_rowpost<256><<<a.rows, 256, 0, c->stream>>>(a);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

wh_rowpost_args rowpost_args(const float* x, float* out, size_t rows, size_t n, size_t ld_in, size_t ld_out) {
    wh_rowpost_args a{};
    a.x = x;
    a.out = out;
    a.rows = (uint32_t)rows;
    a.n = (uint32_t)n;
    a.ld_in = (uint32_t)ld_in;
    a.ld_out = (uint32_t)ld_out;
    return a;
}

int attn_launch(wh_ctx* c, const wh_attn_args& args) {
    wh_attn_args a = args;
    const unsigned gy = (a.heads + 3) / 4, nk = a.n_win + a.n_comp;
    a.wts_ld = (nk + 3) & ~3u;  // each head's weights 16-byte aligned
    k_attn_scores<<<dim3((nk + 63) / 64, gy), 256, 0, c->stream>>>(a);
    k_attn_combine<<<dim3(a.head_dim / 64, gy), 256, 4 * a.wts_ld * sizeof(float), c->stream>>>(a);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int attn_check(size_t heads, size_t head_dim, size_t nope_dim, size_t pairs, size_t n_keys, size_t token_pos) {
    if (heads == 0 || head_dim == 0) return WH_EMPTY_SHAPE;
    if (nope_dim + 2 * pairs > head_dim || (nope_dim & 1)) return WH_INVALID_SHAPE;
    if (head_dim % 64 || head_dim > WH_ATTN_MAX_HEAD_DIM || n_keys == 0 || n_keys > WH_ATTN_MAX_KEYS ||
        heads > 65535u * 4 || token_pos >= (1u << 24))
        return WH_UNSUPPORTED;
    return WH_OK;
}
}  // namespace

int wh_rope_inv_freqs(size_t rope_dim, float theta, const wh_yarn* yarn, float* out, size_t out_len) {
    if (!out && rope_dim / 2) return WH_INVALID_ARGUMENT;
    if (out_len < rope_dim / 2) return WH_OUTPUT_TOO_SMALL;
    rope_inv_freqs_host(rope_dim, theta, yarn, out);
    return WH_OK;
}

int wh_deepseek_rope_for_layer(uint32_t physical_layer, float* theta, wh_yarn* yarn, int* has_yarn) {
    if (!theta || !yarn || !has_yarn) return WH_INVALID_ARGUMENT;
    const uint32_t ratio = physical_layer < 44 ? kCompressRatios[physical_layer] : 0u;
    *has_yarn = ratio > 0;
    *theta = ratio > 0 ? 160000.0f : 10000.0f;
    yarn->factor = 16.0f;
    yarn->beta_fast = 32.0f;
    yarn->beta_slow = 1.0f;
    yarn->original_seq_len = 65536;
    return WH_OK;
}

int wh_rms_norm_async(wh_ctx* c, const float* x_dev, float* out_dev, size_t rows, size_t n,
                      const uint16_t* weight_bf16_dev) {
    if (!c || !x_dev || !out_dev) return WH_INVALID_ARGUMENT;
    if (rows == 0 || n == 0) return WH_OK;  // E/compute.rs:7111-7113: an empty slice is left alone
    if (n > WH_ROWPOST_MAX || rows > 0x7fffffffu) return WH_UNSUPPORTED;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    wh_rowpost_args a = rowpost_args(x_dev, out_dev, rows, n, n, n);
    a.norm = 1;
    a.w = weight_bf16_dev;
    return rowpost_launch(c, a);
}

int wh_rope_async(wh_ctx* c, float* values_dev, size_t rows, size_t row_stride, size_t offset,
                  const float* inv_freqs_dev, size_t pairs, size_t position, int inverse) {
    if (!c) return WH_INVALID_ARGUMENT;
    if (pairs == 0 || rows == 0) return WH_OK;  // E/compute.rs:2630-2632
    if (!values_dev || !inv_freqs_dev) return WH_INVALID_ARGUMENT;
    if (offset + 2 * pairs > row_stride) return WH_INVALID_SHAPE;  // "RoPE input shorter than dim"
    if (row_stride > WH_ROWPOST_MAX || rows > 0x7fffffffu || position >= (1u << 24)) return WH_UNSUPPORTED;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    wh_rowpost_args a = rowpost_args(values_dev, values_dev, rows, row_stride, row_stride, row_stride);
    a.inv_freqs = inv_freqs_dev;
    a.pairs = (uint32_t)pairs;
    a.rope_off = (uint32_t)offset;
    a.position = (uint32_t)position;
    a.inverse = inverse != 0;
    return rowpost_launch(c, a);
}

int wh_act_quant_dequant_async(wh_ctx* c, float* values_dev, size_t n, size_t block) {
    if (!c) return WH_INVALID_ARGUMENT;
    if (block == 0 || n == 0) return WH_OK;  // E/compute.rs:2505-2507
    if (!values_dev) return WH_INVALID_ARGUMENT;
    if (n > 0xffffffffu || (n + block - 1) / block > 0x7fffffffu) return WH_UNSUPPORTED;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    k_act_quant_inplace<<<(unsigned)((n + block - 1) / block), 256, 0, c->stream>>>(values_dev, (uint32_t)n,
                                                                                     (uint32_t)block);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int wh_window_attention_async(wh_ctx* c, const float* q_dev, size_t heads, size_t head_dim, size_t nope_dim,
                              const float* window_dev, size_t n_window, size_t window_stride, const float* comp_dev,
                              size_t n_comp, const float* sink_dev, const float* inv_freqs_dev, size_t pairs,
                              size_t token_pos, float* scores_dev, float* out_dev) {
    if (!c || !q_dev || !out_dev || !scores_dev || (n_window && !window_dev) || (n_comp && !comp_dev) ||
        (pairs && !inv_freqs_dev))
        return WH_INVALID_ARGUMENT;
    WH_TRY(attn_check(heads, head_dim, nope_dim, pairs, n_window + n_comp, token_pos));
    if (n_window > 1 && window_stride < head_dim) return WH_INVALID_SHAPE;
    if (window_stride > 0xffffffffu) return WH_UNSUPPORTED;
    // the score kernel reads keys as float4
    if ((window_stride & 3) || ((uintptr_t)window_dev & 15) || ((uintptr_t)comp_dev & 15)) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    wh_attn_args a{};
    a.q = q_dev;
    a.win = window_dev;
    a.comp = comp_dev;
    a.sink = sink_dev;
    a.inv_freqs = inv_freqs_dev;
    a.scores = scores_dev;
    a.out = out_dev;
    a.heads = (uint32_t)heads;
    a.head_dim = (uint32_t)head_dim;
    a.nope_dim = (uint32_t)nope_dim;
    a.pairs = (uint32_t)pairs;
    a.n_win = (uint32_t)n_window;
    a.n_comp = (uint32_t)n_comp;
    a.win_ld = (uint32_t)window_stride;
    a.token_pos = (uint32_t)token_pos;
    a.scale = powf((float)head_dim, -0.5f);
    return attn_launch(c, a);
}

// The attention's input as its first launch reads it: x (rows ld floats
// apart), optionally the end of hc_pre (y = sum of pre-weighted copies,
// hc > 0) and the RMS norm (norm, weights w or none), then the act-quant.
// The decode layers pass hc_pre's copies and the attention norm, so that
// neither y nor the norm output takes a launch of its own (the same values).
struct MlaIn {
    const float* x;
    size_t ld;
    int norm;
    const uint16_t* w;
    const float* pre;
    size_t hc, hc_stride;
};

// The single-token attention with its input in.x and its output in
// hidden_dev.
static int mla_decode_impl(wh_ctx* c, const wh_mla_layer* L, size_t token_pos, const MlaIn& in, float* hidden_dev,
                           float* kv_cache_dev, size_t kv_stride, size_t kv_capacity, const float* comp_dev,
                           size_t n_comp) {
    const float* in_dev = in.x;
    if (!c || !L || !in_dev || !hidden_dev || !kv_cache_dev || (n_comp && !comp_dev)) return WH_INVALID_ARGUMENT;
    if ((uintptr_t)in_dev & 15) return WH_INVALID_ARGUMENT;
    const size_t heads = L->heads, nope = L->nope_dim, rope = L->rope_dim, head_dim = nope + rope;
    const size_t q_full = heads * head_dim, groups = L->o_groups, o_lora = L->o_lora_rank;
    // E/compute.rs:3932-3950
    if (groups == 0 || o_lora == 0 || q_full == 0 || q_full % groups != 0) return WH_INVALID_SHAPE;
    if (rope % 2) return WH_INVALID_SHAPE;  // "RoPE dim must be even"
    const size_t group_in = q_full / groups, o_mid = groups * o_lora, pairs = rope / 2;
    if (kv_stride < head_dim || token_pos >= kv_capacity) return WH_INVALID_SHAPE;  // "MLA KV cache layout mismatch"
    const size_t context = token_pos + 1, window_start = context > 128 ? context - 128 : 0;
    const size_t n_win = context - window_start;
    WH_TRY(attn_check(heads, head_dim, nope, pairs, n_win + n_comp, token_pos));
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    const Tensor* wq_a = find_tensor(c, L->wq_a);
    const Tensor* wq_b = find_tensor(c, L->wq_b);
    const Tensor* wkv = find_tensor(c, L->wkv);
    const Tensor* wo_a = find_tensor(c, L->wo_a);
    const Tensor* wo_b = find_tensor(c, L->wo_b);
    if (!wq_a || !wq_b || !wkv || !wo_a || !wo_b) return WH_NOT_RESIDENT;
    for (const Tensor* t : {wq_a, wq_b, wkv, wo_a, wo_b})
        if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    const size_t hidden = wq_a->cols, q_lora = wq_a->rows;
    if (wkv->cols != hidden || wkv->rows != head_dim || wq_b->cols != q_lora || wq_b->rows != q_full ||
        wo_a->cols != group_in || wo_a->rows != o_mid || wo_b->cols != o_mid || wo_b->rows != hidden)
        return WH_INVALID_SHAPE;
    if (hidden > WH_ROWPOST_MAX || q_lora > WH_ROWPOST_MAX || kv_stride > 0xffffffffu) return WH_UNSUPPORTED;
    if (((uintptr_t)hidden_dev & 15) || ((uintptr_t)kv_cache_dev & 15) || ((uintptr_t)comp_dev & 15) ||
        (kv_stride & 3))
        return WH_INVALID_ARGUMENT;
    WH_HIP(hipSetDevice(c->device));
    float theta;
    wh_yarn yarn;
    int has_yarn;
    wh_deepseek_rope_for_layer(L->physical_layer, &theta, &yarn, &has_yarn);
    const float* inv = nullptr;
    WH_TRY(rope_table(c, rope, theta, has_yarn ? &yarn : nullptr, &inv));
    // activations, each 256-byte aligned
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t nk = n_win + n_comp;
    const size_t o_xq = 0, o_ql = o_xq + up(hidden), o_q = o_ql + up(q_lora), o_kv = o_q + up(q_full),
                 o_sc = o_kv + up(head_dim), o_at = o_sc + up(heads * nk), o_om = o_at + up(q_full),
                 total = o_om + up(o_mid);
    WH_HIP(c->mla.ensure(total * sizeof(float), false));
    float* base = c->mla.as<float>();
    float *xq = base + o_xq, *ql = base + o_ql, *q = base + o_q, *kvt = base + o_kv, *sc = base + o_sc,
          *at = base + o_at, *om = base + o_om;
    float* kv_row = kv_cache_dev + token_pos * kv_stride;
    // q path (E/compute.rs:3998-4040): act-quant of x, wq_a, q norm + act-quant,
    // wq_b, per-head RMS norm + RoPE
    wh_rowpost_args a = rowpost_args(in_dev, xq, 1, hidden, in.ld ? in.ld : hidden, hidden);
    a.norm = in.norm ? 1u : 0u;
    a.w = in.w;
    a.hc_pre = in.pre;
    a.hc = (uint32_t)in.hc;
    a.hc_stride = (uint32_t)in.hc_stride;
    a.aq_len = (uint32_t)hidden;
    WH_TRY(rowpost_launch(c, a));
    // wq_a and wkv both read the act-quantized x: one launch when they can
    // share it
    const bool pair = fp8_split_k(*wq_a) && fp8_split_k(*wkv) && wq_a->special == wkv->special &&
                      wq_a->scale_fmt == wkv->scale_fmt;
    if (pair)
        WH_TRY(launch_fp8(c, *wq_a, 0, q_lora, xq, ql, 1, hidden, q_lora, 0, 0, wkv, 0, head_dim, kvt));
    else
        WH_TRY(launch_fp8(c, *wq_a, 0, q_lora, xq, ql, 1, hidden, q_lora));
    a = rowpost_args(ql, ql, 1, q_lora, q_lora, q_lora);
    a.norm = 1;
    a.w = L->q_norm_bf16;
    a.aq_len = (uint32_t)q_lora;
    WH_TRY(rowpost_launch(c, a));
    WH_TRY(launch_fp8(c, *wq_b, 0, q_full, ql, q, 1, q_lora, q_full));
    a = rowpost_args(q, q, heads, head_dim, head_dim, head_dim);
    a.norm = 1;
    a.inv_freqs = inv;
    a.pairs = (uint32_t)pairs;
    a.rope_off = (uint32_t)nope;
    a.position = (uint32_t)token_pos;
    WH_TRY(rowpost_launch(c, a));
    // kv path (E/compute.rs:4046-4075): wkv, kv norm, RoPE, act-quant of the
    // non-rope dims, into the cache row of this position
    if (!pair) WH_TRY(launch_fp8(c, *wkv, 0, head_dim, xq, kvt, 1, hidden, head_dim));
    a = rowpost_args(kvt, kv_row, 1, head_dim, head_dim, head_dim);
    a.norm = 1;
    a.w = L->kv_norm_bf16;
    a.inv_freqs = inv;
    a.pairs = (uint32_t)pairs;
    a.rope_off = (uint32_t)nope;
    a.position = (uint32_t)token_pos;
    a.aq_len = (uint32_t)nope;
    WH_TRY(rowpost_launch(c, a));
    // window softmax with sink (E/compute.rs:4106-4197)
    wh_attn_args w{};
    w.q = q;
    w.win = kv_cache_dev + window_start * kv_stride;
    w.comp = comp_dev;
    w.sink = L->sink;
    w.inv_freqs = inv;
    w.scores = sc;
    w.out = at;
    w.heads = (uint32_t)heads;
    w.head_dim = (uint32_t)head_dim;
    w.nope_dim = (uint32_t)nope;
    w.pairs = (uint32_t)pairs;
    w.n_win = (uint32_t)n_win;
    w.n_comp = (uint32_t)n_comp;
    w.win_ld = (uint32_t)kv_stride;
    w.token_pos = (uint32_t)token_pos;
    w.scale = powf((float)head_dim, -0.5f);
    WH_TRY(attn_launch(c, w));
    // grouped output projection (E/compute.rs:4222-4270)
    k_act_quant_inplace<<<(unsigned)((q_full + 63) / 64), 256, 0, c->stream>>>(at, (uint32_t)q_full, 64);
    if (fp8_split_k(*wo_a) && is_pow2(o_lora) && o_lora >= WH_FP8_SK_ROWS && group_in <= 0xffffffffu) {
        WH_TRY(launch_fp8(c, *wo_a, 0, o_mid, at, om, 1, group_in, o_mid, o_lora, group_in));
    } else {
        for (size_t g = 0; g < groups; ++g)
            WH_TRY(launch_fp8(c, *wo_a, g * o_lora, (g + 1) * o_lora, at + g * group_in, om + g * o_lora, 1,
                              group_in, o_lora));
    }
    k_act_quant_inplace<<<(unsigned)((o_mid + 63) / 64), 256, 0, c->stream>>>(om, (uint32_t)o_mid, 64);
    WH_TRY(launch_fp8(c, *wo_b, 0, hidden, om, hidden_dev, 1, o_mid, hidden));
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int wh_mla_attention_decode_async(wh_ctx* c, const wh_mla_layer* L, size_t token_pos, float* hidden_dev,
                                  float* kv_cache_dev, size_t kv_stride, size_t kv_capacity, const float* comp_dev,
                                  size_t n_comp) {
    MlaIn in{};
    in.x = hidden_dev;
    return mla_decode_impl(c, L, token_pos, in, hidden_dev, kv_cache_dev, kv_stride, kv_capacity, comp_dev, n_comp);
}

// The batched MLA attention of prefill and MTP verify
// (compute_deepseek_v4_mla_attention_batch, E/compute.rs:4307-4641): the
// projections over all positions at once (rows_multi, bit-identical per
// input to the single-input kernels in exact numerics), the per-position
// norms, RoPE and KV cache rows, then every position's window softmax (a
// position reads only cache rows at or before its own, so writing every
// row first changes nothing), and the grouped output projections batched
// again.
// in as in mla_decode_impl, npos rows.
static int mla_decode_batch_impl(wh_ctx* c, const wh_mla_layer* L, const size_t* positions, size_t npos,
                                 const MlaIn& in, float* hidden_dev, float* kv_cache_dev, size_t kv_stride,
                                 size_t kv_capacity, const float* const* comp_dev, const size_t* n_comp) {
    const float* in_dev = in.x;
    if (!c || !L || !positions || !in_dev || !hidden_dev || !kv_cache_dev) return WH_INVALID_ARGUMENT;
    if ((uintptr_t)in_dev & 15) return WH_INVALID_ARGUMENT;
    if (npos == 0) return WH_INVALID_SHAPE;  // "MLA batch ys size"
    for (size_t i = 0; i < npos; ++i) {
        if (i && positions[i] <= positions[i - 1]) return WH_INVALID_ARGUMENT;  // ascending positions
        if (n_comp && n_comp[i] && (!comp_dev || !comp_dev[i])) return WH_INVALID_ARGUMENT;
    }
    const size_t heads = L->heads, nope = L->nope_dim, rope = L->rope_dim, head_dim = nope + rope;
    const size_t q_full = heads * head_dim, groups = L->o_groups, o_lora = L->o_lora_rank;
    if (groups == 0 || o_lora == 0 || q_full == 0 || q_full % groups != 0) return WH_INVALID_SHAPE;
    if (rope % 2) return WH_INVALID_SHAPE;
    const size_t group_in = q_full / groups, o_mid = groups * o_lora, pairs = rope / 2;
    if (kv_stride < head_dim || positions[npos - 1] >= kv_capacity) return WH_INVALID_SHAPE;
    size_t max_keys = 0;
    for (size_t i = 0; i < npos; ++i) {
        const size_t ctx_i = positions[i] + 1, nw = ctx_i - (ctx_i > 128 ? ctx_i - 128 : 0);
        const size_t nk = nw + (n_comp ? n_comp[i] : 0);
        WH_TRY(attn_check(heads, head_dim, nope, pairs, nk, positions[i]));
        max_keys = std::max(max_keys, nk);
    }
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    const Tensor* wq_a = find_tensor(c, L->wq_a);
    const Tensor* wq_b = find_tensor(c, L->wq_b);
    const Tensor* wkv = find_tensor(c, L->wkv);
    const Tensor* wo_a = find_tensor(c, L->wo_a);
    const Tensor* wo_b = find_tensor(c, L->wo_b);
    if (!wq_a || !wq_b || !wkv || !wo_a || !wo_b) return WH_NOT_RESIDENT;
    for (const Tensor* t : {wq_a, wq_b, wkv, wo_a, wo_b})
        if (t->kind != kFp8) return WH_INVALID_QUANT_FORMAT;
    const size_t hidden = wq_a->cols, q_lora = wq_a->rows;
    if (wkv->cols != hidden || wkv->rows != head_dim || wq_b->cols != q_lora || wq_b->rows != q_full ||
        wo_a->cols != group_in || wo_a->rows != o_mid || wo_b->cols != o_mid || wo_b->rows != hidden)
        return WH_INVALID_SHAPE;
    if (hidden > WH_ROWPOST_MAX || q_lora > WH_ROWPOST_MAX || kv_stride > 0xffffffffu || npos > 65535)
        return WH_UNSUPPORTED;
    if (((uintptr_t)hidden_dev & 15) || ((uintptr_t)kv_cache_dev & 15) || (kv_stride & 3)) return WH_INVALID_ARGUMENT;
    for (size_t i = 0; comp_dev && i < npos; ++i)
        if ((uintptr_t)comp_dev[i] & 15) return WH_INVALID_ARGUMENT;
    WH_HIP(hipSetDevice(c->device));
    float theta;
    wh_yarn yarn;
    int has_yarn;
    wh_deepseek_rope_for_layer(L->physical_layer, &theta, &yarn, &has_yarn);
    const float* inv = nullptr;
    WH_TRY(rope_table(c, rope, theta, has_yarn ? &yarn : nullptr, &inv));
    // activations of every position, each array 256-byte aligned
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t o_xq = 0, o_ql = o_xq + up(npos * hidden), o_q = o_ql + up(npos * q_lora),
                 o_kv = o_q + up(npos * q_full), o_sc = o_kv + up(npos * head_dim),
                 o_at = o_sc + up(std::min<size_t>(npos, WH_POS_BATCH) * heads * max_keys),
                 o_om = o_at + up(npos * q_full), total = o_om + up(npos * o_mid);
    WH_HIP(c->mla.ensure(total * sizeof(float), false));
    float* base = c->mla.as<float>();
    float *xq = base + o_xq, *ql = base + o_ql, *q = base + o_q, *kvt = base + o_kv, *sc = base + o_sc,
          *at = base + o_at, *om = base + o_om;
    // q and kv paths (E/compute.rs:4420-4490): act-quant of every x; wq_a
    // and wkv over all positions; q norm + act-quant; wq_b over all positions
    wh_rowpost_args a = rowpost_args(in_dev, xq, npos, hidden, in.ld ? in.ld : hidden, hidden);
    a.norm = in.norm ? 1u : 0u;
    a.w = in.w;
    a.hc_pre = in.pre;
    a.hc = (uint32_t)in.hc;
    a.hc_stride = (uint32_t)in.hc_stride;
    a.aq_len = (uint32_t)hidden;
    WH_TRY(rowpost_launch(c, a));
    WH_TRY(wh_fp8_gemv_multi_pair_async(c, L->wq_a, 0, q_lora, ql, q_lora, L->wkv, 0, head_dim, kvt, head_dim, xq, npos,
                                        hidden));
    a = rowpost_args(ql, ql, npos, q_lora, q_lora, q_lora);
    a.norm = 1;
    a.w = L->q_norm_bf16;
    a.aq_len = (uint32_t)q_lora;
    WH_TRY(rowpost_launch(c, a));
    WH_TRY(wh_fp8_gemv_multi_async(c, L->wq_b, 0, q_full, ql, npos, q_lora, q, q_full));
    // per position: per-head norm + RoPE of q; kv norm, RoPE, act-quant of
    // the non-rope dims into the position's cache row; up to WH_POS_BATCH
    // positions per launch
    for (size_t c0 = 0; c0 < npos; c0 += WH_POS_BATCH) {
        const size_t nb = std::min<size_t>(WH_POS_BATCH, npos - c0);
        a = rowpost_args(q + c0 * q_full, q + c0 * q_full, nb * heads, head_dim, head_dim, head_dim);
        a.norm = 1;
        a.inv_freqs = inv;
        a.pairs = (uint32_t)pairs;
        a.rope_off = (uint32_t)nope;
        a.rows_per_pos = (uint32_t)heads;
        for (size_t i = 0; i < nb; ++i) a.bpos[i] = (uint32_t)positions[c0 + i];
        WH_TRY(rowpost_launch(c, a));
        a = rowpost_args(kvt + c0 * head_dim, kv_cache_dev, nb, head_dim, head_dim, kv_stride);
        a.norm = 1;
        a.w = L->kv_norm_bf16;
        a.inv_freqs = inv;
        a.pairs = (uint32_t)pairs;
        a.rope_off = (uint32_t)nope;
        a.aq_len = (uint32_t)nope;
        a.rows_per_pos = 1;
        a.out_at_pos = 1;
        for (size_t i = 0; i < nb; ++i) a.bpos[i] = (uint32_t)positions[c0 + i];
        WH_TRY(rowpost_launch(c, a));
    }
    // every position's window softmax with sink (E/compute.rs:4497-4580),
    // after every cache row is written
    for (size_t c0 = 0; c0 < npos; c0 += WH_POS_BATCH) {
        const size_t nb = std::min<size_t>(WH_POS_BATCH, npos - c0);
        wh_attn_args w{};
        w.q = q + c0 * q_full;
        w.win = kv_cache_dev;
        w.sink = L->sink;
        w.inv_freqs = inv;
        w.scores = sc;
        w.out = at + c0 * q_full;
        w.heads = (uint32_t)heads;
        w.head_dim = (uint32_t)head_dim;
        w.nope_dim = (uint32_t)nope;
        w.pairs = (uint32_t)pairs;
        w.win_ld = (uint32_t)kv_stride;
        w.scale = powf((float)head_dim, -0.5f);
        w.nb = (uint32_t)nb;
        w.q_ld = (uint32_t)q_full;
        w.scores_ld = (uint32_t)(heads * max_keys);
        w.wlen = 128;
        w.wts_ld = (uint32_t)((max_keys + 3) & ~(size_t)3);  // each head's weights 16-byte aligned
        for (size_t i = 0; i < nb; ++i) {
            w.bpos[i] = (uint32_t)positions[c0 + i];
            w.bcomp[i] = comp_dev ? comp_dev[c0 + i] : nullptr;
            w.bncomp[i] = (uint32_t)(n_comp ? n_comp[c0 + i] : 0);
        }
        const unsigned gy = (unsigned)((heads + 3) / 4);
        k_attn_scores<<<dim3((unsigned)((max_keys + 63) / 64), gy, (unsigned)nb), 256, 0, c->stream>>>(w);
        k_attn_combine<<<dim3((unsigned)(head_dim / 64), gy, (unsigned)nb), 256, 4 * w.wts_ld * sizeof(float),
                         c->stream>>>(w);
        WH_HIP(hipGetLastError());
    }
    // o path (E/compute.rs:4582-4631): act-quant per position, wo_a per
    // output group over all positions, act-quant, wo_b over all positions
    k_act_quant_inplace<<<(unsigned)((npos * q_full + 63) / 64), 256, 0, c->stream>>>(at, (uint32_t)(npos * q_full),
                                                                                     64);
    WH_TRY(wh_fp8_gemv_multi_groups_async(c, L->wo_a, 0, o_mid, o_lora, at, group_in, npos, q_full, om, o_mid));
    if (o_mid % 64 == 0)  // (q_full is: head_dim % 64 == 0) the 64-blocks stay inside their position
        k_act_quant_inplace<<<(unsigned)((npos * o_mid + 63) / 64), 256, 0, c->stream>>>(om, (uint32_t)(npos * o_mid),
                                                                                        64);
    else
        for (size_t i = 0; i < npos; ++i)
            k_act_quant_inplace<<<(unsigned)((o_mid + 63) / 64), 256, 0, c->stream>>>(om + i * o_mid, (uint32_t)o_mid,
                                                                                     64);
    WH_TRY(wh_fp8_gemv_multi_async(c, L->wo_b, 0, hidden, om, npos, o_mid, hidden_dev, hidden));
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int wh_mla_attention_decode_batch_async(wh_ctx* c, const wh_mla_layer* L, const size_t* positions, size_t npos,
                                        float* hidden_dev, float* kv_cache_dev, size_t kv_stride, size_t kv_capacity,
                                        const float* const* comp_dev, const size_t* n_comp) {
    MlaIn in{};
    in.x = hidden_dev;
    return mla_decode_batch_impl(c, L, positions, npos, in, hidden_dev, kv_cache_dev, kv_stride, kv_capacity,
                                 comp_dev, n_comp);
}

// ------------------------------------------------------------------ mHC
namespace {
int hc_check(size_t hc, size_t hidden) {
    if (hc == 0 || hidden == 0) return WH_INVALID_SHAPE;  // "hc_pre sizes"
    if ((2 + hc) * hc + 1 > WH_HC_MAX_CHAINS || hc * hidden > 0xffffffffu) return WH_UNSUPPORTED;
    return WH_OK;
}

wh_hc_args hc_args(size_t hc, size_t hidden, size_t iters, float eps) {
    wh_hc_args a{};
    a.hc = (uint32_t)hc;
    a.hidden = (uint32_t)hidden;
    a.hc_dim = (uint32_t)(hc * hidden);
    a.mix_hc = (uint32_t)((2 + hc) * hc);
    a.iters = (uint32_t)std::min<size_t>(iters, 0x7fffffffu);
    a.eps = eps;
    return a;
}
}  // namespace

int wh_hc_split_sinkhorn_async(wh_ctx* c, const float* mixes_dev, const float* scale_dev, const float* base_dev,
                               size_t hc, size_t sinkhorn_iters, float eps, float* pre_dev, float* post_dev,
                               float* comb_dev) {
    if (!c || !mixes_dev || !scale_dev || !base_dev || !pre_dev || !post_dev || !comb_dev) return WH_INVALID_ARGUMENT;
    WH_TRY(hc_check(hc, 1));
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    wh_hc_args a = hc_args(hc, 1, sinkhorn_iters, eps);
    a.scale = scale_dev;
    a.base = base_dev;
    a.mixes_in = mixes_dev;
    a.pre = pre_dev;
    a.post = post_dev;
    a.comb = comb_dev;
    k_hc_finish<<<1, 256, 0, c->stream>>>(a);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

namespace {
// hc_pre of npos streams (x_dev npos x hc * hidden, y_dev npos x hidden,
// post_dev npos x hc, comb_dev npos x hc * hc) in one launch per stage.
// want_y false: y is left to the caller's next launch (a row kernel with
// hc_pre set), and *pre_out gets the pre weights (npos x hc, in the scratch)
int hc_pre_launch(wh_ctx* c, const float* fn_dev, const float* scale_dev, const float* base_dev, size_t hc,
                  size_t hidden, size_t sinkhorn_iters, float eps, const float* x_dev, float* y_dev, float* post_dev,
                  float* comb_dev, size_t npos, bool want_y = true, const float** pre_out = nullptr) {
    wh_hc_args a = hc_args(hc, hidden, sinkhorn_iters, eps);
    a.fn = fn_dev;
    a.scale = scale_dev;
    a.base = base_dev;
    a.x = x_dev;
    a.y = y_dev;
    a.post = post_dev;
    a.comb = comb_dev;
    a.parts = c->exact ? 1u : WH_HC_PARTS;
    const size_t n_sums = (size_t)WH_HC_PARTS * (a.mix_hc + 1);
    a.sums_ld = (uint32_t)((n_sums + 63) & ~(size_t)63);
    WH_HIP(c->hcs.ensure((npos * (a.sums_ld + hc) + 16) * sizeof(float), false));
    a.sums = c->hcs.as<float>();
    a.pre = a.sums + npos * a.sums_ld;
    const unsigned z = (unsigned)npos;
    if (c->exact) {
        k_hc_chains<<<dim3(a.mix_hc + 1, 1, z), 256, 0, c->stream>>>(a);
    } else {
        k_hc_partials<<<dim3(WH_HC_PARTS, a.mix_hc + 1, z), 256, 0, c->stream>>>(a);
    }
    k_hc_finish<<<z, 256, 0, c->stream>>>(a);
    if (want_y) k_hc_y<<<dim3((unsigned)((hidden + 255) / 256), z), 256, 0, c->stream>>>(a);
    if (pre_out) *pre_out = a.pre;
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int hc_post_launch(wh_ctx* c, const float* y_dev, const float* residual_dev, const float* post_dev,
                   const float* comb_dev, float* out_dev, size_t hc, size_t hidden, size_t npos) {
    const size_t n = hc * hidden;
    k_hc_post<<<dim3((unsigned)((n + 255) / 256), (unsigned)npos), 256, 0, c->stream>>>(
        y_dev, residual_dev, post_dev, comb_dev, out_dev, (uint32_t)hc, (uint32_t)hidden);
    WH_HIP(hipGetLastError());
    return WH_OK;
}
}  // namespace

int wh_hc_pre_async(wh_ctx* c, const float* fn_dev, const float* scale_dev, const float* base_dev, size_t hc,
                    size_t hidden, size_t sinkhorn_iters, float eps, const float* x_dev, float* y_dev,
                    float* post_dev, float* comb_dev) {
    if (!c || !fn_dev || !scale_dev || !base_dev || !x_dev || !y_dev || !post_dev || !comb_dev)
        return WH_INVALID_ARGUMENT;
    WH_TRY(hc_check(hc, hidden));
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    return hc_pre_launch(c, fn_dev, scale_dev, base_dev, hc, hidden, sinkhorn_iters, eps, x_dev, y_dev, post_dev,
                         comb_dev, 1);
}

int wh_hc_post_async(wh_ctx* c, const float* y_dev, const float* residual_dev, const float* post_dev,
                     const float* comb_dev, float* out_dev, size_t hc, size_t hidden) {
    if (!c || !y_dev || !residual_dev || !post_dev || !comb_dev || !out_dev) return WH_INVALID_ARGUMENT;
    WH_TRY(hc_check(hc, hidden));
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    return hc_post_launch(c, y_dev, residual_dev, post_dev, comb_dev, out_dev, hc, hidden, 1);
}


// compute_layer_deepseek_mhc (E/compute.rs:1448-1480) with the router between
// its phases (E/server/generation.rs:719-836), each step through the kernels
// of its own entry point.  The state ping-pongs between hidden_dev and
// scratch, so no copy of the residuals is made.
int wh_deepseek_mhc_layer_async(wh_ctx* c, const wh_mhc_layer* L, size_t token_pos, float* hidden_dev,
                                float* kv_cache_dev, size_t kv_stride, size_t kv_capacity, const float* comp_dev,
                                size_t n_comp) {
    if (!c || !L || !hidden_dev || ((uintptr_t)hidden_dev & 15)) return WH_INVALID_ARGUMENT;
    const size_t hc = L->hc, hidden = L->hidden;
    WH_TRY(hc_check(hc, hidden));
    if (L->active == 0) return WH_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    // scratch: the state after the attention sub-block, y, g, z, the two
    // hc_pre outputs (post, comb) and the route list, each 256-byte aligned
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t o_state = 0, o_y = up(hc * hidden), o_g = o_y + up(hidden), o_z = o_g + up(hidden);
    const size_t o_p1 = o_z + up(hidden), o_c1 = o_p1 + up(hc), o_p2 = o_c1 + up(hc * hc), o_c2 = o_p2 + up(hc);
    const size_t o_ids = o_c2 + up(hc * hc), o_w = o_ids + up(WH_ROUTER_MAX_ACTIVE), o_n = o_w + up(WH_ROUTER_MAX_ACTIVE);
    WH_HIP(c->layer.ensure((o_n + 64) * sizeof(float), false));
    float* f = c->layer.as<float>();
    float *state = f + o_state, *y = f + o_y, *g = f + o_g, *z = f + o_z;
    float *post1 = f + o_p1, *comb1 = f + o_c1, *post2 = f + o_p2, *comb2 = f + o_c2;
    uint32_t* ids = reinterpret_cast<uint32_t*>(f + o_ids);
    float* w = f + o_w;
    uint32_t* count = reinterpret_cast<uint32_t*>(f + o_n);
    // attention sub-block (E/compute.rs:1552-1605)
    if (!L->hc_attn_fn || !L->hc_attn_scale || !L->hc_attn_base || !L->hc_ffn_fn || !L->hc_ffn_scale ||
        !L->hc_ffn_base || hidden > WH_ROWPOST_MAX)
        return hidden > WH_ROWPOST_MAX ? WH_UNSUPPORTED : WH_INVALID_ARGUMENT;
    // hc_pre's y and the attention norm in the attention's first launch
    // (with the act-quant of its input); the output in g
    const float* pre = nullptr;
    WH_TRY(hc_pre_launch(c, L->hc_attn_fn, L->hc_attn_scale, L->hc_attn_base, hc, hidden, L->sinkhorn_iters, L->hc_eps,
                         hidden_dev, y, post1, comb1, 1, false, &pre));
    MlaIn in{};
    in.x = hidden_dev;
    in.ld = hc * hidden;
    in.norm = 1;
    in.w = L->attn_norm_bf16;
    in.pre = pre;
    in.hc = hc;
    in.hc_stride = hidden;
    WH_TRY(mla_decode_impl(c, &L->attn, token_pos, in, g, kv_cache_dev, kv_stride, kv_capacity, comp_dev, n_comp));
    WH_TRY(wh_hc_post_async(c, g, hidden_dev, post1, comb1, state, hc, hidden));
    // ffn hc_pre + norm: the gate input (E/compute.rs:1607-1630), y and the
    // norm in one launch
    WH_TRY(hc_pre_launch(c, L->hc_ffn_fn, L->hc_ffn_scale, L->hc_ffn_base, hc, hidden, L->sinkhorn_iters, L->hc_eps,
                         state, y, post2, comb2, 1, false, &pre));
    {
        wh_rowpost_args a = rowpost_args(state, g, 1, hidden, hc * hidden, hidden);
        a.norm = 1;
        a.w = L->ffn_norm_bf16;
        a.hc_pre = pre;
        a.hc = (uint32_t)hc;
        a.hc_stride = (uint32_t)hidden;
        WH_TRY(rowpost_launch(c, a));
    }
    // the router on the gate input, then the experts on its route list
    // (E/compute.rs:1641-1700); the route-list resolve in the router's last
    // workgroup where its one-launch selection applies
    MoeDevPrep mp;
    WH_TRY(moe_dev_prepare(c, L->layer_id, L->active, L->shared_layer, L->shared_expert, &mp));
    bool resolved = false;
    WH_TRY(route_experts(c, L->layer_id, g, hidden, L->active, L->available_dev, L->n_available, &L->route, ids, w,
                         count, &mp, &resolved));
    if (!resolved) WH_TRY(moe_dev_resolve(c, mp, ids, w, count));
    WH_TRY(moe_dev_experts(c, mp, g, 0, z));
    WH_TRY(wh_hc_post_async(c, z, state, post2, comb2, hidden_dev, hc, hidden));
    return WH_OK;
}

// The batched layer of prefill and MTP verify (E/server/generation.rs:
// 2437-2590): compute_layer_deepseek_mhc_phase1_batch (E/compute.rs:4649-
// 4750) over every position, the router per position, the union of the
// selected experts with each position's weights divided by their sum
// (E/server/generation.rs:2487-2506, the batch MoE), and
// finish_layer_deepseek_mhc_phase2_batch (E/compute.rs:1817-1870): shared
// expert + routed sum, hc_post.  hidden_dev holds npos states of hc * hidden.
int wh_deepseek_mhc_layer_batch_async(wh_ctx* c, const wh_mhc_layer* L, const size_t* positions, size_t npos,
                                      float* hidden_dev, float* kv_cache_dev, size_t kv_stride, size_t kv_capacity,
                                      const float* const* comp_dev, const size_t* n_comp,
                                      const int64_t* token_ids) {
    if (!c || !L || !positions || !hidden_dev || ((uintptr_t)hidden_dev & 15)) return WH_INVALID_ARGUMENT;
    if (npos == 0) return WH_INVALID_SHAPE;  // "mHC batch hidden state too small"
    const size_t hc = L->hc, hidden = L->hidden;
    WH_TRY(hc_check(hc, hidden));
    if (L->active == 0) return WH_INVALID_ARGUMENT;
    // the batch MoE takes a fixed number of routes per position: every
    // position's router must find `active` candidates
    if (L->available_dev && L->n_available < L->active) return WH_UNSUPPORTED;
    if (npos > 65535 || hidden % 4) return WH_UNSUPPORTED;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    WH_HIP(hipSetDevice(c->device));
    const size_t hcd = hc * hidden, slots = L->active;
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t o_state = 0, o_y = up(npos * hcd), o_g = o_y + up(npos * hidden), o_z = o_g + up(npos * hidden);
    const size_t o_p1 = o_z + up(npos * hidden), o_c1 = o_p1 + up(npos * hc), o_p2 = o_c1 + up(npos * hc * hc),
                 o_c2 = o_p2 + up(npos * hc), o_ids = o_c2 + up(npos * hc * hc), o_w = o_ids + up(npos * slots),
                 o_n = o_w + up(npos * slots), total = o_n + up(npos);
    WH_HIP(c->layer.ensure(total * sizeof(float), false));
    float* f = c->layer.as<float>();
    float *state = f + o_state, *y = f + o_y, *g = f + o_g, *z = f + o_z;
    float *post1 = f + o_p1, *comb1 = f + o_c1, *post2 = f + o_p2, *comb2 = f + o_c2, *w = f + o_w;
    uint32_t* ids = reinterpret_cast<uint32_t*>(f + o_ids);
    uint32_t* count = reinterpret_cast<uint32_t*>(f + o_n);
    // phase 1: hc_pre + attention norm per position, the batched attention,
    // hc_post, ffn hc_pre + norm per position (E/compute.rs:4679-4750)
    if (!L->hc_attn_fn || !L->hc_attn_scale || !L->hc_attn_base || !L->hc_ffn_fn || !L->hc_ffn_scale ||
        !L->hc_ffn_base)
        return WH_INVALID_ARGUMENT;
    if (hidden > WH_ROWPOST_MAX) return WH_UNSUPPORTED;
    // hc_pre's y and each norm in the launch that follows (the same values)
    const float* pre = nullptr;
    WH_TRY(hc_pre_launch(c, L->hc_attn_fn, L->hc_attn_scale, L->hc_attn_base, hc, hidden, L->sinkhorn_iters, L->hc_eps,
                         hidden_dev, y, post1, comb1, npos, false, &pre));
    MlaIn in{};
    in.x = hidden_dev;
    in.ld = hcd;
    in.norm = 1;
    in.w = L->attn_norm_bf16;
    in.pre = pre;
    in.hc = hc;
    in.hc_stride = hidden;
    WH_TRY(mla_decode_batch_impl(c, &L->attn, positions, npos, in, g, kv_cache_dev, kv_stride, kv_capacity, comp_dev,
                                 n_comp));
    WH_TRY(hc_post_launch(c, g, hidden_dev, post1, comb1, state, hc, hidden, npos));
    WH_TRY(hc_pre_launch(c, L->hc_ffn_fn, L->hc_ffn_scale, L->hc_ffn_base, hc, hidden, L->sinkhorn_iters, L->hc_eps,
                         state, y, post2, comb2, npos, false, &pre));
    {
        wh_rowpost_args a = rowpost_args(state, g, npos, hidden, hcd, hidden);
        a.norm = 1;
        a.w = L->ffn_norm_bf16;
        a.hc_pre = pre;
        a.hc = (uint32_t)hc;
        a.hc_stride = (uint32_t)hidden;
        WH_TRY(rowpost_launch(c, a));
    }
    // the router per position (E/server/generation.rs:2462-2480, each with
    // its own token for a hash layer), then the experts of the whole batch
    // on the device route lists
    WH_TRY(route_batch(c, L->layer_id, g, hidden, hidden, npos, slots, L->available_dev, L->n_available, L->route,
                       token_ids, ids, w, count));
    WH_TRY(wh_moe_batch_async(c, L->layer_id, ids, w, npos, slots, L->shared_layer, L->shared_expert, g, 0, z));
    return hc_post_launch(c, z, state, post2, comb2, hidden_dev, hc, hidden, npos);
}
