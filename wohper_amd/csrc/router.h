// MoE router of a DeepSeek-V4 layer on the GPU: the gate GEMV, the
// sqrt-softplus scores, the biased top-k (or the hash layer's table row) and
// the final weights of route_experts_from_dense_block (E/compute.rs:2129-2268),
// bit-exact, so the routed experts can follow on the device without a host
// round trip.
//
// Gate GEMV: the x86 path of dot_bf16_row (dot_bf16_row_avx2,
// E/compute.rs:6116-6136) per row: AVX lane l of accumulator a (a = 0, 1)
// sums, fused, columns 16c + 8a + l over the 16-column chunks c; the row
// value is hsum256(acc0 + acc1) = ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)) plus a
// sequential unfused tail.  The fast kernel runs one AVX lane per thread,
// eight threads per row, on a resident layout where each 64-column block
// holds lane l's eight values (chunks 4b..4b+3, acc0 and acc1 interleaved)
// in 16 contiguous bytes.  FP8 gates use the FP8 GEMV kernels.
//
// Selection runs in one wave: sqrt-softplus of every row (E/compute.rs:
// 2238-2249, libm-exact: expf, log1pf, IEEE sqrt), then either the hash
// row's available ids in table order or, for the other layers, the stable
// descending sort of score + bias in f32 total order (Rust's total_cmp),
// done as `active` rounds of a wave-wide argmax that breaks ties by position
// in the available list.  The weights are finalize_route_weights
// (E/compute.rs:2254-2268): score / sum * route_scale with the sum taken in
// route order, or route_scale / n when the sum is not positive and finite.
#pragma once
#include "kernels.h"

#define WH_ROUTER_MAX_ROWS 1024u   // gate rows (experts) one selection wave covers
#define WH_ROUTER_MAX_ACTIVE 64u   // experts per token
#define WH_ROUTER_MAX_HASH 64u     // ids per tid2eid row

// IEEE round-to-nearest square root of a finite x > 0 (Rust's f32::sqrt).
// The device's single-precision root is not correctly rounded, so: a
// double-precision root rounded to float, then the exact midpoint test with
// each neighbour.  A midpoint of two adjacent floats has 25 significant bits,
// so its square is exact in double and never equals the 24-bit x.
__device__ __forceinline__ float wh_sqrt_rn(float x) {
    const double xd = x;
    float s = (float)__builtin_sqrt(xd);
    const float up = __uint_as_float(__float_as_uint(s) + 1u);
    const double mu = 0.5 * ((double)s + (double)up);
    if (mu * mu < xd) return up;
    const float dn = __uint_as_float(__float_as_uint(s) - 1u);
    const double md = 0.5 * ((double)s + (double)dn);
    if (md * md > xd) return dn;
    return s;
}

// sqrt_softplus (E/compute.rs:2238-2249): Rust's exp / ln_1p are glibc's
// expf / log1pf, reproduced bit for bit; max(NaN, 0) is 0.
__device__ __forceinline__ float wh_sqrt_softplus(float v) {
    if (v != v) return 0.0f;
    float sp;
    if (v > 20.0f) sp = v;
    else if (v < -20.0f) sp = wh_expf_glibc(v, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
    else sp = wh_log1pf(wh_expf_glibc(v, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT));
    const float m = fmaxf(sp, 0.0f);
    return (m > 0.0f && m <= 3.4028235e38f) ? wh_sqrt_rn(m) : m;  // sqrt(+0) = +0, sqrt(inf) = inf
}

__device__ __forceinline__ float wh_bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float wh_bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Fast bf16 gate GEMV, cols % 64 == 0: grid ceil(rows / 8), 64 threads,
// cols floats of dynamic LDS.  Thread L runs AVX lane L % 8 of row
// 8 * blockIdx.x + L / 8.
__global__ void __launch_bounds__(64) k_router_gemv_bf16(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                         uint32_t rows, uint32_t cols, float* __restrict__ logits) {
    extern __shared__ float xs[];
    for (uint32_t i = threadIdx.x; i < cols; i += 64) xs[i] = x[i];
    __syncthreads();
    const uint32_t L = threadIdx.x, l = L & 7;
    const uint32_t row = blockIdx.x * 8 + (L >> 3);
    const uint32_t r = row < rows ? row : rows - 1;  // spare lanes repeat the last row
    const uint4* wp = reinterpret_cast<const uint4*>(w + (size_t)r * cols) + l;
    float a0 = 0.0f, a1 = 0.0f;
    const uint32_t blocks = cols / 64;
#pragma unroll 4
    for (uint32_t b = 0; b < blocks; ++b) {
        const uint4 q = wp[8 * b];
        const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c0 = 64 * b + 16 * j + l;
            a0 = __builtin_fmaf(wh_bf16_lo(v[j]), xs[c0], a0);
            a1 = __builtin_fmaf(wh_bf16_hi(v[j]), xs[c0 + 8], a1);
        }
    }
    // hsum256(acc0 + acc1): the xor partners add in the reference's pairs
    // (IEEE addition commutes, so both partners hold the same sum)
    float s = a0 + a1;
    s = s + __shfl_xor(s, 1, 64);
    s = s + __shfl_xor(s, 2, 64);
    s = s + __shfl_xor(s, 4, 64);
    if (l == 0 && row < rows) logits[row] = s + 0.0f;  // + the (empty) tail
}

// Any shape: one thread per row over row-major bf16, the sixteen AVX
// accumulators in registers.
__global__ void __launch_bounds__(64) k_router_gemv_bf16_generic(const uint16_t* __restrict__ w,
                                                                 const float* __restrict__ x, uint32_t rows,
                                                                 uint32_t cols, float* __restrict__ logits) {
    const uint32_t row = blockIdx.x * 64 + threadIdx.x;
    if (row >= rows) return;
    const uint16_t* wr = w + (size_t)row * cols;
    float acc[2][8];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[a][l] = 0.0f;
    const uint32_t chunks = cols / 16;
    for (uint32_t c = 0; c < chunks; ++c)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const uint32_t i = 16 * c + 8 * a + l;
                acc[a][l] = __builtin_fmaf(__uint_as_float((uint32_t)wr[i] << 16), x[i], acc[a][l]);
            }
    float s[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) s[l] = acc[0][l] + acc[1][l];
    const float h = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    float tail = 0.0f;
    for (uint32_t i = chunks * 16; i < cols; ++i) {
        const float p = __uint_as_float((uint32_t)wr[i] << 16) * x[i];
        tail = tail + p;
    }
    logits[row] = h + tail;
}

struct wh_router_sel {
    const float* logits;     // gate outputs [rows]
    uint32_t rows;
    const float* bias;       // selection bias [rows] (sqrt-softplus math only), or null
    const uint32_t* avail;   // available expert ids in order, or null for 0..rows-1
    uint32_t n_avail;
    uint32_t active;         // experts to keep (<= WH_ROUTER_MAX_ACTIVE)
    uint32_t math;           // 0: raw logits, 1: DeepSeek-V4 sqrt-softplus
    float route_scale;
    uint32_t n_hash;         // > 0: hash layer, the token's tid2eid row below
    uint32_t hash[WH_ROUTER_MAX_HASH];
    uint32_t* out_ids;       // [active]
    float* out_scores;       // [active]
    uint32_t* out_count;
};

// f32::total_cmp order as a signed key.
__device__ __forceinline__ int32_t wh_total_key(float f) {
    const int32_t k = (int32_t)__float_as_uint(f);
    return k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1);
}

// One wave: scores, selection, weights.  rows <= WH_ROUTER_MAX_ROWS and the
// candidate count <= WH_ROUTER_MAX_ROWS (checked by the host).
__global__ void __launch_bounds__(64) k_router_select(wh_router_sel a) {
    constexpr uint32_t kSlots = WH_ROUTER_MAX_ROWS / 64;
    __shared__ float sc[WH_ROUTER_MAX_ROWS];
    __shared__ uint32_t sel[WH_ROUTER_MAX_ACTIVE];
    __shared__ uint32_t n_sel;
    const uint32_t L = threadIdx.x;
    for (uint32_t i = L; i < a.rows; i += 64) {
        const float v = a.logits[i];
        sc[i] = a.math ? wh_sqrt_softplus(v) : v;
    }
    __syncthreads();
    if (a.n_hash) {
        // hash layer (E/compute.rs:2190-2206): the row's ids that are
        // available and have a score, in table order
        bool ok = false;
        uint32_t id = 0;
        if (L < a.n_hash) {
            // uniform indices keep the argument array out of private memory
#pragma unroll
            for (uint32_t j = 0; j < WH_ROUTER_MAX_HASH; ++j)
                if (j == L) id = a.hash[j];
            ok = id < a.rows;
            if (ok && a.avail) {
                bool found = false;
                for (uint32_t j = 0; j < a.n_avail; ++j) found |= a.avail[j] == id;
                ok = found;
            }
        }
        const uint64_t m = __ballot(ok);
        const uint32_t pos = (uint32_t)__popcll(m & ((1ull << L) - 1ull));
        if (ok && pos < a.active) sel[pos] = id;
        if (L == 0) n_sel = min((uint32_t)__popcll(m), a.active);
    } else {
        // the available experts by score (+ bias), descending, stable
        const uint32_t cnt = a.avail ? a.n_avail : a.rows;
        int32_t key[kSlots];
        bool live[kSlots];
#pragma unroll
        for (uint32_t s = 0; s < kSlots; ++s) {
            const uint32_t p = L + 64 * s;
            const uint32_t id = p < cnt ? (a.avail ? a.avail[p] : p) : 0u;
            live[s] = p < cnt && id < a.rows;
            float v = live[s] ? sc[id] : 0.0f;
            if (a.math && a.bias && live[s]) v = v + a.bias[id];
            key[s] = wh_total_key(v);
        }
        uint32_t t = 0;
        for (; t < a.active; ++t) {
            int32_t bk = INT32_MIN;
            uint32_t bp = 0xffffffffu;
#pragma unroll
            for (uint32_t s = 0; s < kSlots; ++s)
                if (live[s] && (bp == 0xffffffffu || key[s] > bk)) {  // slots ascend in position
                    bk = key[s];
                    bp = L + 64 * s;
                }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const int32_t ok = __shfl_xor(bk, off, 64);
                const uint32_t op = __shfl_xor(bp, off, 64);
                if (op != 0xffffffffu && (bp == 0xffffffffu || ok > bk || (ok == bk && op < bp))) {
                    bk = ok;
                    bp = op;
                }
            }
            if (bp == 0xffffffffu) break;  // uniform: every lane saw the same winner
#pragma unroll
            for (uint32_t s = 0; s < kSlots; ++s)
                if (L + 64 * s == bp) live[s] = false;
            if (L == 0) sel[t] = a.avail ? a.avail[bp] : bp;
        }
        if (L == 0) n_sel = t;
    }
    __syncthreads();
    if (L == 0) {
        const uint32_t n = n_sel;
        float sum = 0.0f;
        for (uint32_t i = 0; i < n; ++i) sum = sum + sc[sel[i]];
        const bool norm = a.math != 0 && n > 0;
        const bool ok = sum > 0.0f && sum <= 3.4028235e38f;
        const float uniform = n ? a.route_scale / (float)n : 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
            const float v = sc[sel[i]];
            a.out_ids[i] = sel[i];
            a.out_scores[i] = !norm ? v : (ok ? v / sum * a.route_scale : uniform);
        }
        *a.out_count = n;
    }
}

// Test support: fn 4 sqrt_softplus(x), fn 5 log1pf(x) (x >= 0), fn 6 expf(x)
// over the whole float line.
__global__ void k_debug_eval_router(int fn, const float* __restrict__ in, float* __restrict__ out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = in[i];
    out[i] = fn == 4 ? wh_sqrt_softplus(x)
                     : fn == 5 ? wh_log1pf(x) : wh_expf_glibc(x, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
}
