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
// Selection runs in one wave after 256 threads took the sqrt-softplus of
// every row (E/compute.rs:
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
__device__ __forceinline__ float wh_sqrt_softplus(float v, const uint64_t* exp_tab) {
    if (v != v) return 0.0f;
    float sp;
    if (v > 20.0f) sp = v;
    else if (v < -20.0f) sp = wh_expf_glibc(v, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT);
    else sp = wh_log1pf(wh_expf_glibc(v, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT));
    const float m = fmaxf(sp, 0.0f);
    return (m > 0.0f && m <= 3.4028235e38f) ? wh_sqrt_rn(m) : m;  // sqrt(+0) = +0, sqrt(inf) = inf
}

__device__ __forceinline__ float wh_bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float wh_bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Fast bf16 gate GEMV body, cols % 128 == 0, one 64-thread workgroup per 4
// rows, x staged in LDS (cols floats).  Thread L runs one AVX accumulator
// chain: accumulator a = (L / 8) % 2, lane l = L % 8 of row
// 4 * blockIdx.x + L / 16.  The resident layout gives the thread the eight
// values of its chain in a 128-column block as 16 contiguous bytes; up to 32
// blocks (4096 columns) are loaded at once, wider rows stream the rest
// eight blocks ahead.  Returns the row's value in every thread of the row.
__device__ __forceinline__ float wh_router_gemv_rows(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                     uint32_t rows, uint32_t cols, float* xs) {
    constexpr int kAll = 32, kDepth = 8;
    const uint32_t L = threadIdx.x, q = L & 15, off = 8 * (q >> 3) + (q & 7);  // column within a chunk
    const uint32_t row = blockIdx.x * 4 + (L >> 4);
    const uint32_t r = row < rows ? row : rows - 1;  // spare lanes repeat the last row
    const uint4* wp = reinterpret_cast<const uint4*>(w + (size_t)r * cols) + q;
    const uint32_t nb = cols / 128;
    // x first (16-byte loads, all in flight), then the weight ring
    const float4* x4 = reinterpret_cast<const float4*>(x);
    constexpr int kX = 16;  // float4 per thread per pass: 4096 columns in one pass
    auto stage_x = [&](uint32_t base, float4 (&xv)[kX]) {
#pragma unroll
        for (int k = 0; k < kX; ++k) {
            const uint32_t i = base + 64 * k + L;
            xv[k] = i < cols / 4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_x = [&](uint32_t base, const float4 (&xv)[kX]) {
#pragma unroll
        for (int k = 0; k < kX; ++k) {
            const uint32_t i = base + 64 * k + L;
            if (i < cols / 4) reinterpret_cast<float4*>(xs)[i] = xv[k];
        }
    };
    float acc = 0.0f;
    auto fma8 = [&](const uint4 q4, uint32_t b) {
        const uint32_t v[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = 128 * b + 32 * j + off;  // chunks 2j and 2j + 1
            acc = __builtin_fmaf(wh_bf16_lo(v[j]), xs[c], acc);
            acc = __builtin_fmaf(wh_bf16_hi(v[j]), xs[c + 16], acc);
        }
    };
    if (nb <= (uint32_t)kAll) {
        // x, then every weight block, then wait for x only: the weights
        // stream while x lands in LDS
        float4 xv[kX];
        stage_x(0, xv);
        uint4 all[kAll];
#pragma unroll
        for (int d = 0; d < kAll; ++d) all[d] = d < (int)nb ? wp[16 * d] : make_uint4(0, 0, 0, 0);
        store_x(0, xv);
        __syncthreads();
#pragma unroll
        for (int d = 0; d < kAll; ++d)
            if (d < (int)nb) fma8(all[d], d);
        goto reduce;
    }
    {
    for (uint32_t base = 0; base < cols / 4; base += 64 * kX) {
        float4 xv[kX];
        stage_x(base, xv);
        store_x(base, xv);
    }
    uint4 ring[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) ring[d] = wp[16 * d];
    __syncthreads();
    for (uint32_t b0 = 0; b0 < nb; b0 += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const uint32_t b = b0 + d;
            if (b < nb) {
                const uint4 q4 = ring[d];
                if (b + kDepth < nb) ring[d] = wp[16 * (b + kDepth)];
                fma8(q4, b);
            }
        }
    }
    }
reduce:
    // acc0 + acc1 of the lane, then hsum256's pairs (IEEE addition commutes,
    // so both partners of each xor step hold the same sum)
    float s = acc + __shfl_xor(acc, 8, 64);
    s = s + __shfl_xor(s, 1, 64);
    s = s + __shfl_xor(s, 2, 64);
    s = s + __shfl_xor(s, 4, 64);
    return s + 0.0f;  // + the (empty) tail
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

// Wave-wide maximum of a 64-bit value, returned to every lane: DPP steps
// (quad xor 1 and 2, half-row and row mirrors, the row broadcasts) leave the
// maximum in lane 63.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t wh_dpp_max_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, kCtrl, kRowMask, 0xf, false);
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, kCtrl, kRowMask, 0xf, false);
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    return o > v ? o : v;
}
__device__ __forceinline__ uint64_t wh_wave_max_u64(uint64_t v) {
    v = wh_dpp_max_u64<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = wh_dpp_max_u64<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = wh_dpp_max_u64<0x141, 0xf>(v);  // row_half_mirror
    v = wh_dpp_max_u64<0x140, 0xf>(v);  // row_mirror
    v = wh_dpp_max_u64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = wh_dpp_max_u64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// f32::total_cmp order as a signed key.
__device__ __forceinline__ int32_t wh_total_key(float f) {
    const int32_t k = (int32_t)__float_as_uint(f);
    return k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1);
}

// Selection and weights by one wave (threads 0..63) from the scores in sc
// (LDS, sqrt-softplus already applied).
template <uint32_t kSlots>
__device__ __forceinline__ void wh_router_select_wave_n(const wh_router_sel& a, const float* sc, const float* sk,
                                                        uint32_t* sel, uint32_t& n_sel) {
    const uint32_t L = threadIdx.x & 63;
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
            if (sk) v = live[s] ? sk[id] : 0.0f;  // score + bias, summed by the row's workgroup
            else if (a.math && a.bias && live[s]) v = v + a.bias[id];
            key[s] = wh_total_key(v);
        }
        uint32_t t = 0;
        for (; t < a.active; ++t) {
            // the lane's best: larger key, then smaller position; packed so
            // that the unsigned maximum picks the winner (0: none)
            uint64_t best = 0;
#pragma unroll
            for (uint32_t s = 0; s < kSlots; ++s) {
                const uint64_t p = live[s] ? (((uint64_t)((uint32_t)key[s] ^ 0x80000000u) << 32) |
                                              (0xffffffffu - (L + 64 * s)))
                                           : 0ull;
                best = p > best ? p : best;
            }
            const uint64_t win = wh_wave_max_u64(best);
            if (win == 0) break;  // uniform
            const uint32_t bp = 0xffffffffu - (uint32_t)win;
#pragma unroll
            for (uint32_t s = 0; s < kSlots; ++s)
                if (L + 64 * s == bp) live[s] = false;
            if (L == 0) sel[t] = a.avail ? a.avail[bp] : bp;
        }
        if (L == 0) n_sel = t;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
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

// kSlots candidates per lane: 4 up to 256 candidates, else 16.  sk: the
// selection keys (score + bias) when precomputed, else null.
__device__ __forceinline__ void wh_router_select_wave(const wh_router_sel& a, const float* sc, const float* sk,
                                                      uint32_t* sel, uint32_t& n_sel) {
    const uint32_t cnt = a.avail ? a.n_avail : a.rows;
    if (cnt <= 256) wh_router_select_wave_n<4>(a, sc, sk, sel, n_sel);
    else wh_router_select_wave_n<WH_ROUTER_MAX_ROWS / 64>(a, sc, sk, sel, n_sel);
}

// 256 threads: the scores, then wave 0 selects and weighs.  rows <=
// WH_ROUTER_MAX_ROWS and the candidate count <= WH_ROUTER_MAX_ROWS (checked
// by the host).  Used after the FP8 gate GEMV.
__global__ void __launch_bounds__(256) k_router_select(wh_router_sel a) {
    __shared__ float sc[WH_ROUTER_MAX_ROWS];
    __shared__ uint32_t sel[WH_ROUTER_MAX_ACTIVE];
    __shared__ uint32_t n_sel;
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    if (threadIdx.x < WH_EXP_TAB_LEN) exp_tab[threadIdx.x] = kExpTab[threadIdx.x];
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < a.rows; i += 256) {
        const float v = a.logits[i];
        sc[i] = a.math ? wh_sqrt_softplus(v, exp_tab) : v;
    }
    __syncthreads();
    if (threadIdx.x < 64) wh_router_select_wave(a, sc, nullptr, sel, n_sel);
}

// The bf16 router in one launch: grid ceil(rows / 4), 64 threads, cols
// floats of dynamic LDS.  Each workgroup computes four gate rows, their
// scores and selection keys (score + bias) and publishes them (coherent
// stores into a.logits [2 * rows]); the last workgroup to arrive selects.
// *counter is 0 at launch and left at 0.
__global__ void __launch_bounds__(64) k_router_bf16(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                    uint32_t cols, wh_router_sel a, uint32_t* counter) {
    extern __shared__ float xs[];
    __shared__ float sc[WH_ROUTER_MAX_ROWS], sk[WH_ROUTER_MAX_ROWS];
    __shared__ uint32_t sel[WH_ROUTER_MAX_ACTIVE];
    __shared__ uint32_t n_sel;
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 4);
    const bool writer = (threadIdx.x & 15) == 0 && row < a.rows;
    const float bias = writer && a.math && a.bias ? a.bias[row] : 0.0f;  // loaded before the weights
    const uint64_t tv = threadIdx.x < WH_EXP_TAB_LEN ? kExpTab[threadIdx.x] : 0ull;
    if (threadIdx.x < WH_EXP_TAB_LEN) exp_tab[threadIdx.x] = tv;  // ordered before the GEMV's barrier
    const float v = wh_router_gemv_rows(w, x, a.rows, cols, xs);
    if (writer) {
        const float score = a.math ? wh_sqrt_softplus(v, exp_tab) : v;
        float* pub = const_cast<float*>(a.logits);
        wh_store_coherent(pub + row, score);
        wh_store_coherent(pub + a.rows + row, a.math && a.bias ? score + bias : score);
    }
    wh_stores_done();
    uint32_t last = 0;
    if (threadIdx.x == 0) last = wh_arrive(counter) == gridDim.x - 1;
    last = __shfl(last, 0, 64);
    if (!last) return;
    // all published scores and keys are requested before the first LDS
    // store, so the wave waits for one round trip, not one per pass
    constexpr uint32_t kPass = WH_ROUTER_MAX_ROWS / 64;
    float rs[kPass], rk[kPass];
#pragma unroll
    for (uint32_t k = 0; k < kPass; ++k) {
        const uint32_t i = threadIdx.x + 64 * k;
        if (i < a.rows) {
            rs[k] = wh_load_coherent(a.logits + i);
            rk[k] = wh_load_coherent(a.logits + a.rows + i);
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < kPass; ++k) {
        const uint32_t i = threadIdx.x + 64 * k;
        if (i < a.rows) {
            sc[i] = rs[k];
            sk[i] = rk[k];
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    wh_router_select_wave(a, sc, sk, sel, n_sel);
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Test support: fn 4 sqrt_softplus(x), fn 5 log1pf(x) (x >= 0), fn 6 expf(x)
// over the whole float line.
__global__ void k_debug_eval_router(int fn, const float* __restrict__ in, float* __restrict__ out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = in[i];
    out[i] = fn == 4 ? wh_sqrt_softplus(x, kExpTab)
                     : fn == 5 ? wh_log1pf(x) : wh_expf_glibc(x, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
}
