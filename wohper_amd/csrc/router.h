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
// values of its chain in a 128-column block as 16 contiguous bytes; x is
// staged so that the matching eight x values are contiguous too: column
// 128 b + 32 j + 16 h + o (o = 8 a + l) at float (16 b + o) * 8 + 2 j + h.
// 4096 columns: every weight block in flight at once and the x values of a
// block read four blocks ahead of its FMAs; wider rows stream the weights
// eight blocks ahead.  Returns the row's value in every thread of the row.
__device__ __forceinline__ uint32_t wh_router_xs_index(uint32_t c) {
    const uint32_t b = c >> 7, r = c & 127;
    return ((b << 4) | (r & 15)) * 8 + 2 * (r >> 5) + ((r >> 4) & 1);
}
// late(): loads of the caller's, issued right after the weight loads (an
// earlier load would be waited for before the first weight load issues).
template <class Late>
__device__ __forceinline__ float wh_router_gemv_rows(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                     uint32_t rows, uint32_t cols, float* xs, Late&& late) {
    const uint32_t L = threadIdx.x, q = L & 15;  // q = 8 a + l: the chain's column within a 16-column chunk
    const uint32_t row = blockIdx.x * 4 + (L >> 4);
    const uint32_t r = row < rows ? row : rows - 1;  // spare lanes repeat the last row
    const uint4* wp = reinterpret_cast<const uint4*>(w + (size_t)r * cols) + q;
    const uint32_t nb = cols / 128;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* xq = reinterpret_cast<const float4*>(xs) + 2 * q;  // block b at xq[32 b], xq[32 b + 1]
    // the four x values of float4 i go to four chains' slots, 8 floats apart
    auto store_x4 = [&](uint32_t i, float4 v) {
        const uint32_t k = wh_router_xs_index(4 * i);
        xs[k] = v.x;
        xs[k + 8] = v.y;
        xs[k + 16] = v.z;
        xs[k + 24] = v.w;
    };
    float acc = 0.0f;
    auto fma8 = [&](const uint4 w4, const float4 x0, const float4 x1) {
        acc = __builtin_fmaf(wh_bf16_lo(w4.x), x0.x, acc);
        acc = __builtin_fmaf(wh_bf16_hi(w4.x), x0.y, acc);
        acc = __builtin_fmaf(wh_bf16_lo(w4.y), x0.z, acc);
        acc = __builtin_fmaf(wh_bf16_hi(w4.y), x0.w, acc);
        acc = __builtin_fmaf(wh_bf16_lo(w4.z), x1.x, acc);
        acc = __builtin_fmaf(wh_bf16_hi(w4.z), x1.y, acc);
        acc = __builtin_fmaf(wh_bf16_lo(w4.w), x1.z, acc);
        acc = __builtin_fmaf(wh_bf16_hi(w4.w), x1.w, acc);
    };
    if (nb == 32) {
        // x (16-byte loads), then every weight block, then x into LDS: the
        // weights stream while x lands
        constexpr int kNb = 32, kX = 16, kPf = 4;
        float4 xv[kX];
#pragma unroll
        for (int k = 0; k < kX; ++k) xv[k] = x4[64 * k + L];
        uint4 all[kNb];
#pragma unroll
        for (int d = 0; d < kNb; ++d) all[d] = wp[16 * d];
        late();
        __builtin_amdgcn_sched_barrier(0);  // every load is issued before the first x store waits
#pragma unroll
        for (int k = 0; k < kX; ++k) store_x4(64 * k + L, xv[k]);
        __syncthreads();
        WH_TL(0, 1);
#ifdef WH_TIMELINE
        WH_TL_USE(all[kNb - 1].x);
        WH_TL(0, 2);
#endif
        float4 pf[kPf][2];
#pragma unroll
        for (int d = 0; d < kPf; ++d) {
            pf[d][0] = xq[32 * d];
            pf[d][1] = xq[32 * d + 1];
        }
        // the barriers keep each block's x reads kPf blocks ahead of its
        // FMAs (the scheduler would sink them next to their use)
#pragma unroll
        for (int d = 0; d < kNb; ++d) {
            const float4 x0 = pf[d % kPf][0], x1 = pf[d % kPf][1];
            if (d + kPf < kNb) {
                pf[d % kPf][0] = xq[32 * (d + kPf)];
                pf[d % kPf][1] = xq[32 * (d + kPf) + 1];
            }
            __builtin_amdgcn_sched_barrier(0);
            fma8(all[d], x0, x1);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        for (uint32_t i = L; i < cols / 4; i += 64) store_x4(i, x4[i]);
        constexpr int kDepth = 8;
        uint4 ring[kDepth];
#pragma unroll
        for (int d = 0; d < kDepth; ++d) ring[d] = (uint32_t)d < nb ? wp[16 * d] : make_uint4(0, 0, 0, 0);
        late();
        __syncthreads();
        for (uint32_t b0 = 0; b0 < nb; b0 += kDepth) {
#pragma unroll
            for (int d = 0; d < kDepth; ++d) {
                const uint32_t b = b0 + d;
                if (b < nb) {
                    const uint4 w4 = ring[d];
                    if (b + kDepth < nb) ring[d] = wp[16 * (b + kDepth)];
                    fma8(w4, xq[32 * b], xq[32 * b + 1]);
                }
            }
        }
    }
    // acc0 + acc1 of the lane (DPP row_ror:8 = lane ^ 8), then hsum256's
    // pairs (quad_perm lane ^ 1, lane ^ 2; then row_half_mirror pairs lane l
    // with 7 - l, which after the first two steps holds the same sum as
    // l ^ 4).  IEEE addition commutes, so both partners of a step hold the
    // same sum.
    float s = acc + wh_dpp_f<0x128>(acc);
    s = s + wh_dpp_f<0xB1>(s);
    s = s + wh_dpp_f<0x4E>(s);
    s = s + wh_dpp_f<0x141>(s);
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
    // k_router_bf16 only: every workgroup's 4 rows are published already in
    // selection order (rows % 4 == 0, rows <= 256, no available list, no
    // hash row); logits then holds [rows] u64 (score, key) and [rows] u32 ids
    uint32_t sorted;
    // k_router_bf16<true> with sorted: the last arriver also resolves the
    // selected routes against a layer's expert table into rs_out (the work
    // of k_moe_resolve, one launch fewer before the experts)
    wh_moe_dyn* rs_out;
    const wh_expert_ptrs* rs_table;
    uint32_t rs_table_n, rs_slots, rs_has_shared;
    uint32_t* rs_status;
    wh_expert_ptrs rs_shared;
};

// f32::total_cmp order as a signed key.
__device__ __forceinline__ int32_t wh_total_key(float f) {
    const int32_t k = (int32_t)__float_as_uint(f);
    return k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1);
}

// Wave-wide maximum of a signed / minimum of an unsigned 32-bit value,
// returned to every lane: DPP steps (quad xor 1 and 2, half-row and row
// mirrors, then the row broadcasts into rows 1, 3 and 2, 3) leave the result
// in lane 63.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ int32_t wh_dpp_i32(int32_t v) {
    // full row mask: every lane is written, no copy of the old value needed
    if constexpr (kRowMask == 0xf) return __builtin_amdgcn_mov_dpp(v, kCtrl, 0xf, 0xf, false);
    else return __builtin_amdgcn_update_dpp(v, v, kCtrl, kRowMask, 0xf, false);
}
__device__ __forceinline__ int32_t wh_wave_max_i32(int32_t v) {
    v = max(v, wh_dpp_i32<0xb1, 0xf>(v));
    v = max(v, wh_dpp_i32<0x4e, 0xf>(v));
    v = max(v, wh_dpp_i32<0x141, 0xf>(v));
    v = max(v, wh_dpp_i32<0x140, 0xf>(v));
    v = max(v, wh_dpp_i32<0x142, 0xa>(v));
    v = max(v, wh_dpp_i32<0x143, 0xc>(v));
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ uint32_t wh_wave_min_u32(uint32_t u) {
    int32_t v = (int32_t)u;
    v = (int32_t)min((uint32_t)v, (uint32_t)wh_dpp_i32<0xb1, 0xf>(v));
    v = (int32_t)min((uint32_t)v, (uint32_t)wh_dpp_i32<0x4e, 0xf>(v));
    v = (int32_t)min((uint32_t)v, (uint32_t)wh_dpp_i32<0x141, 0xf>(v));
    v = (int32_t)min((uint32_t)v, (uint32_t)wh_dpp_i32<0x140, 0xf>(v));
    v = (int32_t)min((uint32_t)v, (uint32_t)wh_dpp_i32<0x142, 0xa>(v));
    v = (int32_t)min((uint32_t)v, (uint32_t)wh_dpp_i32<0x143, 0xc>(v));
    return (uint32_t)__builtin_amdgcn_readlane(v, 63);
}

// Selection and weights by one wave (threads 0..63) from the scores in sc
// (LDS, sqrt-softplus already applied).  Round t of the stable descending
// sort takes the largest key, ties to the smallest candidate position: a
// wave maximum of the lanes' best keys, then a wave minimum of the positions
// holding it.  Lane i keeps the i-th selected id.
template <uint32_t kSlots>
__device__ __forceinline__ void wh_router_select_wave_n(const wh_router_sel& a, const float* sc, const float* sk,
                                                        uint32_t* sel, uint32_t& n_sel) {
    const uint32_t L = threadIdx.x & 63;
    uint32_t my_sel = 0, n = 0;
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
        n = min((uint32_t)__popcll(m), a.active);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
        if (L < n) my_sel = sel[L];
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
        // the lane's live candidates in selection order (larger key first,
        // then smaller position): an insertion sort of its slots
        int32_t qk[kSlots];
        uint32_t qp[kSlots];
        uint32_t qn = 0;
#pragma unroll
        for (uint32_t s = 0; s < kSlots; ++s) {
            // slots come in position order, so an equal key goes after
            const int32_t k = key[s];
            const uint32_t p = L + 64 * s;
            bool placed = !live[s];
#pragma unroll
            for (int i = (int)kSlots - 1; i >= 0; --i) {
                if (placed || (uint32_t)i > qn) continue;
                const bool shift = i > 0 && k > qk[i - 1];
                if (shift) {
                    qk[i] = qk[i - 1];
                    qp[i] = qp[i - 1];
                } else {
                    qk[i] = k;
                    qp[i] = p;
                    placed = true;
                }
            }
            qn += live[s] ? 1u : 0u;
        }
#ifdef WH_TIMELINE
        WH_TL_USE(qk[0]);
        WH_TL(0, 8);
#endif
        for (; n < a.active; ++n) {
            const bool has = qn > 0;
            if (__ballot(has) == 0) break;  // uniform: no candidate left
            const int32_t bk = has ? qk[0] : INT32_MIN;
            const int32_t mk = wh_wave_max_i32(bk);
            // one lane holding the maximum key: its head; several: the
            // smallest of their heads
            const uint64_t at = __ballot(has && bk == mk);
            const uint32_t mp = __popcll(at) == 1
                                    ? (uint32_t)__builtin_amdgcn_readlane((int)qp[0], (int)__ffsll((long long)at) - 1)
                                    : wh_wave_min_u32(has && bk == mk ? qp[0] : 0xffffffffu);
            if (has && qp[0] == mp) {  // the winner pops its head
#pragma unroll
                for (uint32_t i = 0; i + 1 < kSlots; ++i) {
                    qk[i] = qk[i + 1];
                    qp[i] = qp[i + 1];
                }
                --qn;
            }
            if (L == n) my_sel = mp;
        }
        if (a.avail && L < n) my_sel = a.avail[my_sel];
        WH_TL(0, 9);
    }
    // finalize_route_weights (E/compute.rs:2254-2268): the sum in route
    // order, then every lane its own weight
    const float v = L < n ? sc[my_sel] : 0.0f;
    float sum = 0.0f;
#pragma unroll 1
    for (uint32_t i = 0; i < n; ++i) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
    const bool norm = a.math != 0 && n > 0;
    const bool ok = sum > 0.0f && sum <= 3.4028235e38f;
    const float uniform = n ? a.route_scale / (float)n : 0.0f;
#ifdef WH_TIMELINE
    WH_TL_USE(sum);
    WH_TL(0, 10);
#endif
    if (L < n) {
        a.out_ids[L] = my_sel;
        a.out_scores[L] = !norm ? v : (ok ? v / sum * a.route_scale : uniform);
    }
    if (L == 0) {
        *a.out_count = n;
        n_sel = n;
    }
}

// Selection and weights when every workgroup of k_router_bf16 published its
// 4 candidates in selection order (key descending, then row ascending):
// lane L takes workgroup L's list, already sorted, with the scores beside
// the keys, so the last workgroup's wave loads one list per lane and goes
// straight to the rounds of wh_router_select_wave_n (the same order: the
// largest key, ties to the smallest row); the winner's lane hands its score
// to the selected slot's lane.
template <bool kResolve>
__device__ __forceinline__ void wh_router_select_sorted(const wh_router_sel& a) {
    const uint32_t L = threadIdx.x & 63, n_lists = a.rows / 4;
    const uint64_t* kv = (const uint64_t*)a.logits;
    const uint64_t* idp = (const uint64_t*)(a.logits + 2 * a.rows);
    int32_t qk[4];
    float qs[4];
    uint32_t qp[4], qn = 0;
    if (L < n_lists) {
        uint64_t d[4], e[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = __hip_atomic_load(kv + 4 * L + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 2; ++i) e[i] = __hip_atomic_load(idp + 2 * L + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qs[i] = __uint_as_float((uint32_t)d[i]);
            qk[i] = (int32_t)(uint32_t)(d[i] >> 32);
            qp[i] = (uint32_t)(e[i >> 1] >> (32 * (i & 1)));
        }
        qn = 4;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) qk[i] = INT32_MIN, qs[i] = 0.0f, qp[i] = 0xffffffffu;
    }
#ifdef WH_TIMELINE
    WH_TL_USE(qk[0]);
    WH_TL(0, 6);
    WH_TL(0, 8);
#endif
    uint32_t my_sel = 0, n = 0;
    float my_sc = 0.0f;
    for (; n < a.active; ++n) {
        const bool has = qn > 0;
        if (__ballot(has) == 0) break;  // uniform: no candidate left
        const int32_t bk = has ? qk[0] : INT32_MIN;
        const int32_t mk = wh_wave_max_i32(bk);
        const uint64_t at = __ballot(has && bk == mk);
        const uint32_t mp = __popcll(at) == 1
                                ? (uint32_t)__builtin_amdgcn_readlane((int)qp[0], (int)__ffsll((long long)at) - 1)
                                : wh_wave_min_u32(has && bk == mk ? qp[0] : 0xffffffffu);
        const bool win = has && bk == mk && qp[0] == mp;  // one lane: rows are distinct
        const int wl = (int)__ffsll((long long)__ballot(win)) - 1;
        const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qs[0]), wl));
        if (win) {  // the winner pops its head
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                qk[i] = qk[i + 1];
                qs[i] = qs[i + 1];
                qp[i] = qp[i + 1];
            }
            --qn;
        }
        if (L == n) {
            my_sel = mp;
            my_sc = ws;
        }
    }
    WH_TL(0, 9);
    // finalize_route_weights (E/compute.rs:2254-2268): the sum in route
    // order, then every lane its own weight
    const float v = L < n ? my_sc : 0.0f;
    float sum = 0.0f;
#pragma unroll 1
    for (uint32_t i = 0; i < n; ++i) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
    const bool norm = a.math != 0 && n > 0;
    const bool ok = sum > 0.0f && sum <= 3.4028235e38f;
    const float uniform = n ? a.route_scale / (float)n : 0.0f;
#ifdef WH_TIMELINE
    WH_TL_USE(sum);
    WH_TL(0, 10);
#endif
    const float wv = !norm ? v : (ok ? v / sum * a.route_scale : uniform);
    if (L < n) {
        a.out_ids[L] = my_sel;
        a.out_scores[L] = wv;
    }
    if (L == 0) *a.out_count = n;
    if (kResolve) {
        __shared__ wh_expert_ptrs got[64];
        const uint32_t cnt = n < a.rs_slots ? n : a.rs_slots;
        wh_moe_resolve_wave(L < cnt ? my_sel : 0u, L < cnt ? wv : 0.0f, cnt, a.rs_table, a.rs_table_n, a.rs_shared,
                            a.rs_has_shared, a.rs_slots, a.rs_out, a.rs_status, got);
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
// *counter is 0 at launch and left at 0.  grid.y > 1 routes several inputs
// at once: input z = blockIdx.y reads x + z * x_ld, publishes into
// a.logits + z * pub_ld, arrives on counter[z] and writes its ids and
// weights at z * active and its count at z.
// kResolve: with a.sorted, the route-list resolve in the last arriver
// (a single input).
template <bool kResolve>
__global__ void __launch_bounds__(64) k_router_bf16(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                    uint32_t cols, wh_router_sel a0, uint32_t* counter, uint32_t x_ld,
                                                    uint32_t pub_ld) {
    const uint32_t z = blockIdx.y;
    wh_router_sel a = a0;
    x += (size_t)z * x_ld;
    counter += z;
    a.logits += (size_t)z * pub_ld;
    a.out_ids += (size_t)z * a0.active;
    a.out_scores += (size_t)z * a0.active;
    a.out_count += z;
    extern __shared__ float xs[];
    __shared__ float sc[WH_ROUTER_MAX_ROWS], sk[WH_ROUTER_MAX_ROWS];
    __shared__ uint32_t sel[WH_ROUTER_MAX_ACTIVE];
    __shared__ uint32_t n_sel;
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 4);
    const bool writer = (threadIdx.x & 15) == 0 && row < a.rows;
    WH_TL(0, 0);
    float bias = 0.0f;
    uint64_t tv = 0;
    const float v = wh_router_gemv_rows(w, x, a.rows, cols, xs, [&]() {
        if (writer && a.math && a.bias) bias = a.bias[row];
        if (threadIdx.x < WH_EXP_TAB_LEN) tv = kExpTab[threadIdx.x];
    });
    // the expf table goes to LDS once the GEMV is done
    if (threadIdx.x < WH_EXP_TAB_LEN) exp_tab[threadIdx.x] = tv;
    __syncthreads();
    WH_TL(0, 3);
    if (a.sorted) {
        // the workgroup's 4 rows in selection order: writer j (lane 16 j)
        // takes rank = the rows ahead of it (a larger key, or an equal key
        // and a smaller row)
        const float score = a.math ? wh_sqrt_softplus(v, exp_tab) : v;
        const int32_t key = wh_total_key(a.math && a.bias ? score + bias : score);
        const uint32_t j = threadIdx.x >> 4;
        uint32_t rank = 0;
#pragma unroll
        for (uint32_t o = 0; o < 4; ++o) {
            const int32_t ko = __shfl(key, (int)(16 * o), 64);
            rank += (ko > key || (ko == key && o < j)) ? 1u : 0u;
        }
        if (writer) {
            const uint32_t at = blockIdx.x * 4 + rank;
            const uint64_t d = ((uint64_t)(uint32_t)key << 32) | __float_as_uint(score);
            __hip_atomic_store((uint64_t*)a.logits + at, d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store((uint32_t*)(a.logits + 2 * a.rows) + at, row, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (writer) {
        const float score = a.math ? wh_sqrt_softplus(v, exp_tab) : v;
        float* pub = const_cast<float*>(a.logits);
        wh_store_coherent(pub + row, score);
        wh_store_coherent(pub + a.rows + row, a.math && a.bias ? score + bias : score);
    }
    WH_TL(0, 4);
    wh_stores_done();
    uint32_t last = 0;
    if (threadIdx.x == 0) last = wh_arrive(counter) == gridDim.x - 1;
    last = __shfl(last, 0, 64);
    WH_TL(0, 5);
    if (!last) return;
    if (a.sorted) {
        wh_router_select_sorted<kResolve>(a);
        WH_TL(0, 7);
        if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // all published scores and keys are requested before the first LDS
    // store, so the wave waits for one round trip, not one per pass
    auto gather = [&](auto pass) {
        constexpr uint32_t kPass = decltype(pass)::value;
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
    };
    if (a.rows <= 256) gather(std::integral_constant<uint32_t, 4>());
    else gather(std::integral_constant<uint32_t, WH_ROUTER_MAX_ROWS / 64>());
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    WH_TL(0, 6);
    wh_router_select_wave(a, sc, sk, sel, n_sel);
    WH_TL(0, 7);
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
