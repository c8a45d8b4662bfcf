// Ragged batched routed experts on gfx950.
//
// The expert-major batch path of the reference: per-position weights and the
// union of selected experts (E/server/generation.rs:2487-2506), then for each
// expert in ascending id and each of its positions acc_p += y * w
// (accumulate_expert_for_positions, E/compute.rs:1779-1810), and with a
// shared expert out_p = shared(x_p) + acc_p (E/compute.rs:1838-1852).
//
// Launch sequence (one stream):
//   k_moe_batch_pack     workgroup 0: weights, the per-expert token lists
//                        (counts, offsets, placement), the used experts in
//                        ascending id, their work order, each position's
//                        accumulation order; the others: act-quant (block
//                        64) of every position's input
//   k_moe_batch_mx       (exact numerics off) persistent MFMA kernel of the
//                        MFMA experts' gate and up matvecs (moe_bmx.h)
//   k_moe_batch_gateup   persistent: (expert, row tile) items from a queue,
//                        gate and up matvecs of every slot (after
//                        k_moe_batch_mx: the exact experts only)
//   k_moe_batch_swiglu_quant  SwiGLU of every slot and its act-quant
//   k_moe_batch_mx       down of the MFMA experts
//   k_moe_batch_down     persistent, as gate/up
//   k_moe_batch_accumulate
// Experts with at least `mfma_min` tokens take the MFMA items (block-scaled
// FP8 MFMA over the whole token group, fp32 accumulation: results within
// rounding of the reference order); the others take the exact lane-chain
// items, bit-identical to the reference's AVX2 kernel.
#pragma once
#include "kernels.h"

#define WH_BATCH_MAX_TABLE 1024u   // expert ids per layer
#define WH_BATCH_MAX_ASSIGN 4096u  // slots per pack
#define WH_BATCH_MAX_TOPK 16u

typedef int wh_v8i __attribute__((ext_vector_type(8)));
typedef float wh_v4f __attribute__((ext_vector_type(4)));

// A virtual expert of the MFMA kernels (moe_bmx.h): one MFMA expert's
// slots slot0 .. slot0 + count - 1 (count <= 16) and its matrices.
struct wh_bmx_vt {
    const uint8_t *w1, *s1, *w3, *s3, *w2, *s2;
    uint32_t slot0, count;
};

struct wh_batch_args {
    const wh_expert_ptrs* table;   // the layer's experts by id (null w1 = not resident)
    uint32_t n_table;              // valid ids are < n_table
    const uint32_t* route_ids;     // [npos][topk]
    const float* route_scores;     // [npos][topk]
    uint32_t npos, topk, hidden, inter;
    uint32_t has_shared;           // the shared expert runs on every position
    wh_expert_ptrs shared;         // ... under the id n_table
    uint32_t mfma_min;             // experts with this many slots take MFMA items (0: never)
    uint32_t mfma_external;        // the MFMA experts run in k_moe_batch_mx (moe_bmx.h), not here
    uint32_t mx_fallback;          // every used expert is an MFMA expert and no exact-item kernel
                                   // is launched: after an inf or NaN input k_moe_batch_mx's
                                   // gate/up computes them in fp32
    const void* x;                 // [npos][hidden], f32 or bf16
    uint32_t x_is_bf16;
    // assignments: i = p * topk + k for the routes, A + p for the shared
    // expert (A = npos * topk); S = A + has_shared * npos slots
    float* wgt;                    // [A] per position: its route weights, in acc_order's order
    uint32_t* sorted;              // [S] assignments grouped by expert id: the slots
    uint32_t* uexp;                // [S] used expert ids, ascending
    uint32_t* uoff;                // [S + 1] their slot ranges
    uint32_t* uorder;              // [S] used-expert indices, most slots first
    uint32_t* acc_order;           // [A] per position: its route slots by ascending expert id
    uint32_t* meta;                // [0] used experts, [1] routes valid, [2]/[3] work queues
                                   // of gate/up and down, [4] experts on MFMA items, [6] an
                                   // input block held an inf or NaN (set by the act-quant
                                   // of x; then no expert runs on MFMA items, or with
                                   // mx_fallback the gate/up ones run in fp32; the
                                   // accumulate clears it), [7] virtual experts
    wh_bmx_vt* vtab;               // [S] the MFMA experts' virtual experts, in work order
    uint32_t* pos;                 // [S] position of each slot
    float* xq;                     // [npos][hidden] act-quantized inputs (column order)
    uint8_t* xq8;                  // [npos][hidden] their E4M3 codes, MFMA group order
    uint8_t* xs8;                  // [npos][hidden / 32] E8M0 scale bytes (x 1/8)
    float* g;                      // [S][inter] gate matvec (w1) by slot
    float* u;                      // [S][inter] up matvec (w3) by slot
    float* hq;                     // [S][inter] act-quantized
    uint8_t* hq8;                  // [S][inter] codes
    uint8_t* hs8;                  // [S][inter / 32] scale bytes
    float* y;                      // [S][hidden] expert outputs by slot
    float* out;                    // [npos][hidden]
    uint32_t* status;
};

__device__ __forceinline__ uint32_t wh_slot_pos(const wh_batch_args& a, uint32_t i) {
    const uint32_t A = a.npos * a.topk;
    return i < A ? i / a.topk : i - A;
}
__device__ __forceinline__ wh_expert_ptrs wh_batch_expert(const wh_batch_args& a, uint32_t id) {
    return id == a.n_table ? a.shared : a.table[id];
}

// ------------------------------------------------------------------ packing
// Exclusive prefix sum over the 256 threads of a workgroup (wave scans, then
// the four wave totals); `tot` is 4 words of LDS.  Returns the thread's
// exclusive prefix; *total receives the sum.
__device__ __forceinline__ uint32_t wh_wg_exclusive_scan(uint32_t v, uint32_t* tot, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
    }
    if (lane == 63) tot[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t w = 0; w < 4; ++w) {
        before += w < wave ? tot[w] : 0u;
        all += tot[w];
    }
    *total = all;
    __syncthreads();  // tot may be reused
    return before + incl - v;
}

// Act-quant (block 64) of rows of `n` values, 16 values per thread (a quad
// of threads holds one 64-block; E/compute.rs:2504-2521): block `blk` of 256
// threads of rows * n / 4096.  Writes the values in column order, their E4M3
// codes in MFMA group order (per 32-col group, byte 4c + k holds column
// c + 8k) and one E8M0 byte per group: the block scale divided by 8, which
// takes the x8 of the FP4 integer LUT values.  Non-finite inputs follow the
// reference (wh_xq_quant16); a block that held one sets *nonfinite, and the
// gate/up and down kernels then run every expert on the exact items: -480 (a
// NaN's code) and an infinite scale have no E4M3 / E8M0 encoding.  `thr` is
// 256 words of LDS.
__device__ __forceinline__ void wh_batch_quant_rows(const void* __restrict__ src, uint32_t src_bf16, uint32_t rows,
                                                    uint32_t n, float* __restrict__ q32, uint8_t* __restrict__ q8,
                                                    uint8_t* __restrict__ s8, uint32_t* nonfinite, uint32_t blk,
                                                    uint32_t* thr) {
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_thr_stage_store(ts, thr);
    __syncthreads();
    const uint32_t per_row = n / 16;
    const uint32_t i = blk * 256 + threadIdx.x;
    const uint32_t r = i / per_row, t = i - r * per_row;
    const bool on = r < rows;
    const bool bf16 = src_bf16 != 0;
    const size_t base = (size_t)(on ? r : 0) * n;
    const void* row = bf16 ? (const void*)((const uint16_t*)src + base) : (const void*)((const float*)src + base);
    wh_xq_stage st;
    wh_xq_stage_load(st, row, bf16, on ? n : 0u, t);
    float q[16], sc = 1.0f;
    bool bad = false;
    if (!wh_xq_quant16(st, bf16, thr, q, sc, &bad)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) q[j] = 0.0f;  // rows past the end: the DPP partner below still reads
    }
    // codes: column c + 8k of the group sits at byte 4c + k; this thread
    // holds k = 2h + (j >> 3) for c = j & 7 (h = which half of the group)
    const uint32_t h = t & 1;
    uint32_t pair[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
        pair[c] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[c], q[c + 8], 0, false) & 0xffffu;
    uint32_t dw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t send = h ? pair[j] : pair[4 + j];
        const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xb1, 0xf, 0xf, false);  // lane ^ 1
        dw[j] = h ? (recv | (pair[4 + j] << 16)) : (pair[j] | (recv << 16));
    }
    if (!on) return;
    if (bad) atomicOr(nonfinite, 1u);
    float4* d32 = (float4*)(q32 + base + 16 * t);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        d32[j] = make_float4(q[4 * j] * sc, q[4 * j + 1] * sc, q[4 * j + 2] * sc, q[4 * j + 3] * sc);
    const uint32_t g = t >> 1;  // 32-col group of the row
    *(uint4*)(q8 + base + 32 * g + 16 * h) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    // sc = 2^k: E8M0 byte 127 + k - 3 is its biased exponent - 3 (0xFF for an
    // infinite scale, never read: such a batch runs no MFMA item)
    const uint32_t be = (__float_as_uint(sc) >> 23) & 0xffu;
    if (!h) s8[(size_t)r * (n / 32) + g] = (uint8_t)(be == 0xffu ? 0xffu : be - 3u);
}

// Workgroup 0 (256 threads; S <= 4096 slots, n_table < 1024) packs; the
// others (npos * hidden / 4096 of them) act-quantize x.  An expert's slots
// come in no particular order (each slot is computed on its own); the
// accumulation order of a position is fixed by acc_order alone.  The split
// into MFMA and exact experts does not wait for the act-quant: when an
// input block held an inf or NaN, the consumers take every expert as exact.
__global__ void __launch_bounds__(256) k_moe_batch_pack(wh_batch_args a) {
    __shared__ uint32_t ids[WH_BATCH_MAX_ASSIGN];
    __shared__ uint32_t slot_of[WH_BATCH_MAX_ASSIGN];
    __shared__ float wsh[WH_BATCH_MAX_ASSIGN];  // route weights in route order until they are permuted
    __shared__ uint32_t cnt[WH_BATCH_MAX_TABLE], off[WH_BATCH_MAX_TABLE];
    __shared__ __align__(16) uint32_t ucnt[WH_BATCH_MAX_TABLE];
    __shared__ uint32_t uoffl[WH_BATCH_MAX_TABLE], uexpl[WH_BATCH_MAX_TABLE], uordl[WH_BATCH_MAX_TABLE];
    __shared__ uint32_t vst[WH_BATCH_MAX_TABLE];  // per work-order position: its virtual experts, then their start
    __shared__ uint32_t tot[4];
    __shared__ uint32_t bad, n_mfma, mfma_min;
    if (blockIdx.x != 0) {  // the other workgroups act-quantize x meanwhile
        wh_batch_quant_rows(a.x, a.x_is_bf16, a.npos, a.hidden, a.xq, a.xq8, a.xs8, a.meta + 6, blockIdx.x - 1, ids);
        return;
    }
    const uint32_t A = a.npos * a.topk, S = A + a.has_shared * a.npos, tid = threadIdx.x;
    const uint32_t n_ids = a.n_table + a.has_shared;  // the shared expert is id n_table
    if (tid == 0) {
        bad = 0;
        n_mfma = 0;
        mfma_min = a.mfma_min;
    }
    for (uint32_t e = tid; e < n_ids; e += 256) cnt[e] = 0;
    // ids, checked against the table
    for (uint32_t i = tid; i < S; i += 256) {
        uint32_t e = a.n_table;
        if (i < A) {
            e = a.route_ids[i];
            if (e >= a.n_table || a.table[e].w1 == nullptr) {
                bad = 1;
                e = 0;
            }
        }
        ids[i] = e;
    }
    // per-position weights: score / sum, or 1 / len when the sequential sum
    // is not finite and positive or a score is not finite
    // (E/server/generation.rs:2495-2503)
    for (uint32_t p = tid; p < a.npos; p += 256) {
        // the position's scores requested together (unconditional loads from
        // clamped indices: a load in the loop was waited for before the next)
        const float* sc = a.route_scores + (size_t)p * a.topk;
        float sv[WH_BATCH_MAX_TOPK];
#pragma unroll
        for (uint32_t k = 0; k < WH_BATCH_MAX_TOPK; ++k) sv[k] = sc[k < a.topk ? k : 0u];
        float sum = 0.0f;
        bool finite = true;
#pragma unroll
        for (uint32_t k = 0; k < WH_BATCH_MAX_TOPK; ++k) {
            if (k < a.topk) {
                finite = finite && fabsf(sv[k]) <= 3.4028235e38f;
                sum = sum + sv[k];
            }
        }
        finite = finite && fabsf(sum) <= 3.4028235e38f && sum > 0.0f;
        const float uniform = 1.0f / (float)a.topk;
#pragma unroll
        for (uint32_t k = 0; k < WH_BATCH_MAX_TOPK; ++k)
            if (k < a.topk) wsh[p * a.topk + k] = finite ? sv[k] / sum : uniform;
    }
    __syncthreads();
    if (bad) {
        if (tid == 0) {
            for (int i = 0; i < 5; ++i) a.meta[i] = 0;
            a.meta[7] = 0;
            atomicOr(a.status, WH_ST_NOT_RESIDENT);
        }
        return;
    }
    for (uint32_t i = tid; i < S; i += 256) atomicAdd(&cnt[ids[i]], 1u);
    __syncthreads();
    // slot offsets and used-expert indices in ascending id: thread t owns
    // ids [4t, 4t + 4)
    uint32_t c4[4], sum4 = 0, used4 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = 4 * tid + j;
        c4[j] = e < n_ids ? cnt[e] : 0u;
        sum4 += c4[j];
        used4 += c4[j] != 0;
    }
    uint32_t S_total, U;
    uint32_t o = wh_wg_exclusive_scan(sum4, tot, &S_total);
    uint32_t u = wh_wg_exclusive_scan(used4, tot, &U);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = 4 * tid + j;
        if (e < n_ids) {
            off[e] = o;
            cnt[e] = 0;  // reused as the placement cursor
            if (c4[j]) {
                a.uexp[u] = e;
                a.uoff[u] = o;
                uexpl[u] = e;
                uoffl[u] = o;
                ucnt[u] = c4[j];
                if (mfma_min && c4[j] >= mfma_min) atomicAdd(&n_mfma, 1u);
                ++u;
            }
        }
        o += c4[j];
    }
    if (tid == 0) a.uoff[U] = S;
    __syncthreads();
    // placement; the shared expert (the largest id, offset A) keeps position
    // order, so position p's shared slot is A + p
    for (uint32_t i = tid; i < S; i += 256) {
        const uint32_t e = ids[i];
        const uint32_t s = i >= A ? i : off[e] + atomicAdd(&cnt[e], 1u);
        a.sorted[s] = i;
        a.pos[s] = wh_slot_pos(a, i);
        slot_of[i] = s;
    }
    // work order: most slots first, ties by ascending id (rank counting);
    // thread t owns used experts t, t + 256, ... and requests their matrices
    // first, so that the round trip overlaps the counting
    constexpr int kOwn = WH_BATCH_MAX_TABLE / 256;
    wh_expert_ptrs own[kOwn];
    uint32_t own_r[kOwn];
#pragma unroll
    for (int k = 0; k < kOwn; ++k) {
        const uint32_t v = tid + 256 * k;
        if (v < U) own[k] = wh_batch_expert(a, uexpl[v]);
    }
#pragma unroll
    for (int k = 0; k < kOwn; ++k) {
        const uint32_t v = tid + 256 * k;
        own_r[k] = 0;
        if (v >= U) continue;
        const uint32_t cv = ucnt[v];
        uint32_t r = 0, w = 0;
        for (; w + 4 <= U; w += 4) {
            const uint4 c = *(const uint4*)&ucnt[w];
            r += (c.x > cv || (c.x == cv && w < v)) + (c.y > cv || (c.y == cv && w + 1 < v)) +
                 (c.z > cv || (c.z == cv && w + 2 < v)) + (c.w > cv || (c.w == cv && w + 3 < v));
        }
        for (; w < U; ++w) {
            const uint32_t cw = ucnt[w];
            r += cw > cv || (cw == cv && w < v);
        }
        own_r[k] = r;
        a.uorder[r] = v;
        uordl[r] = v;
        // the MFMA experts (the first n_mfma of the work order) become
        // virtual experts of at most 16 slots
        vst[r] = r < n_mfma ? (cv + 15) / 16 : 0u;
    }
    __syncthreads();
    // their start in the list: a scan over the work order (positions
    // 4t .. 4t + 3 per thread)
    {
        uint32_t ch[4], csum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = 4 * tid + j;
            ch[j] = i < U ? vst[i] : 0u;
            csum += ch[j];
        }
        uint32_t V;
        uint32_t v0 = wh_wg_exclusive_scan(csum, tot, &V);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = 4 * tid + j;
            if (i < U) vst[i] = v0;
            v0 += ch[j];
        }
        if (tid == 0) a.meta[7] = V;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kOwn; ++k) {
        const uint32_t v = tid + 256 * k;
        if (v >= U || own_r[k] >= n_mfma) continue;
        const wh_expert_ptrs ep = own[k];
        uint32_t vi = vst[own_r[k]];
        for (uint32_t c = 0; 16 * c < ucnt[v]; ++c, ++vi) {
            wh_bmx_vt t;
            t.w1 = ep.w1, t.s1 = ep.s1, t.w3 = ep.w3, t.s3 = ep.s3, t.w2 = ep.w2, t.s2 = ep.s2;
            t.slot0 = uoffl[v] + 16 * c;
            t.count = ucnt[v] - 16 * c < 16 ? ucnt[v] - 16 * c : 16u;
            a.vtab[vi] = t;
        }
    }
    // each position's route slots by ascending expert id, equal ids in route
    // order (E/server/generation.rs:2491-2506 pushes targets in that order):
    // key (id, route index) is distinct, and its rank among the position's
    // keys is its place (compile-time indices only: the keys stay in
    // registers).  The weights (in LDS, in route order) are permuted into
    // that order too, so the accumulate reads them beside the slots.
    for (uint32_t p = tid; p < a.npos; p += 256) {
        const uint32_t k0 = p * a.topk;
        uint32_t key[WH_BATCH_MAX_TOPK];
        float wk[WH_BATCH_MAX_TOPK];
#pragma unroll
        for (uint32_t k = 0; k < WH_BATCH_MAX_TOPK; ++k) {
            key[k] = k < a.topk ? (ids[k0 + k] << 4) | k : 0xffffffffu;
            wk[k] = k < a.topk ? wsh[k0 + k] : 0.0f;
        }
#pragma unroll
        for (uint32_t k = 0; k < WH_BATCH_MAX_TOPK; ++k) {
            if (k < a.topk) {
                uint32_t r = 0;
#pragma unroll
                for (uint32_t j = 0; j < WH_BATCH_MAX_TOPK; ++j) r += key[j] < key[k];
                a.acc_order[k0 + r] = slot_of[k0 + k];
                a.wgt[k0 + r] = wk[k];
            }
        }
    }
    if (tid == 0) {
        a.meta[0] = U;
        a.meta[1] = 1;
        a.meta[2] = 0;
        a.meta[3] = 0;
        a.meta[4] = n_mfma;
    }
}

// ------------------------------------------------------------------ act-quant
// amax over the 64 / kV lanes that hold one 64-block, kV values each (kV = 4
// or 8; NaN skipped, as f32::max does): quad swaps, then the half-row mirror
// (8 lanes) and, for kV = 4, the row mirror (16 lanes).
template <int kV>
__device__ __forceinline__ float wh_amax_block(float m) {
    static_assert(kV == 4 || kV == 8, "64-block over 16 or 8 lanes");
    m = fmaxf(m, wh_dpp_quad_swap1(m));
    m = fmaxf(m, wh_dpp_quad_swap2(m));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x141, 0xf, 0xf, false)));  // row_half_mirror
    if constexpr (kV == 4)
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x140, 0xf, 0xf, false)));  // row_mirror
    return m;
}

// Act-quant (E/compute.rs:2504-2521, block 64) of kV consecutive values held
// by one thread, the block's threads being 64 / kV consecutive lanes: q = the
// E4M3 values before the scale 2^k.  The reference's semantics for
// non-finite inputs, as wh_xq_quant16: NaN quantizes to -480, an infinite
// amax gives an infinite scale; bad reports an inf or NaN among the kV.
template <int kV>
__device__ __forceinline__ void wh_aq_vals(const float (&v)[kV], const uint32_t* log2_thr, float (&q)[kV], int& k,
                                           float& sc, bool& bad) {
    float amax = 0.0f;
    bad = false;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        const float m = fabsf(v[i]);
        bad |= !(m <= 3.4028235e38f);
        amax = fmaxf(amax, m);
    }
    amax = wh_amax_block<kV>(amax);
    const bool inf_scale = !(amax <= 3.4028235e38f);
    k = inf_scale ? 0 : wh_aq_scale_exp(amax, log2_thr);
    const float inv = inf_scale ? 0.0f : wh_pow2f(-k);  // v / inf is v * 0
    sc = inf_scale ? __uint_as_float(0x7f800000u) : wh_pow2f(k);
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        const float t = v[i] * inv;
        q[i] = t != t ? -480.0f : wh_e4m3_round(wh_clamp448_finite(t));
    }
}

// SwiGLU (E/deepseek_v4.rs:590-594) of the gate and up matvecs, h =
// silu(min(g, 10)) * clamp(u, -10, 10), and the act-quant of h (block 64,
// E/compute.rs:2504-2521) in one pass: 4 values per thread, a 64-block over
// 16 lanes.  Writes what wh_batch_quant_rows writes for x (the dequantized
// values, the codes in MFMA group order, one E8M0 byte per 32-col group);
// h itself is never stored.  n = slots * inter values (inter a multiple of
// 64, so a block's 16 lanes are all in range or all out).  Grid: n / 1024
// blocks of 256 threads, rounded up.
__global__ void __launch_bounds__(256) k_moe_batch_swiglu_quant(const float* __restrict__ g,
                                                                const float* __restrict__ u, uint32_t n,
                                                                float* __restrict__ q32, uint8_t* __restrict__ q8,
                                                                uint8_t* __restrict__ s8) {
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    __shared__ uint32_t thr[256];
    wh_thr_stage ts;
    wh_exp_stage es;
    wh_thr_stage_load(ts);
    wh_exp_stage_load(es);
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const bool on = 4 * i < n;
    float4 gv = make_float4(0.0f, 0.0f, 0.0f, 0.0f), uv = gv;  // lanes past the end quantize zeros
    if (on) {
        gv = ((const float4*)g)[i];
        uv = ((const float4*)u)[i];
    }
    wh_thr_stage_store(ts, thr);
    wh_exp_stage_store(es, exp_tab);
    __syncthreads();
    const float v[4] = {wh_swiglu(gv.x, uv.x, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT),
                        wh_swiglu(gv.y, uv.y, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT),
                        wh_swiglu(gv.z, uv.z, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT),
                        wh_swiglu(gv.w, uv.w, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT)};
    float q[4], sc;
    int k;
    bool bad;
    wh_aq_vals<4>(v, thr, q, k, sc, bad);
    // this thread's codes, column 4j + e of its 32-col group in byte e
    // (j = lane % 8)
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    const uint32_t p = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
    // MFMA group order: byte 4c + m of the group holds column c + 8m, so
    // dword d = j gathers byte d % 4 of the lanes d / 4 + 2m, m = 0..3
    const uint32_t lane = threadIdx.x & 63u, j = lane & 7u;
    const int src = (int)((lane & ~7u) + (j >> 2));
    const uint32_t sh = 8u * (j & 3u);
    uint32_t dw = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) dw |= (((uint32_t)__shfl((int)p, src + 2 * m, 64) >> sh) & 0xffu) << (8 * m);
    if (!on) return;
    ((float4*)q32)[i] = make_float4(q[0] * sc, q[1] * sc, q[2] * sc, q[3] * sc);
    ((uint32_t*)q8)[i] = dw;
    // sc = 2^k: E8M0 byte 127 + k - 3 (0xFF for an infinite scale), as
    // wh_batch_quant_rows
    const uint32_t be = (__float_as_uint(sc) >> 23) & 0xffu;
    if (j == 0) s8[i >> 3] = (uint8_t)(be == 0xffu ? 0xffu : be - 3u);
}

// ------------------------------------------------------------ exact items
// One 32-col group of one of two act-quantized vectors, loaded early: thread
// t takes group t of the first vector or group t - G of the second (2G <=
// 256), so the loads can be issued before the weight row's.
struct wh_xq_group_stage {
    float4 v[8];
    float* dst;
    uint32_t g;
    bool on;
};
__device__ __forceinline__ void wh_xq_group_load(wh_xq_group_stage& st, const float* __restrict__ src0,
                                                 const float* __restrict__ src1, bool two, uint32_t G, float* xs0,
                                                 float* xs1) {
    const uint32_t i = threadIdx.x;
    st.on = i < (two ? 2 * G : G);
    const bool second = i >= G;
    st.g = second ? i - G : i;
    st.dst = second ? xs1 : xs0;
    if (st.on) {
        const float4* p = (const float4*)((second ? src1 : src0) + 32 * st.g);
#pragma unroll
        for (int q = 0; q < 8; ++q) st.v[q] = p[q];
    }
}
__device__ __forceinline__ void wh_xq_group_store(const wh_xq_group_stage& st) {
    if (!st.on) return;
    float v[32];
#pragma unroll
    for (int m = 0; m < 32; ++m) v[m] = wh_f4_get(st.v[m >> 2], m & 3);
    wh_stage_fp4_store_group(st.dst, st.g, v);
}

// One or two act-quantized vectors (column order, n floats, n % 32 == 0)
// into LDS in FP4 lane order: one 32-col group per thread and pass, the
// groups of both vectors spread over the workgroup.
__device__ __forceinline__ void wh_stage_xq_lanes2(const float* __restrict__ src0, const float* __restrict__ src1,
                                                   bool two, uint32_t n, float* xs0, float* xs1) {
    const uint32_t G = n / 32;
    for (uint32_t i = threadIdx.x; i < (two ? 2 * G : G); i += 256) {
        const bool second = i >= G;
        const uint32_t g = second ? i - G : i;
        const float4* p = (const float4*)((second ? src1 : src0) + 32 * g);
        float v[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 f = p[q];
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
        wh_stage_fp4_store_group(second ? xs1 : xs0, g, v);
    }
}

// One dword of one lane (two groups) against two inputs: one decode, and
// each input keeps the reference chain of the single-input path.
__device__ __forceinline__ void wh_fp4_lane_pair2(uint32_t word, const float4* xg0, const float4* xg1, uint32_t ja,
                                                  uint32_t jb, float sa, float sb, bool two, float& acc0,
                                                  float& acc1, uint32_t lut_hi = WH_FP4_LUT_HI) {
    const wh_fp4x8 e = wh_fp4_decode8(word, lut_hi);
    {
        const float4 xa = xg0[ja], xb = xg0[jb];
        float ga = __builtin_fmaf(e.a01.x, xa.x, 0.0f);
        ga = __builtin_fmaf(e.a01.y, xa.y, ga);
        ga = __builtin_fmaf(e.a23.x, xa.z, ga);
        ga = __builtin_fmaf(e.a23.y, xa.w, ga);
        acc0 = __builtin_fmaf(ga, sa, acc0);
        float gb = __builtin_fmaf(e.b01.x, xb.x, 0.0f);
        gb = __builtin_fmaf(e.b01.y, xb.y, gb);
        gb = __builtin_fmaf(e.b23.x, xb.z, gb);
        gb = __builtin_fmaf(e.b23.y, xb.w, gb);
        acc0 = __builtin_fmaf(gb, sb, acc0);
    }
    if (two) {
        const float4 xa = xg1[ja], xb = xg1[jb];
        float ga = __builtin_fmaf(e.a01.x, xa.x, 0.0f);
        ga = __builtin_fmaf(e.a01.y, xa.y, ga);
        ga = __builtin_fmaf(e.a23.x, xa.z, ga);
        ga = __builtin_fmaf(e.a23.y, xa.w, ga);
        acc1 = __builtin_fmaf(ga, sa, acc1);
        float gb = __builtin_fmaf(e.b01.x, xb.x, 0.0f);
        gb = __builtin_fmaf(e.b01.y, xb.y, gb);
        gb = __builtin_fmaf(e.b23.x, xb.z, gb);
        gb = __builtin_fmaf(e.b23.y, xb.w, gb);
        acc1 = __builtin_fmaf(gb, sb, acc1);
    }
}
__device__ __forceinline__ void wh_fp4_lane_block2(uint4 w, const float4* xp0, const float4* xp1, const float* s8row,
                                                   uint32_t b, bool two, float& acc0, float& acc1) {
    const float4 s0 = ((const float4*)s8row)[2 * b], s1 = ((const float4*)s8row)[2 * b + 1];
    const float4* g0 = xp0 + 68 * b;
    const float4* g1 = xp1 + 68 * b;
    wh_fp4_lane_pair2(w.x, g0, g1, wh_xs_f4(0, 0), wh_xs_f4(1, 0), s0.x, s0.y, two, acc0, acc1);
    wh_fp4_lane_pair2(w.y, g0, g1, wh_xs_f4(2, 0), wh_xs_f4(3, 0), s0.z, s0.w, two, acc0, acc1);
    wh_fp4_lane_pair2(w.z, g0, g1, wh_xs_f4(4, 0), wh_xs_f4(5, 0), s1.x, s1.y, two, acc0, acc1);
    wh_fp4_lane_pair2(w.w, g0, g1, wh_xs_f4(6, 0), wh_xs_f4(7, 0), s1.z, s1.w, two, acc0, acc1);
}
// A lane's row (registers for kBlk > 0, else read per block) against one or
// two staged inputs.
template <int kBlk>
__device__ __forceinline__ void wh_fp4_lane_dot2(const wh_fp4_lane_row<(kBlk > 0 ? kBlk : 1)>& r,
                                                 const uint8_t* __restrict__ wrow, uint32_t blocks, const float* xs0,
                                                 const float* xs1, const float* s8row, uint32_t lane, bool two,
                                                 float& acc0, float& acc1) {
    const float4* xp0 = (const float4*)xs0 + lane;
    const float4* xp1 = (const float4*)xs1 + lane;
    acc0 = 0.0f;
    acc1 = 0.0f;
    if constexpr (kBlk > 0) {

        // the LDS reads of each half block are tied to the running sum, so
        // they cannot be hoisted ahead of the arithmetic before them (which
        // would keep every block's operands live)
#pragma unroll
        for (int b = 0; b < kBlk; ++b) {
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const uint32_t dep = wh_opaque_zero(acc0);
                const float4 sv = ((const float4*)(s8row + dep))[2 * b + hb];
                const float4* g0 = xp0 + dep + 68 * b;
                const float4* g1 = xp1 + dep + 68 * b;
                const uint32_t w0 = hb ? r.w[b].z : r.w[b].x, w1 = hb ? r.w[b].w : r.w[b].y;
                wh_fp4_lane_pair2(w0, g0, g1, wh_xs_f4(4 * hb, 0), wh_xs_f4(4 * hb + 1, 0), sv.x, sv.y, two, acc0,
                                  acc1);
                wh_fp4_lane_pair2(w1, g0, g1, wh_xs_f4(4 * hb + 2, 0), wh_xs_f4(4 * hb + 3, 0), sv.z, sv.w, two,
                                  acc0, acc1);
            }
        }
    } else {
        const uint4* p = (const uint4*)wrow + lane;
        for (uint32_t b = 0; b < blocks; ++b) wh_fp4_lane_block2(p[8 * b], xp0, xp1, s8row, b, two, acc0, acc1);
    }
}

// LDS bytes of an exact item over `cols` input columns: two staged inputs and
// the 32-row scale table.
__host__ __device__ constexpr size_t wh_exact_item_lds(size_t cols) {
    return sizeof(float) * (2 * (size_t)wh_xs_floats((uint32_t)cols) + 32 * (size_t)wh_s8_stride((uint32_t)(cols / 32)));
}

// One exact item: 32 rows (octet o runs row row_of(o)) of the expert against
// every slot in [s_beg, s_end), two slots per pass.  `in` gives a slot's
// act-quantized input row (column order); `emit` takes the two octet-lane
// sums of a pass.
template <int kBlk, class In, class Emit>
__device__ __forceinline__ void wh_exact_item(const uint8_t* wrow, const uint8_t* srow, uint32_t cols,
                                              uint32_t s_beg, uint32_t s_end, float* lds, In in, Emit emit) {
    const uint32_t G = cols >> 5, xsf = wh_xs_floats(cols);
    float* xs0 = lds;
    float* xs1 = lds + xsf;
    const uint32_t lane = threadIdx.x & 7, oct = threadIdx.x >> 3;
    float* s8row = lds + 2 * xsf + oct * wh_s8_stride(G);
    wh_fp4_lane_row<(kBlk > 0 ? kBlk : 1)> r;
    const bool early = kBlk > 0 && 2 * G <= 256;
    if constexpr (kBlk > 0) {
        // the first pair's inputs and the scales are loaded before the row,
        // so waiting for them does not wait for the row's bytes (loads
        // complete in issue order)
        const bool two = s_beg + 1 < s_end;
        wh_xq_group_stage xst;
        if (early) wh_xq_group_load(xst, in(s_beg), in(two ? s_beg + 1 : s_beg), two, G, xs0, xs1);
        wh_s8_stage<kBlk> ss;
        wh_s8_stage_load<kBlk>(ss, srow, lane);
        wh_fp4_lane_row_load<kBlk>(r, wrow, lane);
        __builtin_amdgcn_sched_barrier(0);
        wh_s8_stage_store<kBlk>(ss, s8row, lane);
        if (early) wh_xq_group_store(xst);
    } else {
        wh_s8_stage_rt(srow, G, s8row, lane);
    }
    for (uint32_t s = s_beg; s < s_end; s += 2) {
        const bool two = s + 1 < s_end;
        if (s != s_beg) {
            __syncthreads();  // the previous pair is done with xs
            wh_stage_xq_lanes2(in(s), in(two ? s + 1 : s), two, cols, xs0, xs1);
        } else if (!early) {
            wh_stage_xq_lanes2(in(s), in(two ? s + 1 : s), two, cols, xs0, xs1);
        }
        __syncthreads();
        float acc0, acc1;
        if constexpr (kBlk > 0) {
            // the row's words are opaque per pass: hoisted out of this loop,
            // their decoded codes would double the row's registers
#pragma unroll
            for (int b = 0; b < kBlk; ++b) asm volatile("" : "+v"(r.w[b].x), "+v"(r.w[b].y), "+v"(r.w[b].z), "+v"(r.w[b].w));
        }
        wh_fp4_lane_dot2<kBlk>(r, wrow, G >> 3, xs0, xs1, s8row, lane, two, acc0, acc1);
        emit(s, two, wh_hsum8(acc0) + 0.0f, wh_hsum8(acc1) + 0.0f);
    }
}

// ------------------------------------------------------------- MFMA items
// v_mfma_scale_f32_16x16x128_f8f6f4 with E4M3 operands: lane L holds 32
// codes of A row L % 16 (and of B column L % 16); bytes i of lane groups
// g = L / 16 pair up between A and B; the 16-byte half h of lane group g is
// scaled by the E8M0 byte of lane group 2h + g / 2 (same row / column); the
// accumulator's register r of lane L is C[4 * (L / 16) + r][L % 16].
//
// Per 256-col block (8 groups, two MFMAs u = 0, 1) lane group g takes dword
// d = 2 * (g / 2) + u of the resident chunks c = 4 * (g % 2) .. + 3: byte
// half 0 = the codes of group 2d (columns c + 8k, k = 0..3), half 1 = group
// 2d + 1.  Its scale lane group s provides group 4 * (s % 2) + 2u + s / 2.
#define WH_MFMA_TOK 64u       // tokens per pass: 4 N-tiles of 16
#define WH_MFMA_TSTRIDE 272u  // LDS bytes per token per block: 8 groups x 32 codes + 16
#define WH_MFMA_BUF (WH_MFMA_TOK * WH_MFMA_TSTRIDE + WH_MFMA_TOK * 8u)
__host__ __device__ constexpr size_t wh_mfma_item_lds() { return 2 * (size_t)WH_MFMA_BUF; }

// The E4M3 codes of the reference's x8 integer values of the two groups of a
// resident FP4 dword (the first half of wh_fp4_decode8).
__device__ __forceinline__ void wh_fp4_codes(uint32_t w, uint32_t& fa, uint32_t& fb) {
    fa = __builtin_amdgcn_perm(WH_FP4_LUT_HI, WH_FP4_LUT_LO, w & 0x07070707u);
    const uint32_t r = __builtin_amdgcn_alignbit(w, w, 4);
    fa |= r & 0x80808080u;
    fb = __builtin_amdgcn_perm(WH_FP4_LUT_HI, WH_FP4_LUT_LO, r & 0x07070707u) | (w & 0x80808080u);
}
// Scale byte that scale lane group s provides for MFMA u, from a block's 8
// scale bytes.
template <int u>
__device__ __forceinline__ uint32_t wh_mfma_sbyte(uint2 s8, uint32_t s) {
    const uint32_t w = (s & 1) ? s8.y : s8.x;
    return (w >> (8 * (2 * u + (s >> 1)))) & 0xffu;
}

// One 256-col block of A rows in registers: 4 chunks x 2 dwords (u = 0, 1).
struct wh_mfma_a {
    uint2 c[4];
    uint2 s;  // the row's 8 scale bytes of the block
};
template <int u>
__device__ __forceinline__ wh_v8i wh_mfma_a_codes(const wh_mfma_a& a) {
    wh_v8i v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t fa, fb;
        wh_fp4_codes(u ? a.c[j].y : a.c[j].x, fa, fb);
        v[j] = (int)fa;
        v[4 + j] = (int)fb;
    }
    return v;
}

// A operand loads.  The MFMA lane (m, g) needs, per 256-col block of row m,
// the dword pair 2(g/2), 2(g/2) + 1 of the four 16-byte chunks
// 4(g%2) .. 4(g%2) + 3 (wh_mfma_a): four 8-byte pieces 16 bytes apart.  As
// loads those stream at ~4 TB/s; instead each lane loads 32 contiguous bytes
// - chunks 4(g%2) + 2(g/2) and the next - and lanes L and L ^ 32 (the two
// values of g/2) trade the dword pairs each needs from the other's chunks
// with v_permlane32_swap, at ~5.4 TB/s.
struct wh_mx_raw {
    uint4 p, q;  // the lane's two chunks as loaded
    uint2 s;     // the row's 8 scale bytes of the block
};
// wlane = row base + 64 (g % 2) + 32 (g / 2); srow = the row's scale bytes.
__device__ __forceinline__ void wh_mx_raw_load(wh_mx_raw& r, const uint8_t* wlane, const uint8_t* srow, uint32_t blk) {
    r.p = *(const uint4*)(wlane + blk * 128);
    r.q = *(const uint4*)(wlane + blk * 128 + 16);
    r.s = *(const uint2*)(srow + blk * 8);
}
// The exchange: the lower half of the wave (g / 2 = 0) keeps dwords 0, 1 and
// takes dwords 0, 1 of the upper lanes' chunks; the upper half keeps
// dwords 2, 3 and takes dwords 2, 3 of the lower lanes' chunks.  All 64
// lanes must take part.
__device__ __forceinline__ wh_mfma_a wh_mx_fix(const wh_mx_raw& r) {
    const auto sp0 = __builtin_amdgcn_permlane32_swap(r.p.x, r.p.z, false, false);
    const auto sp1 = __builtin_amdgcn_permlane32_swap(r.p.y, r.p.w, false, false);
    const auto sq0 = __builtin_amdgcn_permlane32_swap(r.q.x, r.q.z, false, false);
    const auto sq1 = __builtin_amdgcn_permlane32_swap(r.q.y, r.q.w, false, false);
    wh_mfma_a a;
    a.c[0] = make_uint2(sp0[0], sp1[0]);  // chunk 4(g%2):     own (lower) or from lower (upper)
    a.c[1] = make_uint2(sq0[0], sq1[0]);  // chunk 4(g%2) + 1
    a.c[2] = make_uint2(sp0[1], sp1[1]);  // chunk 4(g%2) + 2: from upper (lower) or own (upper)
    a.c[3] = make_uint2(sq0[1], sq1[1]);  // chunk 4(g%2) + 3
    a.s = r.s;
    return a;
}

// B staging: thread t copies 64 code bytes (groups 2q, 2q + 1 of the block,
// q = t % 4) and, for q = 0, the 8 scale bytes of token t / 4.
struct wh_mfma_b {
    uint4 v[4];
    uint2 s;
};
__device__ __forceinline__ void wh_mfma_b_load(wh_mfma_b& b, const uint8_t* rec, const uint8_t* srec, bool on,
                                               uint32_t blk) {
    const uint32_t q = threadIdx.x & 3;
    if (on) {
        const uint4* p = (const uint4*)(rec + blk * 256 + q * 64);
#pragma unroll
        for (int j = 0; j < 4; ++j) b.v[j] = p[j];
        b.s = *(const uint2*)(srec + blk * 8);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) b.v[j] = make_uint4(0, 0, 0, 0);
        b.s = make_uint2(0x7f7f7f7fu, 0x7f7f7f7fu);
    }
}
__device__ __forceinline__ void wh_mfma_b_store(const wh_mfma_b& b, uint8_t* buf) {
    const uint32_t n = threadIdx.x >> 2, q = threadIdx.x & 3;
    uint4* d = (uint4*)(buf + n * WH_MFMA_TSTRIDE + q * 64);
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = b.v[j];
    if (q == 0) *(uint2*)(buf + WH_MFMA_TOK * WH_MFMA_TSTRIDE + n * 8) = b.s;
}
// B operand and scale byte of MFMA u for token n of the staged block.
template <int u>
__device__ __forceinline__ wh_v8i wh_mfma_b_codes(const uint8_t* buf, uint32_t n, uint32_t g) {
    const uint8_t* p = buf + n * WH_MFMA_TSTRIDE + (4 * (g >> 1) + 2 * u) * 32 + 16 * (g & 1);
    const uint4 lo = *(const uint4*)p, hi = *(const uint4*)(p + 32);
    wh_v8i v;
    v[0] = (int)lo.x;
    v[1] = (int)lo.y;
    v[2] = (int)lo.z;
    v[3] = (int)lo.w;
    v[4] = (int)hi.x;
    v[5] = (int)hi.y;
    v[6] = (int)hi.z;
    v[7] = (int)hi.w;
    return v;
}

// One MFMA item: kMat (1 or 2) weight matrices x 64 rows (16 per wave)
// against every slot in [s_beg, s_end), 64 slots per pass.  `rec(s)` gives
// a slot's code row and scale row; `emit(s0, count, acc)` takes a pass's
// accumulators (acc[m][nt]: matrix m, N-tile nt).
template <int kMat, class Rec, class Emit>
__device__ __forceinline__ void wh_mfma_item(const uint8_t* const* wmat, const uint8_t* const* smat, uint32_t row0,
                                             uint32_t cols, uint32_t s_beg, uint32_t s_end, uint8_t* lds, Rec rec,
                                             Emit emit) {
    const uint32_t L = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t m = L & 15, g = L >> 4;
    const uint32_t row = row0 + wave * 16 + m;
    const uint32_t nblk = cols / 256, G = cols / 32;
    const uint8_t* wl[kMat];
    const uint8_t* sr[kMat];
#pragma unroll
    for (int i = 0; i < kMat; ++i) {
        wl[i] = wmat[i] + (size_t)row * (cols / 2) + 64 * (g & 1) + 32 * (g >> 1);
        sr[i] = smat[i] + (size_t)row * G;
    }
    for (uint32_t s0 = s_beg; s0 < s_end; s0 += WH_MFMA_TOK) {
        const uint32_t count = min(WH_MFMA_TOK, s_end - s0);
        const uint32_t tn = threadIdx.x >> 2;
        const bool ton = tn < count;
        const uint8_t* brec = nullptr;
        const uint8_t* bsrec = nullptr;
        rec(ton ? s0 + tn : s0, brec, bsrec);
        wh_v4f acc[kMat][4];
#pragma unroll
        for (int i = 0; i < kMat; ++i)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) acc[i][nt] = wh_v4f{0.0f, 0.0f, 0.0f, 0.0f};
        wh_mx_raw ra[kMat], na[kMat];
        wh_mfma_b rb;
#pragma unroll
        for (int i = 0; i < kMat; ++i) wh_mx_raw_load(ra[i], wl[i], sr[i], 0);
        wh_mfma_b_load(rb, brec, bsrec, ton, 0);
        if (s0 != s_beg) __syncthreads();  // the previous pass is done with the LDS
        wh_mfma_b_store(rb, lds);
        __syncthreads();
        for (uint32_t blk = 0; blk < nblk; ++blk) {
            const bool more = blk + 1 < nblk;
            if (more) {
#pragma unroll
                for (int i = 0; i < kMat; ++i) wh_mx_raw_load(na[i], wl[i], sr[i], blk + 1);
                wh_mfma_b_load(rb, brec, bsrec, ton, blk + 1);
            }
            const uint8_t* buf = lds + (blk & 1) * WH_MFMA_BUF;
            const uint8_t* bsc = buf + WH_MFMA_TOK * WH_MFMA_TSTRIDE;
            wh_mfma_a fa[kMat];
#pragma unroll
            for (int i = 0; i < kMat; ++i) fa[i] = wh_mx_fix(ra[i]);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                wh_v8i av[kMat];
                uint32_t as[kMat];
#pragma unroll
                for (int i = 0; i < kMat; ++i) {
                    av[i] = u ? wh_mfma_a_codes<1>(fa[i]) : wh_mfma_a_codes<0>(fa[i]);
                    as[i] = u ? wh_mfma_sbyte<1>(fa[i].s, g) : wh_mfma_sbyte<0>(fa[i].s, g);
                }
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    if (nt * 16 < count) {
                        const uint32_t n = nt * 16 + m;
                        const wh_v8i bv = u ? wh_mfma_b_codes<1>(buf, n, g) : wh_mfma_b_codes<0>(buf, n, g);
                        const uint2 bs2 = *(const uint2*)(bsc + n * 8);
                        const uint32_t bs = u ? wh_mfma_sbyte<1>(bs2, g) : wh_mfma_sbyte<0>(bs2, g);
#pragma unroll
                        for (int i = 0; i < kMat; ++i)
                            acc[i][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                av[i], bv, acc[i][nt], 0, 0, 0, (int)as[i], 0, (int)bs);
                    }
                }
            }
            if (more) {
                wh_mfma_b_store(rb, lds + ((blk + 1) & 1) * WH_MFMA_BUF);
#pragma unroll
                for (int i = 0; i < kMat; ++i) ra[i] = na[i];
            }
            __syncthreads();
        }
        emit(s0, count, acc);
    }
}

// ------------------------------------------------------- persistent kernels

// LDS of a persistent routed-expert workgroup over `cols` input columns:
// the larger of the exact and the MFMA items'.
__host__ __device__ constexpr size_t wh_batch_wg_lds(size_t cols) {
    return wh_exact_item_lds(cols) > wh_mfma_item_lds() ? wh_exact_item_lds(cols) : wh_mfma_item_lds();
}

// Work queue of a persistent workgroup (counter zeroed by the pack).  The
// next item's index is fetched when an item starts, so the atomic's round
// trip overlaps the item's own loads.
struct wh_queue {
    uint32_t* counter;
    uint32_t* item_s;  // LDS broadcast slot
    uint32_t next;     // thread 0: the fetched index
    __device__ __forceinline__ uint32_t first() {
        if (threadIdx.x == 0) *item_s = atomicAdd(counter, 1u);
        __syncthreads();
        return *item_s;
    }
    __device__ __forceinline__ void prefetch() {
        if (threadIdx.x == 0) next = atomicAdd(counter, 1u);
    }
    __device__ __forceinline__ uint32_t advance() {
        __syncthreads();  // the item is done with the LDS and item_s
        if (threadIdx.x == 0) *item_s = next;
        __syncthreads();
        return *item_s;
    }
};

// MFMA item epilogue: the accumulators of a pass into dst[slot][row]
// (C register r of lane L = row 4 * (L / 16) + r of the wave's 16, token
// L % 16 of the N-tile).
__device__ __forceinline__ void wh_mfma_store(const wh_batch_args& a, float* dst, uint32_t ld, uint32_t row0,
                                              uint32_t s0, uint32_t count, const wh_v4f (&acc)[1][4]) {
    const uint32_t L = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = row0 + wave * 16 + 4 * (L >> 4);
    bool nf = false;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const uint32_t n = nt * 16 + (L & 15);
        if (n < count) {
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                o[r] = acc[0][nt][r] + 0.0f;
                nf = nf || !(fabsf(o[r]) <= 3.4028235e38f);
            }
            *(float4*)(dst + (size_t)(s0 + n) * ld + r0) = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
    if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
}

// Gate and up matvecs of every slot.  The queue holds the MFMA items first -
// (expert, matrix w1 or w3, 64 rows of inter) for the experts at the head of
// the work order - then the exact items - (expert, 16 rows of inter), octet
// 2r running the w1 row r of the tile and octet 2r + 1 the w3 row r.  One
// queue keeps the MFMA items, few and bound by memory, running beside the
// exact ones, bound by VALU issue.
// Three workgroups per CU: the register budget (168) is what the LDS allows.
template <int kBlk>
__global__ void __launch_bounds__(256, 2) k_moe_batch_gateup(wh_batch_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t item_s;
    const uint32_t n_mfma = a.meta[6] ? 0u : a.meta[4], mt = a.inter >> 6, et = a.inter >> 4;
    const uint32_t n_m = a.mfma_external ? 0u : n_mfma * 2 * mt, n_items = n_m + (a.meta[0] - n_mfma) * et;
    if (n_items == 0) return;  // before the queue's atomic: every workgroup would take one
    wh_queue q{a.meta + 2, &item_s, 0};
    for (uint32_t item = q.first(); item < n_items; item = q.advance()) {
        q.prefetch();
        if (item < n_m) {
            const uint32_t u = a.uorder[item / (2 * mt)], rest = item % (2 * mt);
            const bool up = rest >= mt;
            const uint32_t row0 = (up ? rest - mt : rest) * 64;
            const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
            const uint8_t* wm[1] = {up ? ep.w3 : ep.w1};
            const uint8_t* sm[1] = {up ? ep.s3 : ep.s1};
            float* dst = up ? a.u : a.g;
            wh_mfma_item<1>(
                wm, sm, row0, a.hidden, a.uoff[u], a.uoff[u + 1], (uint8_t*)lds,
                [&](uint32_t s, const uint8_t*& rec, const uint8_t*& srec) {
                    const uint32_t p = wh_slot_pos(a, a.sorted[s]);
                    rec = a.xq8 + (size_t)p * a.hidden;
                    srec = a.xs8 + (size_t)p * (a.hidden / 32);
                },
                [&](uint32_t s0, uint32_t count, const wh_v4f (&acc)[1][4]) {
                    wh_mfma_store(a, dst, a.inter, row0, s0, count, acc);
                });
            continue;
        }
        const uint32_t e = item - n_m;
        const uint32_t u = a.uorder[n_mfma + e / et], tile = e % et;
        const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
        const uint32_t oct = threadIdx.x >> 3;
        const uint32_t row = tile * 16 + (oct >> 1);
        const bool up = oct & 1;
        const uint32_t G = a.hidden >> 5;
        wh_exact_item<kBlk>(
            (up ? ep.w3 : ep.w1) + (size_t)row * (a.hidden >> 1), (up ? ep.s3 : ep.s1) + (size_t)row * G, a.hidden,
            a.uoff[u], a.uoff[u + 1], lds,
            [&](uint32_t s) { return a.xq + (size_t)wh_slot_pos(a, a.sorted[s]) * a.hidden; },
            [&](uint32_t s, bool two, float v0, float v1) {
                if ((threadIdx.x & 7) == 0) {
                    float* dst = up ? a.u : a.g;
                    bool nf = !(fabsf(v0) <= 3.4028235e38f);
                    dst[(size_t)s * a.inter + row] = v0;
                    if (two) {
                        nf = nf || !(fabsf(v1) <= 3.4028235e38f);
                        dst[(size_t)(s + 1) * a.inter + row] = v1;
                    }
                    if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
                }
            });
    }
}

// Down of every slot: MFMA items (expert, 64 output rows) first, then exact
// items (expert, 32 output rows); inputs are the act-quantized SwiGLU
// outputs of the slots.
// Four workgroups per CU (128 registers).
template <int kBlk>
__global__ void __launch_bounds__(256, 3) k_moe_batch_down(wh_batch_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t item_s;
    const uint32_t n_mfma = a.meta[6] ? 0u : a.meta[4], mt = a.hidden >> 6, et = a.hidden >> 5;
    const uint32_t n_m = a.mfma_external ? 0u : n_mfma * mt, n_items = n_m + (a.meta[0] - n_mfma) * et;
    if (n_items == 0) return;  // before the queue's atomic: every workgroup would take one
    wh_queue q{a.meta + 3, &item_s, 0};
    for (uint32_t item = q.first(); item < n_items; item = q.advance()) {
        q.prefetch();
        if (item < n_m) {
            const uint32_t u = a.uorder[item / mt], row0 = (item % mt) * 64;
            const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
            const uint8_t* wm[1] = {ep.w2};
            const uint8_t* sm[1] = {ep.s2};
            wh_mfma_item<1>(
                wm, sm, row0, a.inter, a.uoff[u], a.uoff[u + 1], (uint8_t*)lds,
                [&](uint32_t s, const uint8_t*& rec, const uint8_t*& srec) {
                    rec = a.hq8 + (size_t)s * a.inter;
                    srec = a.hs8 + (size_t)s * (a.inter / 32);
                },
                [&](uint32_t s0, uint32_t count, const wh_v4f (&acc)[1][4]) {
                    wh_mfma_store(a, a.y, a.hidden, row0, s0, count, acc);
                });
            continue;
        }
        const uint32_t e = item - n_m;
        const uint32_t u = a.uorder[n_mfma + e / et], tile = e % et;
        const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
        const uint32_t G = a.inter >> 5;
        const uint32_t row = tile * 32 + (threadIdx.x >> 3);
        wh_exact_item<kBlk>(
            ep.w2 + (size_t)row * (a.inter >> 1), ep.s2 + (size_t)row * G, a.inter, a.uoff[u], a.uoff[u + 1], lds,
            [&](uint32_t s) { return a.hq + (size_t)s * a.inter; },
            [&](uint32_t s, bool two, float v0, float v1) {
                if ((threadIdx.x & 7) == 0) {
                    bool nf = !(fabsf(v0) <= 3.4028235e38f);
                    a.y[(size_t)s * a.hidden + row] = v0;
                    if (two) {
                        nf = nf || !(fabsf(v1) <= 3.4028235e38f);
                        a.y[(size_t)(s + 1) * a.hidden + row] = v1;
                    }
                    if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
                }
            });
    }
}

// out_p = sum over p's experts in ascending id of y * w, from 0, unfused
// (E/compute.rs:1804-1807: `*slot += *value * weight`), then with the shared
// expert out_p = shared + routed (E/compute.rs:1838-1848).  Grid
// (hidden / 256, npos).  Nothing is written when a route was not resident.
// The last kernel of a call: it clears the non-finite input flag (and with
// it, unless k_moe_batch_mx fell back to fp32, the counts of MFMA and virtual
// experts, none of which ran).
__global__ void __launch_bounds__(256) k_moe_batch_accumulate(wh_batch_args a) {
    const uint32_t p = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    if (p == 0 && r == 0 && a.meta[6]) {
        if (!a.mx_fallback) {
            a.meta[4] = 0;
            a.meta[7] = 0;
        }
        a.meta[6] = 0;
    }
    if (r >= a.hidden || a.meta[1] == 0) return;
    float acc = 0.0f;
    for (uint32_t k = 0; k < a.topk; ++k) {
        const uint32_t s = a.acc_order[p * a.topk + k];
        const float v = a.y[(size_t)s * a.hidden + r] * a.wgt[p * a.topk + k];
        acc = acc + v;
    }
    if (a.has_shared) acc = a.y[(size_t)(a.npos * a.topk + p) * a.hidden + r] + acc;
    a.out[(size_t)p * a.hidden + r] = acc;
}
