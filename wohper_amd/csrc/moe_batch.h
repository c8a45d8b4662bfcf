// Ragged batched routed experts on gfx950.
//
// The expert-major batch path of the reference: per-position weights and the
// union of selected experts (E/server/generation.rs:2487-2506), then for each
// expert in ascending id and each of its positions acc_p += y * w
// (accumulate_expert_for_positions, E/compute.rs:1779-1810), and with a
// shared expert out_p = shared(x_p) + acc_p (E/compute.rs:1838-1852).
//
// Launch sequence (one stream):
//   k_moe_batch_pack     one workgroup: weights, the per-expert token lists
//                        (a bitonic sort of (expert id, assignment) keys), the
//                        used experts, their work order, per-position
//                        accumulation order
//   k_moe_batch_quant    act-quant (block 64) of every position's input
//   k_moe_batch_gateup   persistent: (expert, row tile) items from a queue
//   k_moe_batch_quant    act-quant of every slot's SwiGLU output
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

struct wh_batch_args {
    const wh_expert_ptrs* table;   // the layer's experts by id (null w1 = not resident)
    uint32_t n_table;              // valid ids are < n_table
    const uint32_t* route_ids;     // [npos][topk]
    const float* route_scores;     // [npos][topk]
    uint32_t npos, topk, hidden, inter;
    uint32_t has_shared;           // the shared expert runs on every position
    wh_expert_ptrs shared;         // ... under the id n_table
    uint32_t mfma_min;             // experts with this many slots take MFMA items (0: never)
    uint32_t debug_raw;            // test support: gate/up write gate into h and up into hq
    const void* x;                 // [npos][hidden], f32 or bf16
    uint32_t x_is_bf16;
    // assignments: i = p * topk + k for the routes, A + p for the shared
    // expert (A = npos * topk); S = A + has_shared * npos slots
    float* wgt;                    // [A] weight of route assignment i
    uint32_t* sorted;              // [S] assignments by (expert id, i): the slots
    uint32_t* uexp;                // [S] used expert ids, ascending
    uint32_t* uoff;                // [S + 1] their slot ranges
    uint32_t* uorder;              // [S] used-expert indices, most slots first
    uint32_t* acc_order;           // [A] per position: its route slots by ascending expert id
    uint32_t* meta;                // [0] used experts, [1] routes valid, [2]/[3] exact-item
                                   // queues, [4] experts on MFMA items, [5]/[6] MFMA queues
    float* xq;                     // [npos][hidden] act-quantized inputs (column order)
    uint8_t* xq8;                  // [npos][hidden] their E4M3 codes, MFMA group order
    uint8_t* xs8;                  // [npos][hidden / 32] E8M0 scale bytes (x 1/8)
    float* h;                      // [S][inter] SwiGLU outputs by slot
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
// One workgroup of 256 threads; S <= 4096 slots, n_table < 1024.
__global__ void __launch_bounds__(256) k_moe_batch_pack(wh_batch_args a) {
    __shared__ uint32_t key[WH_BATCH_MAX_ASSIGN];
    __shared__ uint32_t slot_of[WH_BATCH_MAX_ASSIGN];
    __shared__ uint32_t ubeg[WH_BATCH_MAX_TABLE + 1];  // slot ranges of the used experts
    __shared__ uint32_t scan[256];
    __shared__ uint32_t bad, n_used, n_mfma;
    const uint32_t A = a.npos * a.topk, S = A + a.has_shared * a.npos, tid = threadIdx.x;
    uint32_t N = 1;
    while (N < S) N <<= 1;
    if (tid == 0) {
        bad = 0;
        n_mfma = 0;
    }
    __syncthreads();
    // keys (expert id << 13 | assignment); ids are checked against the table
    for (uint32_t i = tid; i < N; i += 256) {
        uint32_t k = 0xffffffffu;
        if (i < A) {
            const uint32_t e = a.route_ids[i];
            if (e >= a.n_table || a.table[e].w1 == nullptr) bad = 1;
            else k = (e << 13) | i;
        } else if (i < S) {
            k = (a.n_table << 13) | i;
        }
        key[i] = k;
    }
    // per-position weights: score / sum, or 1 / len when the sequential sum
    // is not finite and positive or a score is not finite
    // (E/server/generation.rs:2495-2503)
    for (uint32_t p = tid; p < a.npos; p += 256) {
        const float* sc = a.route_scores + (size_t)p * a.topk;
        float sum = 0.0f;
        bool finite = true;
        for (uint32_t k = 0; k < a.topk; ++k) {
            finite = finite && fabsf(sc[k]) <= 3.4028235e38f;
            sum = sum + sc[k];
        }
        finite = finite && fabsf(sum) <= 3.4028235e38f && sum > 0.0f;
        const float uniform = 1.0f / (float)a.topk;
        for (uint32_t k = 0; k < a.topk; ++k) a.wgt[(size_t)p * a.topk + k] = finite ? sc[k] / sum : uniform;
    }
    __syncthreads();
    if (bad) {
        if (tid == 0) {
            for (int i = 0; i < 7; ++i) a.meta[i] = 0;
            atomicOr(a.status, WH_ST_NOT_RESIDENT);
        }
        return;
    }
    // bitonic sort, ascending: slots in (expert id, assignment) order
    for (uint32_t k = 2; k <= N; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < N; i += 256) {
                const uint32_t o = i ^ j;
                if (o > i) {
                    const uint32_t x0 = key[i], x1 = key[o];
                    if ((x0 > x1) == ((i & k) == 0)) {
                        key[i] = x1;
                        key[o] = x0;
                    }
                }
            }
            __syncthreads();
        }
    }
    // runs of equal ids: the used experts.  Thread t scans slots
    // [t * per, (t + 1) * per).
    const uint32_t per = (S + 255) / 256, s0 = min(tid * per, S), s1 = min(s0 + per, S);
    uint32_t starts = 0;
    for (uint32_t s = s0; s < s1; ++s) {
        const uint32_t i = key[s] & 0x1fffu;
        a.sorted[s] = i;
        slot_of[i] = s;
        starts += s == 0 || (key[s] >> 13) != (key[s - 1] >> 13);
    }
    scan[tid] = starts;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (uint32_t t = 0; t < 256; ++t) {
            const uint32_t v = scan[t];
            scan[t] = run;
            run += v;
        }
        n_used = run;
        a.uoff[run] = S;
        ubeg[run] = S;
    }
    __syncthreads();
    {
        uint32_t u = scan[tid];
        for (uint32_t s = s0; s < s1; ++s) {
            if (s == 0 || (key[s] >> 13) != (key[s - 1] >> 13)) {
                a.uexp[u] = key[s] >> 13;
                a.uoff[u] = s;
                ubeg[u] = s;
                ++u;
            }
        }
    }
    __syncthreads();
    const uint32_t U = n_used;
    // each position's route slots in ascending slot order = ascending expert
    // id, equal ids in route order
    for (uint32_t p = tid; p < a.npos; p += 256) {
        uint32_t sl[WH_BATCH_MAX_TOPK];
        const uint32_t k0 = p * a.topk;
        for (uint32_t k = 0; k < a.topk; ++k) {
            const uint32_t s = slot_of[k0 + k];
            uint32_t j = k;
            while (j > 0 && sl[j - 1] > s) {
                sl[j] = sl[j - 1];
                --j;
            }
            sl[j] = s;
        }
        for (uint32_t k = 0; k < a.topk; ++k) a.acc_order[k0 + k] = sl[k];
    }
    // work order: most slots first, ties by ascending id (keys reused)
    uint32_t N2 = 1;
    while (N2 < U) N2 <<= 1;
    for (uint32_t u = tid; u < N2; u += 256) {
        uint32_t k = 0xffffffffu;
        if (u < U) {
            const uint32_t c = ubeg[u + 1] - ubeg[u];
            k = ((WH_BATCH_MAX_ASSIGN - c) << 11) | u;
            if (a.mfma_min && c >= a.mfma_min) atomicAdd(&n_mfma, 1u);
        }
        key[u] = k;
    }
    __syncthreads();
    for (uint32_t k = 2; k <= N2; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < N2; i += 256) {
                const uint32_t o = i ^ j;
                if (o > i) {
                    const uint32_t x0 = key[i], x1 = key[o];
                    if ((x0 > x1) == ((i & k) == 0)) {
                        key[i] = x1;
                        key[o] = x0;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (uint32_t r = tid; r < U; r += 256) a.uorder[r] = key[r] & 0x7ffu;
    if (tid == 0) {
        a.meta[0] = U;
        a.meta[1] = 1;
        a.meta[2] = 0;
        a.meta[3] = 0;
        a.meta[4] = n_mfma;
        a.meta[5] = 0;
        a.meta[6] = 0;
    }
}

// ------------------------------------------------------------------ act-quant
// Act-quant (block 64) of rows of `n` values, 16 values per thread (a quad
// of threads holds one 64-block; E/compute.rs:2504-2521).  Writes the values
// in column order, their E4M3 codes in MFMA group order (per 32-col group,
// byte 4c + k holds column c + 8k) and one E8M0 byte per group: the block
// scale divided by 8, which takes the x8 of the FP4 integer LUT values.
// Grid: rows * n / 4096 blocks of 256 threads.
__global__ void __launch_bounds__(256) k_moe_batch_quant(const void* __restrict__ src, uint32_t src_bf16,
                                                         uint32_t rows, uint32_t n, float* __restrict__ q32,
                                                         uint8_t* __restrict__ q8, uint8_t* __restrict__ s8,
                                                         uint32_t* status, uint32_t report_nonfinite) {
    __shared__ uint32_t thr[256];
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_thr_stage_store(ts, thr);
    __syncthreads();
    const uint32_t per_row = n / 16;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t r = i / per_row, t = i - r * per_row;
    const bool on = r < rows;
    const bool bf16 = src_bf16 != 0;
    const size_t base = (size_t)(on ? r : 0) * n;
    const void* row = bf16 ? (const void*)((const uint16_t*)src + base) : (const void*)((const float*)src + base);
    wh_xq_stage st;
    wh_xq_stage_load(st, row, bf16, on ? n : 0u, t);
    float v[16];
    if (bf16) {
        const uint32_t w[8] = {st.raw[0].x, st.raw[0].y, st.raw[0].z, st.raw[0].w,
                               st.raw[1].x, st.raw[1].y, st.raw[1].z, st.raw[1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[4 * j] = __uint_as_float(st.raw[j].x);
            v[4 * j + 1] = __uint_as_float(st.raw[j].y);
            v[4 * j + 2] = __uint_as_float(st.raw[j].z);
            v[4 * j + 3] = __uint_as_float(st.raw[j].w);
        }
    }
    float amax = 0.0f;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float m = fabsf(v[j]);
        bad |= !(m <= 3.4028235e38f);
        amax = fmaxf(amax, m);
    }
    amax = fmaxf(amax, wh_dpp_quad_swap1(amax));
    amax = fmaxf(amax, wh_dpp_quad_swap2(amax));
    if (!(amax <= 3.4028235e38f)) amax = 1.0f;
    const int k = wh_aq_scale_exp(amax, thr);
    const float inv = wh_pow2f(-k), sc = wh_pow2f(k);
    float q[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] = wh_e4m3_round(wh_clamp448(v[j] * inv));
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
    if (bad && report_nonfinite) atomicOr(status, WH_ST_NONFINITE_INPUT);
    float4* d32 = (float4*)(q32 + base + 16 * t);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        d32[j] = make_float4(q[4 * j] * sc, q[4 * j + 1] * sc, q[4 * j + 2] * sc, q[4 * j + 3] * sc);
    const uint32_t g = t >> 1;  // 32-col group of the row
    *(uint4*)(q8 + base + 32 * g + 16 * h) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    if (!h) s8[(size_t)(on ? r : 0) * (n / 32) + g] = (uint8_t)(127 + k - 3);
}

// ------------------------------------------------------------ exact items
// An act-quantized vector (column order, n floats, n % 32 == 0) into LDS in
// FP4 lane order: one 32-col group per thread and pass.
__device__ __forceinline__ void wh_stage_xq_lanes(const float* __restrict__ src, uint32_t n, float* xs) {
    for (uint32_t g = threadIdx.x; g < n / 32; g += 256) {
        const float4* p = (const float4*)(src + 32 * g);
        float v[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 f = p[q];
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
        wh_stage_fp4_store_group(xs, g, v);
    }
}

// One dword of one lane (two groups) against two inputs: one decode, and
// each input keeps the reference chain of the single-input path.
__device__ __forceinline__ void wh_fp4_lane_pair2(uint32_t word, const float4* xg0, const float4* xg1, uint32_t ja,
                                                  uint32_t jb, float sa, float sb, bool two, float& acc0,
                                                  float& acc1) {
    const wh_fp4x8 e = wh_fp4_decode8(word);
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
        // each block's LDS reads are tied to the running sum, so they cannot
        // all be hoisted ahead of the arithmetic (which would spill)
#pragma unroll
        for (int b = 0; b < kBlk; ++b) {
            const uint32_t dep = wh_opaque_zero(acc0);
            wh_fp4_lane_block2(r.w[b], xp0 + dep, xp1 + dep, s8row + dep, b, two, acc0, acc1);
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
    if constexpr (kBlk > 0) {
        wh_s8_stage<kBlk> ss;
        wh_s8_stage_load<kBlk>(ss, srow, lane);
        wh_fp4_lane_row_load<kBlk>(r, wrow, lane);
        wh_s8_stage_store<kBlk>(ss, s8row, lane);
    } else {
        wh_s8_stage_rt(srow, G, s8row, lane);
    }
    for (uint32_t s = s_beg; s < s_end; s += 2) {
        const bool two = s + 1 < s_end;
        if (s != s_beg) __syncthreads();  // the previous pair is done with xs
        wh_stage_xq_lanes(in(s), cols, xs0);
        if (two) wh_stage_xq_lanes(in(s + 1), cols, xs1);
        __syncthreads();
        float acc0, acc1;
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
__device__ __forceinline__ void wh_mfma_a_load(wh_mfma_a& a, const uint8_t* wlane, const uint8_t* srow, uint32_t blk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) a.c[j] = *(const uint2*)(wlane + blk * 128 + j * 16);
    a.s = *(const uint2*)(srow + blk * 8);
}
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
        wl[i] = wmat[i] + (size_t)row * (cols / 2) + (4 * (g & 1)) * 16 + (g >> 1) * 8;
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
        wh_mfma_a ra[kMat], na[kMat];
        wh_mfma_b rb;
#pragma unroll
        for (int i = 0; i < kMat; ++i) wh_mfma_a_load(ra[i], wl[i], sr[i], 0);
        wh_mfma_b_load(rb, brec, bsrec, ton, 0);
        if (s0 != s_beg) __syncthreads();  // the previous pass is done with the LDS
        wh_mfma_b_store(rb, lds);
        __syncthreads();
        for (uint32_t blk = 0; blk < nblk; ++blk) {
            const bool more = blk + 1 < nblk;
            if (more) {
#pragma unroll
                for (int i = 0; i < kMat; ++i) wh_mfma_a_load(na[i], wl[i], sr[i], blk + 1);
                wh_mfma_b_load(rb, brec, bsrec, ton, blk + 1);
            }
            const uint8_t* buf = lds + (blk & 1) * WH_MFMA_BUF;
            const uint8_t* bsc = buf + WH_MFMA_TOK * WH_MFMA_TSTRIDE;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                wh_v8i av[kMat];
                uint32_t as[kMat];
#pragma unroll
                for (int i = 0; i < kMat; ++i) {
                    av[i] = u ? wh_mfma_a_codes<1>(ra[i]) : wh_mfma_a_codes<0>(ra[i]);
                    as[i] = u ? wh_mfma_sbyte<1>(ra[i].s, g) : wh_mfma_sbyte<0>(ra[i].s, g);
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

// Next item of a persistent workgroup's queue (counter zeroed by the pack).
__device__ __forceinline__ uint32_t wh_next_item(uint32_t* queue, uint32_t* item_s) {
    __syncthreads();  // the previous item is done with the LDS and item_s
    if (threadIdx.x == 0) *item_s = atomicAdd(queue, 1u);
    __syncthreads();
    return *item_s;
}

// Gate/up + SwiGLU, MFMA items: (expert, 64 rows of inter), w1 and w3 on the
// same rows, for the experts at the head of the work order.
__global__ void __launch_bounds__(256) k_moe_batch_gateup_mfma(wh_batch_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t item_s;
    const uint32_t mt = a.inter >> 6, n_items = a.meta[4] * mt;
    for (;;) {
        const uint32_t item = wh_next_item(a.meta + 5, &item_s);
        if (item >= n_items) break;
        const uint32_t u = a.uorder[item / mt], tile = item % mt;
        const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
        const uint8_t* wm[2] = {ep.w1, ep.w3};
        const uint8_t* sm[2] = {ep.s1, ep.s3};
        const uint32_t row0 = tile * 64;
        wh_mfma_item<2>(
            wm, sm, row0, a.hidden, a.uoff[u], a.uoff[u + 1], (uint8_t*)lds,
            [&](uint32_t s, const uint8_t*& rec, const uint8_t*& srec) {
                const uint32_t p = wh_slot_pos(a, a.sorted[s]);
                rec = a.xq8 + (size_t)p * a.hidden;
                srec = a.xs8 + (size_t)p * (a.hidden / 32);
            },
            [&](uint32_t s0, uint32_t count, const wh_v4f (&acc)[2][4]) {
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
                            const float gv = acc[0][nt][r] + 0.0f, uv = acc[1][nt][r] + 0.0f;
                            nf = nf || !(fabsf(gv) <= 3.4028235e38f) || !(fabsf(uv) <= 3.4028235e38f);
                            o[r] = wh_swiglu(gv, uv, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT);
                        }
                        float* hp = a.h + (size_t)(s0 + n) * a.inter + r0;
                        if (a.debug_raw) {
                            *(float4*)hp = make_float4(acc[0][nt][0], acc[0][nt][1], acc[0][nt][2], acc[0][nt][3]);
                            *(float4*)(a.hq + (size_t)(s0 + n) * a.inter + r0) =
                                make_float4(acc[1][nt][0], acc[1][nt][1], acc[1][nt][2], acc[1][nt][3]);
                        } else {
                            *(float4*)hp = make_float4(o[0], o[1], o[2], o[3]);
                        }
                    }
                }
                if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            });
    }
}

// Gate/up + SwiGLU, exact items: (expert, 16 rows of inter) for the experts
// after the MFMA ones; octet 2r runs the w1 row r of the tile and octet
// 2r + 1 the w3 row r.
template <int kBlk>
__global__ void __launch_bounds__(256) k_moe_batch_gateup(wh_batch_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t item_s;
    const uint32_t n_mfma = a.meta[4], et = a.inter >> 4, n_items = (a.meta[0] - n_mfma) * et;
    for (;;) {
        const uint32_t item = wh_next_item(a.meta + 2, &item_s);
        if (item >= n_items) break;
        const uint32_t u = a.uorder[n_mfma + item / et], tile = item % et;
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
                const float u0 = wh_dpp_row_shl8(v0), u1 = wh_dpp_row_shl8(v1);  // the w3 rows
                if ((threadIdx.x & 15) == 0) {
                    bool nf = !(fabsf(v0) <= 3.4028235e38f) || !(fabsf(u0) <= 3.4028235e38f);
                    if (a.debug_raw) {
                        a.h[(size_t)s * a.inter + row] = v0;
                        a.hq[(size_t)s * a.inter + row] = u0;
                    } else {
                        a.h[(size_t)s * a.inter + row] = wh_swiglu(v0, u0, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT);
                    }
                    if (two) {
                        nf = nf || !(fabsf(v1) <= 3.4028235e38f) || !(fabsf(u1) <= 3.4028235e38f);
                        if (a.debug_raw) {
                            a.h[(size_t)(s + 1) * a.inter + row] = v1;
                            a.hq[(size_t)(s + 1) * a.inter + row] = u1;
                        } else {
                            a.h[(size_t)(s + 1) * a.inter + row] =
                                wh_swiglu(v1, u1, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT);
                        }
                    }
                    if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
                }
            });
    }
}

// Down, MFMA items: (expert, 64 output rows); inputs are the act-quantized
// SwiGLU outputs of the slots.
__global__ void __launch_bounds__(256) k_moe_batch_down_mfma(wh_batch_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t item_s;
    const uint32_t mt = a.hidden >> 6, n_items = a.meta[4] * mt;
    for (;;) {
        const uint32_t item = wh_next_item(a.meta + 6, &item_s);
        if (item >= n_items) break;
        const uint32_t u = a.uorder[item / mt], tile = item % mt;
        const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
        const uint8_t* wm[1] = {ep.w2};
        const uint8_t* sm[1] = {ep.s2};
        const uint32_t row0 = tile * 64;
        wh_mfma_item<1>(
            wm, sm, row0, a.inter, a.uoff[u], a.uoff[u + 1], (uint8_t*)lds,
            [&](uint32_t s, const uint8_t*& rec, const uint8_t*& srec) {
                rec = a.hq8 + (size_t)s * a.inter;
                srec = a.hs8 + (size_t)s * (a.inter / 32);
            },
            [&](uint32_t s0, uint32_t count, const wh_v4f (&acc)[1][4]) {
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
                        *(float4*)(a.y + (size_t)(s0 + n) * a.hidden + r0) = make_float4(o[0], o[1], o[2], o[3]);
                    }
                }
                if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            });
    }
}

// Down, exact items: (expert, 32 output rows).
template <int kBlk>
__global__ void __launch_bounds__(256) k_moe_batch_down(wh_batch_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t item_s;
    const uint32_t n_mfma = a.meta[4], et = a.hidden >> 5, n_items = (a.meta[0] - n_mfma) * et;
    for (;;) {
        const uint32_t item = wh_next_item(a.meta + 3, &item_s);
        if (item >= n_items) break;
        const uint32_t u = a.uorder[n_mfma + item / et], tile = item % et;
        const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[u]);
        const uint32_t row = tile * 32 + (threadIdx.x >> 3);
        const uint32_t G = a.inter >> 5;
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
__global__ void __launch_bounds__(256) k_moe_batch_accumulate(wh_batch_args a) {
    const uint32_t p = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    if (r >= a.hidden || a.meta[1] == 0) return;
    float acc = 0.0f;
    for (uint32_t k = 0; k < a.topk; ++k) {
        const uint32_t s = a.acc_order[p * a.topk + k];
        const float v = a.y[(size_t)s * a.hidden + r] * a.wgt[a.sorted[s]];
        acc = acc + v;
    }
    if (a.has_shared) acc = a.y[(size_t)(a.npos * a.topk + p) * a.hidden + r] + acc;
    a.out[(size_t)p * a.hidden + r] = acc;
}
