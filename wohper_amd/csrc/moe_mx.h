// Routed-expert kernels for decode tokens on block-scaled FP8 MFMA (gfx950),
// the summation-order-free mode of the token entry points.
//
// The reference's expert forward (E/deepseek_v4.rs:551-601) act-quantizes x
// and h (block 64, power-of-two scales, E/compute.rs:2504-2521) before each
// FP4 matvec, so every product it forms is exact: an E4M3 code times an FP4
// LUT value.  These kernels feed the same exact operands to
// v_mfma_scale_f32_16x16x128_f8f6f4:
//   A = the weights as E4M3 codes of the reference's x8 LUT integers
//       {0, 1, 8, 12, 16, 24, 32, 48} (E/deepseek_v4.rs:285-287), two v_perm
//       lookups per resident dword, with the UE8M0 group scale as the E8M0
//       A scale;
//   B = the act-quantized input as E4M3 codes with the E8M0 byte
//       127 + k - 3 of the block scale 2^k (the -3 takes the x8 back out).
// Only the order of the fp32 sums differs from the CPU kernel, so every
// matvec stays within max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2 of it, and
// the dequantized weights are the reference's values exactly.  A decode
// token is one B column of the 16; the other columns are don't-cares (each
// C element depends only on its own row and column).
//
// Per resident FP4 weight the decode costs ~1.25 VALU instructions (the
// lane-chain kernels need ~2.6), so the kernels are bound by the weight
// stream, not by issue.
//
//   k_moe_gateup_mx: x act-quant (every workgroup redoes the token's 4096
//                    values: cheaper than a launch) + gate and up of 16 rows
//                    per workgroup + SwiGLU.  A token whose x holds an inf or
//                    NaN has no E4M3 code for the -480 a NaN quantizes to;
//                    its workgroups take an fp32 lane loop instead.
//   k_moe_down_mx:   act-quant of h while staging it + down of 32 rows per
//                    workgroup + the ordered routed sum (wh_moe_routed_sum).
#pragma once
#include "moe_batch.h"

#ifndef WH_MX_GU_DEPTH
#define WH_MX_GU_DEPTH 8  // 256-col blocks of a gate/up wave's row slice in flight
#endif

// The A blocks of a wave's 16 rows held in registers (a ring of kBlocks).
template <int kBlocks>
struct wh_mx_rows {
    wh_mx_raw a[kBlocks];
};
template <int kBlocks>
__device__ __forceinline__ void wh_mx_rows_load(wh_mx_rows<kBlocks>& r, const uint8_t* wlane, const uint8_t* srow) {
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) wh_mx_raw_load(r.a[b], wlane, srow, b);
}

// One 256-col block of A x B for the wave's 16 rows, into acc: xc are the
// input's codes of the block (32 B per 32-col group, byte 4c + k = column
// c + 8k of the group), xsb its 8 E8M0 bytes.
__device__ __forceinline__ void wh_mx_block(wh_v4f& acc, const wh_mfma_a& a, const uint8_t* xc, const uint8_t* xsb,
                                            uint32_t g) {
    const uint2 bs8 = *(const uint2*)xsb;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const wh_v8i av = u ? wh_mfma_a_codes<1>(a) : wh_mfma_a_codes<0>(a);
        const uint32_t as = u ? wh_mfma_sbyte<1>(a.s, g) : wh_mfma_sbyte<0>(a.s, g);
        const uint32_t bs = u ? wh_mfma_sbyte<1>(bs8, g) : wh_mfma_sbyte<0>(bs8, g);
        // lane group g: half 0 = group 4(g/2) + 2u of the block, half 1 = the next group
        const uint8_t* p = xc + (4 * (g >> 1) + 2 * u) * 32 + 16 * (g & 1);
        const uint4 lo = *(const uint4*)p, hi = *(const uint4*)(p + 32);
        const wh_v8i bv = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 0, 0, 0, (int)as, 0, (int)bs);
    }
}

// Sum over kBlocks blocks for the wave's 16 rows, the A blocks streaming
// through a ring of kDepth (the first kDepth were loaded by the caller into
// r.a[0 .. kDepth)); wlane / srow as for wh_mx_rows_load.  A refill's
// address depends on the accumulator of the block before it (an opaque
// zero), so the compiler cannot issue every block's loads up front, which
// would hold the whole row range in registers.
template <int kBlocks, int kDepth>
__device__ __forceinline__ wh_v4f wh_mx_dot(wh_mx_rows<kDepth>& r, const uint8_t* wlane, const uint8_t* srow,
                                            const uint8_t* xc, const uint8_t* xsb, uint32_t g) {
    wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // Block b is decoded only after block b - 1's MFMAs (block 0 after the
    // first LDS read of the input): its words pass through an opaque zero
    // tied to the running sum.  Hoisted decodes would make a wave wait for
    // several blocks' bytes before its first MFMA, and the slowest waves'
    // bytes arrive last; in order, each block's arithmetic overlaps the
    // arrival of the next.
    uint32_t dep = wh_opaque_zero(__uint_as_float(*(const uint32_t*)xsb));
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
        wh_mx_raw rb = r.a[b % kDepth];
        rb.p.x += dep;
        rb.p.y += dep;
        rb.q.x += dep;
        rb.q.y += dep;
        wh_mx_block(acc, wh_mx_fix(rb), xc + 256 * b, xsb + 8 * b, g);
        dep = wh_opaque_zero(acc[0]);
        if (b + kDepth < kBlocks) wh_mx_raw_load(r.a[b % kDepth], wlane + dep, srow + dep, b + kDepth);
    }
    // The MFMAs read every lane's A and B; the caller keeps only some lanes'
    // results, and the compiler would otherwise sink the last MFMAs into that
    // lane-conditional code, where the other lanes no longer take part.
    asm volatile("" : "+v"(acc));
    return acc;
}

// The 16 codes of a thread's act-quantized values q[0..16) at columns
// 16t' .. 16t' + 15 of a 32-col group (h = which half of the group) as the
// 16 bytes of the group's record that the thread and its partner lane
// (lane ^ 1, the other half) exchange: returns the record's half h.
__device__ __forceinline__ uint4 wh_mx_codes16(const float (&q)[16], uint32_t h) {
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
    return make_uint4(dw[0], dw[1], dw[2], dw[3]);
}

// Fallback of a gate/up wave for a token with a non-finite input: its 16
// rows over its kCols/kSl-column slice in fp32 from the dequantized x in
// LDS (xf, column order).  Lane L: row L % 16, a quarter of the slice.
// Returns the row sum in lanes 0..15.
__device__ __forceinline__ float wh_mx_rows_fp32(const uint8_t* wrow, const uint8_t* srow, const float* xf,
                                                 uint32_t blk0, uint32_t nblk, uint32_t L) {
    const uint32_t quarter = L >> 4, per = nblk / 4;
    float acc = 0.0f;
    for (uint32_t b = blk0 + quarter * per; b < blk0 + (quarter + 1) * per; ++b) {
        for (uint32_t c = 0; c < 8; ++c) {
            const uint4 wv = *(const uint4*)(wrow + b * 128 + c * 16);
            const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (uint32_t d = 0; d < 4; ++d) {
                const wh_fp4x8 e = wh_fp4_decode8(words[d]);
                const uint32_t ga = 8 * b + 2 * d;
                const float* xa = xf + 32 * ga + c;
                const float* xb = xa + 32;
                float sa = xa[0] * e.a01.x;
                sa = __builtin_fmaf(xa[8], e.a01.y, sa);
                sa = __builtin_fmaf(xa[16], e.a23.x, sa);
                sa = __builtin_fmaf(xa[24], e.a23.y, sa);
                float sb = xb[0] * e.b01.x;
                sb = __builtin_fmaf(xb[8], e.b01.y, sb);
                sb = __builtin_fmaf(xb[16], e.b23.x, sb);
                sb = __builtin_fmaf(xb[24], e.b23.y, sb);
                acc = __builtin_fmaf(sa, wh_ue8m0(srow[ga]) * 0.125f, acc);
                acc = __builtin_fmaf(sb, wh_ue8m0(srow[ga + 1]) * 0.125f, acc);
            }
        }
    }
    acc += __shfl_xor(acc, 16, 64);
    acc += __shfl_xor(acc, 32, 64);
    return acc;
}

// Gate/up + SwiGLU, hidden = 2048 * kSl, inter rows in tiles of 16:
// grid (n_experts * inter / 16, n_tokens), 128 * kSl threads.  Wave
// (m, s) = (wave / kSl, wave % kSl) runs the tile's 16 rows of w1 (m = 0) or
// w3 (m = 1) over column slice s (2048 columns = 8 blocks of 256).
template <int kSl>
__global__ void __launch_bounds__(128 * kSl, 3) k_moe_gateup_mx(wh_moe_args a) {
    constexpr uint32_t kCols = 2048 * kSl, kG = kCols / 32, kWaves = 2 * kSl;
    __shared__ __align__(16) uint8_t xc[kCols];  // codes, 32 B per group
    __shared__ __align__(16) uint8_t xsb[kG];    // E8M0 byte per group
    __shared__ float red[kWaves * 16];
    __shared__ uint32_t thr[256];
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    __shared__ __align__(16) float xf[kCols];    // the dequantized x, non-finite tokens only
    const uint32_t tok = blockIdx.y;
    wh_moe_clear_arrivals(a, tok);
    const uint32_t per_e = a.inter >> 4;
    const uint32_t e = blockIdx.x / per_e;
    const uint32_t row0 = (blockIdx.x - e * per_e) * 16;
    const uint32_t wave = threadIdx.x >> 6, L = threadIdx.x & 63;
    const uint32_t m = wave / kSl, s = wave - m * kSl, g = L >> 4;
    const wh_expert_ptrs ep = a.ex[e];
    const uint8_t* wrow = (m ? ep.w3 : ep.w1) + (size_t)(row0 + (L & 15)) * (kCols / 2);
    const uint8_t* srow = (m ? ep.s3 : ep.s1) + (size_t)(row0 + (L & 15)) * kG;
    const bool bf16 = a.x_is_bf16 != 0;
    const void* xt = bf16 ? (const void*)((const uint16_t*)a.x + (size_t)tok * kCols)
                          : (const void*)((const float*)a.x + (size_t)tok * kCols);
    // staging loads (x, the tables) go out before the weight rows, so
    // waiting for them never waits for weight bytes
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_exp_stage es;
    wh_exp_stage_load(es);
    wh_xq_stage xst;
    wh_xq_stage_load(xst, xt, bf16, kCols, threadIdx.x);
    constexpr int kDepth = WH_MX_GU_DEPTH;
    const uint8_t* wlane = wrow + 1024 * s + 64 * (g & 1) + 32 * (g >> 1);
    wh_mx_rows<kDepth> rows;
    wh_mx_rows_load<kDepth>(rows, wlane, srow + 64 * s);
    __builtin_amdgcn_sched_barrier(0);
    wh_thr_stage_store(ts, thr);
    wh_exp_stage_store(es, exp_tab);
    __syncthreads();
    // act-quant of x (E/compute.rs:2504-2521): 16 columns per thread
    float q[16], sc = 1.0f;
    bool bad = false;
    wh_xq_quant16(xst, bf16, thr, q, sc, &bad);
    const uint32_t c0 = 16 * threadIdx.x, h = threadIdx.x & 1;
    const uint4 rec = wh_mx_codes16(q, h);
    *(uint4*)(xc + c0) = rec;  // group c0 / 32, half h: bytes 32 (c0 / 32) + 16 h = c0
    if (!h) xsb[c0 >> 5] = (uint8_t)(((__float_as_uint(sc) >> 23) & 0xffu) - 3u);
    if (__syncthreads_or(bad)) {
        // -480 (a NaN's value) and an infinite scale have no E4M3 / E8M0
        // code: this token's rows run in fp32 from the dequantized x
#pragma unroll
        for (int j = 0; j < 16; ++j) xf[c0 + j] = q[j] * sc;
        __syncthreads();
        const float v = wh_mx_rows_fp32(wrow, srow, xf, 8 * s, 8, L);
        if (L < 16) red[wave * 16 + L] = v;
    } else {
        const wh_v4f acc = wh_mx_dot<8, kDepth>(rows, wlane, srow + 64 * s, xc + 2048 * s, xsb + 64 * s, g);
        // C[4 (L / 16) + r][L % 16]: column 0 is the token
        if ((L & 15) == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave * 16 + 4 * g + r] = acc[r];
        }
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const uint32_t r = threadIdx.x;
        float gv = red[r], uv = red[kSl * 16 + r];
#pragma unroll
        for (int k = 1; k < kSl; ++k) {
            gv += red[k * 16 + r];
            uv += red[(kSl + k) * 16 + r];
        }
        if (!(fabsf(gv) <= 3.4028235e38f) || !(fabsf(uv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        const size_t he = ((size_t)tok * a.n_experts + e) * a.inter;
        a.h[he + row0 + r] = wh_swiglu(gv, uv, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT);
        if (a.gu) {
            a.gu[2 * he + row0 + r] = gv;
            a.gu[2 * he + a.inter + row0 + r] = uv;
        }
    }
}

// Down + ordered routed sum, inter = 2048: grid (n_experts * hidden / 32,
// n_tokens), 256 threads.  Wave w runs 16 of the workgroup's 32 output rows
// (w & 1) over half of the 2048 columns (w >> 1); the act-quant of h
// (E/deepseek_v4.rs:595) is redone by every workgroup while staging it.
__global__ void __launch_bounds__(256, 4) k_moe_down_mx(wh_moe_args a) {
    constexpr uint32_t kCols = 2048, kG = kCols / 32;
    __shared__ __align__(16) uint8_t hc[kCols];
    __shared__ __align__(16) uint8_t hsb[kG];
    __shared__ float red[4 * 16];
    __shared__ uint32_t thr[256];
    __shared__ uint32_t last;
    const uint32_t tok = blockIdx.y;
    const uint32_t per_e = a.hidden >> 5;
    const uint32_t e = blockIdx.x / per_e;
    const uint32_t rb = blockIdx.x - e * per_e;  // 32-row slice of the output
    const uint32_t wave = threadIdx.x >> 6, L = threadIdx.x & 63, g = L >> 4;
    const uint32_t rt = wave & 1, kh = wave >> 1;
    const uint32_t row = rb * 32 + rt * 16 + (L & 15);
    const wh_expert_ptrs ep = a.ex[e];
    const float* hrow = a.h + ((size_t)tok * a.n_experts + e) * kCols;
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_h_stage hst;
    wh_h_stage_load(hst, hrow, kCols, threadIdx.x);  // 8 values per thread
    const uint8_t* wlane = ep.w2 + (size_t)row * (kCols / 2) + 512 * kh + 64 * (g & 1) + 32 * (g >> 1);
    const uint8_t* srow = ep.s2 + (size_t)row * kG + 32 * kh;
    wh_mx_rows<4> rows;
    wh_mx_rows_load<4>(rows, wlane, srow);
    __builtin_amdgcn_sched_barrier(0);
    wh_thr_stage_store(ts, thr);
    __syncthreads();
    {
        // act-quant of h, block 64 = 8 threads; codes into the group records
        const float v[8] = {hst.p.x, hst.p.y, hst.p.z, hst.p.w, hst.q.x, hst.q.y, hst.q.z, hst.q.w};
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
        amax = fmaxf(amax, wh_dpp_quad_swap1(amax));
        amax = fmaxf(amax, wh_dpp_quad_swap2(amax));
        const float lo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x104, 0xf, 0xf, false));
        const float hi = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x114, 0xf, 0xf, false));
        amax = fmaxf(amax, (threadIdx.x & 4) ? hi : lo);  // the other quad of the 64-block
        // h is finite whenever gate/up was (a non-finite gate/up output is
        // already reported); keep the arithmetic in range regardless
        if (!(amax <= 3.4028235e38f)) amax = 1.0f;
        const int k = wh_aq_scale_exp(amax, thr);
        const float inv = wh_pow2f(-k);
        // thread t holds columns 8t + j of group t / 4 at in-group column
        // 8 (t % 4) + j: record byte 4 j + t % 4
        uint8_t* grp = hc + 32 * (threadIdx.x >> 2) + (threadIdx.x & 3);
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const uint32_t two = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                wh_e4m3_round(wh_clamp448_finite(v[j] * inv)), wh_e4m3_round(wh_clamp448_finite(v[j + 1] * inv)), 0,
                false);
            grp[4 * j] = (uint8_t)two;
            grp[4 * j + 4] = (uint8_t)(two >> 8);
        }
        if ((threadIdx.x & 3) == 0) hsb[threadIdx.x >> 2] = (uint8_t)(127 + k - 3);
    }
    __syncthreads();
    const wh_v4f acc = wh_mx_dot<4, 4>(rows, wlane, srow, hc + 1024 * kh, hsb + 32 * kh, g);
    if ((L & 15) == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * 16 + 4 * g + r] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        // rows r of tile t: waves t (columns 0..1023) and t + 2 (1024..2047)
        const uint32_t t = threadIdx.x >> 4, r = threadIdx.x & 15;
        const float yv = red[t * 16 + r] + red[(t + 2) * 16 + r];
        if (!(fabsf(yv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        wh_store_coherent(a.y + ((size_t)tok * a.n_experts + e) * a.hidden + rb * 32 + threadIdx.x, yv);
    }
    wh_moe_routed_sum(a, tok, rb, &last);
}
