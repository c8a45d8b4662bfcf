// Persistent routed-expert kernels for decode tokens on block-scaled FP8 MFMA
// (gfx950): the summation-order-free mode of the token entry points.
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
// A per-wave timeline of the one-tile-per-workgroup kernels (768 workgroups,
// 3 per CU) showed each wave spending its time in series on staging x,
// act-quantizing it (every workgroup redoes all 4096 values) and only then
// the dot, and the down kernel paying the same for h plus a cross-workgroup
// routed sum.  Two facts of the hardware shape the kernels here:
//   * a CU's memory loads complete in issue order, so a small load issued
//     after a wave of weight loads waits for all of them;
//   * while the memory system is saturated a wave cannot issue a load until
//     earlier requests drain, so a wave that requests all of its weight
//     blocks before some arithmetic reaches that arithmetic late.
// Hence one workgroup of 8 waves per CU (about), staging loads first, only
// WH_PX_PRO weight blocks per wave requested before the staged input is
// act-quantized once per workgroup, and then a ring of register blocks:
//   k_moe_gateup_px: row tiles kTiles*b .. kTiles*b + kTiles - 1 (16 rows of
//                    w1 and w3 of one expert each); wave (m, s) runs matrix m
//                    (w1, w3) over 1024-column slice s of every tile.
//   k_moe_down_px:   output rows 16b .. 16b + 15 of every expert, so the
//                    routed sum stays in the workgroup; wave w runs (expert,
//                    512-column quarter) units w, w + 8, ...
#pragma once
#include "moe_batch.h"

#ifndef WH_PX_GU_DEPTH
#define WH_PX_GU_DEPTH 4  // weight blocks of a gate/up wave in flight
#endif
#ifndef WH_PX_DN_DEPTH
#define WH_PX_DN_DEPTH 4  // weight blocks of a down wave in flight
#endif
// Weight blocks a wave requests before the workgroup's staged input is in
// LDS; the rest of its ring goes out after the act-quant.
#ifndef WH_PX_PRO
#define WH_PX_PRO 2
#endif
// The same for the down kernel, whose act-quant covers only the wave's own
// units.
#ifndef WH_PX_DN_PRO
#define WH_PX_DN_PRO 2
#endif

// Optional per-wave timeline of the two kernels (build with -DWH_TIMELINE):
// lane 0 of each wave stores the 100 MHz realtime counter at fixed points of
// the kernel into wh_tl_buf[kernel][(workgroup * 16 + wave) * 16 + point],
// for the first 512 workgroups of token 0; wh_debug_timeline reads it back.
// WH_TL_USE(v) makes the wave wait for a loaded value before the next stamp.
#ifdef WH_TIMELINE
#define WH_TL_POINTS 16
__device__ uint64_t wh_tl_buf[2][512 * 16 * WH_TL_POINTS];
#define WH_TL(kern, k)                                                                                    \
    do {                                                                                                  \
        if ((threadIdx.x & 63) == 0 && blockIdx.x < 512 && blockIdx.y == 0 && (threadIdx.x >> 6) < 16)     \
            wh_tl_buf[kern][((size_t)blockIdx.x * 16 + (threadIdx.x >> 6)) * WH_TL_POINTS + (k)] =         \
                __builtin_amdgcn_s_memrealtime();                                                         \
    } while (0)
#define WH_TL_USE(v) asm volatile("" ::"v"(v))
#else
#define WH_TL_USE(v) \
    do {             \
    } while (0)
#define WH_TL(kern, k) \
    do {               \
    } while (0)
#endif

// An execution barrier (no memory fence): every wave of the workgroup has
// issued its loads up to here before any wave issues the next one.
__device__ __forceinline__ void wh_issue_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// The B operands of one 256-col block of an input in the record layout (32
// code bytes per 32-col group, byte 4j + k = column j + 8k of the group; one
// E8M0 byte per group) in registers: lane group g's half h of MFMA u holds
// the codes of group 4 (g / 2) + 2u + h, bytes 16 (g % 2) .. + 15.
struct wh_mx_bop {
    wh_v8i v[2];
    uint32_t s[2];
};
__device__ __forceinline__ void wh_mx_bop_load(wh_mx_bop& b, const uint8_t* xc, const uint8_t* xsb, uint32_t g) {
    const uint2 bs8 = *(const uint2*)xsb;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint8_t* p = xc + (4 * (g >> 1) + 2 * u) * 32 + 16 * (g & 1);
        const uint4 lo = *(const uint4*)p, hi = *(const uint4*)(p + 32);
        b.v[u] = wh_v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        b.s[u] = u ? wh_mfma_sbyte<1>(bs8, g) : wh_mfma_sbyte<0>(bs8, g);
    }
}
// One block of a ring: the weights in r against the B operands bo.  The
// block's words pass through an opaque zero (dep) tied to the previous
// block's accumulator, so the decode of block b starts after block b - 1's
// MFMAs: hoisted decodes would make a wave wait for several blocks' bytes
// before its first MFMA, and would hold them all in registers.
__device__ __forceinline__ void wh_px_step(wh_v4f& acc, const wh_mx_raw& r, uint32_t& dep, const wh_mx_bop& bo,
                                           uint32_t g) {
    wh_mx_raw rb = r;
    rb.p.x += dep;
    rb.p.y += dep;
    rb.q.x += dep;
    rb.q.y += dep;
    const wh_mfma_a a = wh_mx_fix(rb);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const wh_v8i av = u ? wh_mfma_a_codes<1>(a) : wh_mfma_a_codes<0>(a);
        const uint32_t as = u ? wh_mfma_sbyte<1>(a.s, g) : wh_mfma_sbyte<0>(a.s, g);
        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bo.v[u], acc, 0, 0, 0, (int)as, 0, (int)bo.s[u]);
    }
    dep = wh_opaque_zero(acc[0]);
}

// 8 consecutive input values of one thread, bf16 or f32.
struct wh_in8 {
    uint4 r0, r1;
};
__device__ __forceinline__ void wh_in8_load(wh_in8& st, const void* x, bool bf16, uint32_t c) {
    if (bf16) {
        st.r0 = ((const uint4*)x)[c];
        st.r1 = make_uint4(0, 0, 0, 0);
    } else {
        st.r0 = ((const uint4*)x)[2 * c];
        st.r1 = ((const uint4*)x)[2 * c + 1];
    }
}
__device__ __forceinline__ void wh_in8_values(const wh_in8& st, bool bf16, float (&v)[8]) {
    const uint32_t w[4] = {st.r0.x, st.r0.y, st.r0.z, st.r0.w};
    if (bf16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    } else {
        const uint32_t u[4] = {st.r1.x, st.r1.y, st.r1.z, st.r1.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = __uint_as_float(w[i]);
            v[4 + i] = __uint_as_float(u[i]);
        }
    }
}

// Stores the codes of the 8 values at columns 8c .. 8c + 7 into a record
// array and, for the first chunk of a group, its E8M0 byte 127 + k - 3 (the
// -3 takes back the x8 of the weights' integer codes).
__device__ __forceinline__ void wh_px_store_codes8(uint8_t* rec, uint8_t* sb, uint32_t c, const float (&q)[8], int k) {
    uint8_t* grp = rec + 32 * (c >> 2) + (c & 3);  // column 8c + j: byte 4j + c % 4 of group c / 4
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const uint32_t two = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[j], q[j + 1], 0, false);
        grp[4 * j] = (uint8_t)two;
        grp[4 * j + 4] = (uint8_t)(two >> 8);
    }
    if ((c & 3) == 0) sb[c >> 2] = (uint8_t)(127 + k - 3);
}

// The amax of a 64-block held as 8 values by each of 8 consecutive lanes,
// and its act-quant scale exponent k (E/compute.rs:2504-2521); bad: a
// non-finite value in the thread's 8.  The maxima run on the magnitudes'
// bit patterns (ordered as integers for non-negative floats), so the DPP
// moves fold into the integer max; a block holding inf or NaN takes amax 1
// (its values are reported as non-finite and not used).
__device__ __forceinline__ int wh_quant8_scale(const float (&v)[8], bool& bad) {
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = max(m, __float_as_uint(v[i]) & 0x7fffffffu);
    bad = m > 0x7f7fffffu;
    m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0xb1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
    m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x4e, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
    m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x141, 0xf, 0xf, false));  // row_half_mirror
    const float amax = m > 0x7f7fffffu ? 1.0f : __uint_as_float(m);
    return wh_aq_scale_exp_fast(amax);
}

// E4M3 codes of 8 finite f32 values under the block exponent k
// (wh_e4m3_code_pow2 for |v / 2^k| <= 448): every value takes the
// normal-range formula, and the whole of wh_e4m3_code_pow2 (the subnormal
// grid below 2^(k - 6) and the select) runs only when some lane of the wave
// holds a value under 2^(k - 6); where no value is that small the two agree.
// A zero keeps its sign (0x80 for -0; the MFMA takes it as 0).
__device__ __forceinline__ void wh_quant8_f32_codes(const float (&v)[8], int k, uint32_t (&c)[8]) {
    uint32_t K = 0x7ffffu - ((uint32_t)(960 + 8 * k) << 20);
    asm volatile("" : "+v"(K));  // one constant per block: a + K + sign is then one add3
    const uint32_t lim = (uint32_t)(121 + k) << 23;
    uint32_t amin = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < 8; ++i) amin = min(amin, __float_as_uint(v[i]) & 0x7fffffffu);
    if (__builtin_amdgcn_ballot_w64(amin < lim) != 0) {  // wave-uniform
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = wh_e4m3_code_pow2(v[i], k);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t b = __float_as_uint(v[i]), sg = b >> 31;
            c[i] = (((b & 0x7fffffffu) + K + sg) >> 20) | (sg << 7);
        }
    }
}

// Act-quant of 8 values held by one thread into the record layout: the
// thread owns record dwords 2q and 2q + 1 of 32-col group G (q = t % 4,
// G = t / 4), i.e. v[2k] = column 2q + 8k, v[2k + 1] = column 2q + 1 + 8k
// (k = 0..3); the 64-block is the 8 lanes t & ~7 .. + 7.  Returns the two
// code dwords and the block's scale exponent; bad: a non-finite value.
template <bool kBf16>
__device__ __forceinline__ void wh_tok_quant8(const float (&v)[8], uint32_t& d0, uint32_t& d1, int& k, bool& bad) {
    k = wh_quant8_scale(v, bad);
    if constexpr (kBf16) {
        const float inv = wh_pow2f(-k);
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float s = v[i] * inv;
            t[i] = __builtin_fmaf(-fabsf(s), 2.44140625e-4f, s);  // s - |s| 2^-12: ties toward -inf
        }
        d0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(t[0], t[2], 0, false);
        d0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(t[4], t[6], (int)d0, true);
        d1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(t[1], t[3], 0, false);
        d1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(t[5], t[7], (int)d1, true);
    } else {
        uint32_t c[8];
        wh_quant8_f32_codes(v, k, c);
        d0 = c[0] | (c[2] << 8) | (c[4] << 16) | (c[6] << 24);
        d1 = c[1] | (c[3] << 8) | (c[5] << 16) | (c[7] << 24);
    }
}

// fp32 fallback of a gate/up wave for a token with a non-finite input: its
// 16 rows over kB blocks of 256 columns from block blk0, from the dequantized
// x in LDS (xf, column order); lane group q = L / 16 takes the AVX lanes
// (16-byte chunks) 2q and 2q + 1 of each block.  Returns the row sums in
// lanes 0..15.
__device__ __forceinline__ float wh_px_rows_fp32(const uint8_t* wrow, const uint8_t* srow, const float* xf,
                                                 uint32_t blk0, uint32_t kB, uint32_t L) {
    const uint32_t qd = L >> 4;
    float acc = 0.0f;
    // rolled loops: this path must not raise the kernel's register count
#pragma unroll 1
    for (uint32_t b = blk0; b < blk0 + kB; ++b) {
#pragma unroll 1
        for (uint32_t c = 2 * qd; c < 2 * qd + 2; ++c) {
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

// Gate/up + SwiGLU, hidden = kCols (2048 or 4096), inter % 16 == 0: grid
// (ceil(n_experts * inter / 16 / kTiles), n_tokens), kCols / 8 threads.
template <int kCols, int kTiles>
__global__ void __launch_bounds__(kCols / 8, 1) k_moe_gateup_px(wh_moe_args a) {
    constexpr uint32_t kG = kCols / 32, kSl = kCols / 1024, kWaves = 2 * kSl, kB = 4;
    constexpr int kJ = kB * kTiles, kDepth = WH_PX_GU_DEPTH < kJ ? WH_PX_GU_DEPTH : kJ;
    constexpr int kPro = WH_PX_PRO < kDepth ? WH_PX_PRO : kDepth;
    __shared__ __align__(16) uint8_t xc[kCols];  // codes, 32 B per group
    __shared__ __align__(16) uint8_t xsb[kG];    // E8M0 byte per group
    __shared__ float red[kTiles * kWaves * 16];
    __shared__ uint32_t thr[256];
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    __shared__ __align__(16) float xf[kCols];  // the dequantized x (non-finite tokens only)
    WH_TL(0, 0);
    const uint32_t tok = blockIdx.y;
    wh_moe_clear_arrivals(a, tok);
    const uint32_t per_e = a.inter >> 4, n_tiles = a.n_experts * per_e;
    const uint32_t tile0 = blockIdx.x * kTiles;
    const uint32_t nt = n_tiles - tile0 < (uint32_t)kTiles ? n_tiles - tile0 : (uint32_t)kTiles;
    const uint32_t wave = threadIdx.x >> 6, L = threadIdx.x & 63, g = L >> 4;
    const uint32_t m = wave / kSl, s = wave - m * kSl;
    const bool bf16 = a.x_is_bf16 != 0;
    const void* xt = bf16 ? (const void*)((const uint16_t*)a.x + (size_t)tok * kCols)
                          : (const void*)((const float*)a.x + (size_t)tok * kCols);
    // staging loads (x, the tables) go out before any weight load of the CU
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_exp_stage es;
    wh_exp_stage_load(es);
    wh_in8 xin;
    wh_in8_load(xin, xt, bf16, threadIdx.x);
    // the rows of the workgroup's tiles (a tile past the end repeats the
    // last one; its results are not stored)
    const uint8_t* wrow[kTiles];
    const uint8_t* srow[kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
        const uint32_t t = tile0 + ((uint32_t)i < nt ? (uint32_t)i : nt - 1);
        const uint32_t e = t / per_e, row = (t - e * per_e) * 16 + (L & 15);
        const wh_expert_ptrs ep = wh_moe_ex(a, e);
        wrow[i] = (m ? ep.w3 : ep.w1) + (size_t)row * (kCols / 2);
        srow[i] = (m ? ep.s3 : ep.s1) + (size_t)row * kG + 32 * s;
    }
    const uint32_t lane_off = 512 * s + 64 * (g & 1) + 32 * (g >> 1);
    wh_issue_barrier();
    wh_mx_raw ring[kDepth];
#pragma unroll
    for (int j = 0; j < kPro; ++j) wh_mx_raw_load(ring[j], wrow[j / kB] + lane_off, srow[j / kB], j % kB);
    __builtin_amdgcn_sched_barrier(0);
    wh_thr_stage_store(ts, thr);
    wh_exp_stage_store(es, exp_tab);
    __syncthreads();
    WH_TL(0, 1);
    WH_TL_USE(xin.r0.x);
    WH_TL_USE(xin.r1.w);
    WH_TL(0, 2);
    // act-quant of x (E/compute.rs:2504-2521): columns 8t .. 8t + 7
    float v[8], q[8], sc;
    int k;
    bool bad;
    wh_in8_values(xin, bf16, v);
    wh_aq_vals<8>(v, thr, q, k, sc, bad);
    wh_px_store_codes8(xc, xsb, threadIdx.x, q, k);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(0, 3);
#pragma unroll
    for (int j = kPro; j < kDepth; ++j) wh_mx_raw_load(ring[j], wrow[j / kB] + lane_off, srow[j / kB], j % kB);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(0, 4);
    if (__syncthreads_or(bad)) {
        // -480 (a NaN's value) and an infinite scale have no E4M3 / E8M0
        // code: this token's rows run in fp32 from the dequantized x
#pragma unroll
        for (int j = 0; j < 8; ++j) xf[8 * threadIdx.x + j] = q[j] * sc;
        __syncthreads();
#pragma unroll 1
        for (uint32_t i = 0; i < nt; ++i) {
            const float r = wh_px_rows_fp32(wrow[i], srow[i] - 32 * s, xf, kB * s, kB, L);
            if (L < 16) red[(i * kWaves + wave) * 16 + L] = r;
        }
    } else {
        WH_TL(0, 5);
        uint32_t dep = wh_opaque_zero(__uint_as_float(*(const uint32_t*)xsb));
        wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const int b = j % kB, i = j / kB;
            // the input's operands of the block, read after the previous
            // block's MFMAs (dep) so that they are not all held at once
            wh_mx_bop bo;
            wh_mx_bop_load(bo, xc + 1024 * s + 256 * b + dep, xsb + 32 * s + 8 * b + dep, g);
            wh_px_step(acc, ring[j % kDepth], dep, bo, g);
            if (j + kDepth < kJ)
                wh_mx_raw_load(ring[j % kDepth], wrow[(j + kDepth) / kB] + lane_off + dep,
                               srow[(j + kDepth) / kB] + dep, (j + kDepth) % kB);
            if (b == kB - 1) {
                // every lane's A and B feed the MFMAs: keep them out of the
                // lane-conditional store below
                asm volatile("" : "+v"(acc));
                if ((L & 15) == 0) {  // C[4 (L / 16) + r][0]: column 0 is the token
#pragma unroll
                    for (int r = 0; r < 4; ++r) red[(i * kWaves + wave) * 16 + 4 * g + r] = acc[r];
                }
                acc = wh_v4f{0.0f, 0.0f, 0.0f, 0.0f};
                if (i < 4) WH_TL(0, 6 + i);
            }
        }
    }
    __syncthreads();
    WH_TL(0, 10);
    // SwiGLU of the tiles' rows, thread t: tile t / 16, row t % 16
    if (threadIdx.x < nt * 16) {
        const uint32_t i = threadIdx.x >> 4, r = threadIdx.x & 15;
        const float* ri = red + i * kWaves * 16 + r;
        float gv = ri[0], uv = ri[kSl * 16];
#pragma unroll
        for (uint32_t sl = 1; sl < kSl; ++sl) {
            gv += ri[sl * 16];
            uv += ri[(kSl + sl) * 16];
        }
        if (!(fabsf(gv) <= 3.4028235e38f) || !(fabsf(uv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        const uint32_t t = tile0 + i, e = t / per_e, row = (t - e * per_e) * 16 + r;
        const size_t he = ((size_t)tok * a.n_experts + e) * a.inter;
        a.h[he + row] = wh_swiglu(gv, uv, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT);
        if (a.gu) {
            a.gu[2 * he + row] = gv;
            a.gu[2 * he + a.inter + row] = uv;
        }
    }
    WH_TL(0, 11);
}


// Down + routed sum for an odd number of experts kN, inter = 2048: grid
// (hidden / 16, n_tokens), 512 threads.  The workgroup's 16 output rows
// are 8 kN blocks of 256 columns; wave w takes the blocks of columns
// [256 w, 256 w + 256) of every expert, kN blocks, so no wave runs a block
// more than another (unit pairs of two blocks would leave four waves one
// unit longer).  Wave w act-quantizes exactly those h values (two experts'
// slices per 8-value chunk of its lanes), and the blocks' partial outputs
// meet in LDS, summed per expert in block order (k_moe_down_px chains each
// unit's two blocks in its MFMA accumulator instead: the same products, the
// sums rounded in another order).
template <int kN>
__global__ void __launch_bounds__(512, 1) k_moe_down_pb(wh_moe_args a) {
    constexpr uint32_t kCols = 2048, kG = kCols / 32;
    constexpr int kJ = kN, kDepth = WH_PX_DN_DEPTH < kJ ? WH_PX_DN_DEPTH : kJ;
    constexpr int kPro = WH_PX_DN_PRO < kDepth ? WH_PX_DN_PRO : kDepth;
    constexpr int kCh = (kN + 1) / 2;  // 8-value chunks of h per lane
    __shared__ __align__(16) uint8_t hc[kN * kCols];
    __shared__ __align__(16) uint8_t hsb[kN * kG];
    __shared__ float red[kN * 8 * 16];
    WH_TL(1, 0);
    const uint32_t tok = blockIdx.y;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), L = threadIdx.x & 63, g = L >> 4;
    const uint32_t row = blockIdx.x * 16 + (L & 15);
    const uint32_t qt = wave >> 1, b = wave & 1;
    const float* htok = a.h + (size_t)tok * kN * kCols;
    // chunk i of lane L: columns 256 w + 8 (L % 32) .. + 7 of expert
    // 2 i + L / 32 (the last expert's when past the end; not stored)
    float4 hv[kCh][2];
#pragma unroll
    for (int i = 0; i < kCh; ++i) {
        const uint32_t e = 2 * i + (L >> 5);
        const float4* hp = (const float4*)(htok + (size_t)(e < (uint32_t)kN ? e : kN - 1) * kCols + 256 * wave +
                                           8 * (L & 31));
        hv[i][0] = hp[0];
        hv[i][1] = hp[1];
    }
    const uint8_t* wl[kJ];
    const uint8_t* sr[kJ];
#pragma unroll
    for (int e = 0; e < kJ; ++e) {
        const wh_expert_ptrs ep = wh_moe_ex(a, e);
        wl[e] = ep.w2 + (size_t)row * (kCols / 2) + 256 * qt + 64 * (g & 1) + 32 * (g >> 1);
        sr[e] = ep.s2 + (size_t)row * kG + 16 * qt;
    }
    wh_issue_barrier();
    wh_mx_raw ring[kDepth];
#pragma unroll
    for (int j = 0; j < kPro; ++j) wh_mx_raw_load(ring[j], wl[j], sr[j], b);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(1, 1);
    WH_TL(1, 2);
    // act-quant of h (as k_moe_down_px): the wave reads back only codes it
    // wrote itself, so no workgroup barrier is needed
    auto quant_chunk = [&](int i) {
        const uint32_t e = 2 * i + (L >> 5), idx = 32 * wave + (L & 31);
        const float v[8] = {hv[i][0].x, hv[i][0].y, hv[i][0].z, hv[i][0].w,
                            hv[i][1].x, hv[i][1].y, hv[i][1].z, hv[i][1].w};
        bool bad;
        const int k = wh_quant8_scale(v, bad);
        uint32_t cd[8];
        wh_quant8_f32_codes(v, k, cd);
        if (e < (uint32_t)kN) {
            uint8_t* grp = hc + kCols * e + 32 * (idx >> 2) + (idx & 3);
#pragma unroll
            for (int j = 0; j < 8; ++j) grp[4 * j] = (uint8_t)cd[j];
            if ((idx & 3) == 0) hsb[kG * e + (idx >> 2)] = (uint8_t)(127 + k - 3);
        }
        asm volatile("" ::: "memory");
    };
#pragma unroll
    for (int i = 0; i < kCh; ++i) quant_chunk(i);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(1, 3);
#pragma unroll
    for (int j = kPro; j < kDepth; ++j) wh_mx_raw_load(ring[j], wl[j], sr[j], b);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(1, 4);
    WH_TL(1, 5);
    {
        uint32_t dep = wh_opaque_zero(__uint_as_float(*(const uint32_t*)hsb));
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
            wh_mx_bop bo;
            wh_mx_bop_load(bo, hc + kCols * j + 256 * wave + dep, hsb + kG * j + 8 * wave + dep, g);
            wh_px_step(acc, ring[j % kDepth], dep, bo, g);
            if (j + kDepth < kJ) wh_mx_raw_load(ring[j % kDepth], wl[j + kDepth] + dep, sr[j + kDepth] + dep, b);
            asm volatile("" : "+v"(acc));
            if ((L & 15) == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) red[(8 * j + wave) * 16 + 4 * g + r] = acc[r];
            }
            if (j < 4) WH_TL(1, 6 + j);
        }
    }
    __syncthreads();
    WH_TL(1, 10);
    // per-expert outputs (the 8 blocks of each expert in order), then the
    // ordered routed sum
    if (threadIdx.x < 16) {
        const uint32_t r = threadIdx.x, orow = blockIdx.x * 16 + r;
        float yv[WH_MAX_EXPERTS];
        bool finite = true;
#pragma unroll
        for (uint32_t e = 0; e < WH_MAX_EXPERTS; ++e) {
            if (e < (uint32_t)kN) {
                const float* p = red + 8 * e * 16 + r;
                float y = p[0];
#pragma unroll
                for (int k = 1; k < 8; ++k) y = y + p[16 * k];
                finite = finite && fabsf(y) <= 3.4028235e38f;
                yv[e] = y;
                a.y[((size_t)tok * kN + e) * a.hidden + orow] = y;
            } else {
                yv[e] = 0.0f;
            }
        }
        if (!finite) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        a.out[(size_t)tok * a.hidden + orow] = wh_route_combine(a, yv);
    }
    WH_TL(1, 11);
}

// Down + routed sum, inter = 2048: grid (hidden / 16, n_tokens), 512
// threads.  Unit u = (expert u / 4, column quarter u % 4 of 512 = blocks
// 2 (u % 4), + 1) of the workgroup's 16 output rows; wave w runs units w,
// w + 8, ... (kU = ceil(n_experts / 2) of them).  Wave w also act-quantizes
// (E/deepseek_v4.rs:595, block 64) exactly the h values of its own units
// (expert w / 4 + 2 i, quarter w % 4), so no wave waits for another before
// its first MFMA.
template <int kU>
__global__ void __launch_bounds__(512, 1) k_moe_down_px(wh_moe_args a) {
    constexpr uint32_t kCols = 2048, kG = kCols / 32;
    constexpr int kJ = 2 * kU, kDepth = WH_PX_DN_DEPTH < kJ ? WH_PX_DN_DEPTH : kJ;
    constexpr int kPro = WH_PX_DN_PRO < kDepth ? WH_PX_DN_PRO : kDepth;
    __shared__ __align__(16) uint8_t hc[WH_MAX_EXPERTS * kCols];
    __shared__ __align__(16) uint8_t hsb[WH_MAX_EXPERTS * kG];
    __shared__ float red[WH_MAX_EXPERTS * 4 * 16];
    WH_TL(1, 0);
    const uint32_t tok = blockIdx.y, n = a.n_experts, n_units = 4 * n;
    // wave-uniform in SGPRs: the expert table reads are scalar loads, which
    // do not queue behind the h loads
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), L = threadIdx.x & 63, g = L >> 4;
    const uint32_t row = blockIdx.x * 16 + (L & 15);
    const float* htok = a.h + (size_t)tok * n * kCols;
    // h of the wave's units: chunk i of thread t = columns 8 (c % 256) ..
    // + 7 of expert c / 256, c = t + 512 i (expert w / 4 + 2 i, quarter
    // w % 4 for wave w); chunks past the last expert load the last expert's
    // and are not stored
    float4 hv[kU][2];
#pragma unroll
    for (int i = 0; i < kU; ++i) {
        const uint32_t c = threadIdx.x + 512 * i, e = c >> 8;
        const float4* hp = (const float4*)(htok + (size_t)(e < n ? e : n - 1) * kCols + 8 * (c & 255));
        hv[i][0] = hp[0];
        hv[i][1] = hp[1];
    }
    // the wave's units (a unit past the end repeats unit n_units - 1; its
    // result is not stored)
    const uint8_t* wl[kU];
    const uint8_t* sr[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        uint32_t u = wave + 8 * k;
        u = u < n_units ? u : n_units - 1;
        const uint32_t e = u >> 2, qt = u & 3;
        const wh_expert_ptrs ep = wh_moe_ex(a, e);
        wl[k] = ep.w2 + (size_t)row * (kCols / 2) + 256 * qt + 64 * (g & 1) + 32 * (g >> 1);
        sr[k] = ep.s2 + (size_t)row * kG + 16 * qt;
    }
    wh_issue_barrier();
    wh_mx_raw ring[kDepth];
#pragma unroll
    for (int j = 0; j < kPro; ++j) wh_mx_raw_load(ring[j], wl[j >> 1], sr[j >> 1], j & 1);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(1, 1);
#ifdef WH_TIMELINE
    {
        float hs = 0.0f;
#pragma unroll
        for (int i = 0; i < kU; ++i) hs += hv[i][0].x + hv[i][1].w;
        WH_TL_USE(hs);
    }
#endif
    WH_TL(1, 2);
    // act-quant of h, chunk i = unit i's 512 values (measured: quantizing
    // each unit just before its MFMAs instead was slower): h is finite whenever
    // gate/up was (a non-finite gate/up output is already reported); the
    // codes go to the record layout (column 8 (c % 4) + j of group c / 4 at
    // byte 4 j + c % 4).  The wave reads back only codes it wrote itself:
    // LDS operations of one wave complete in order, so no workgroup barrier
    // is needed (the clobber keeps the compiler from moving a read above the
    // writes).
    auto quant_chunk = [&](int i) {
        const uint32_t c = threadIdx.x + 512 * i, e = c >> 8, idx = c & 255;
        const float v[8] = {hv[i][0].x, hv[i][0].y, hv[i][0].z, hv[i][0].w,
                            hv[i][1].x, hv[i][1].y, hv[i][1].z, hv[i][1].w};
        bool bad;
        const int k = wh_quant8_scale(v, bad);
        uint32_t cd[8];
        wh_quant8_f32_codes(v, k, cd);
        if (e < n) {
            uint8_t* grp = hc + kCols * e + 32 * (idx >> 2) + (idx & 3);
#pragma unroll
            for (int j = 0; j < 8; ++j) grp[4 * j] = (uint8_t)cd[j];
            if ((idx & 3) == 0) hsb[kG * e + (idx >> 2)] = (uint8_t)(127 + k - 3);
        }
        asm volatile("" ::: "memory");
    };
#pragma unroll
    for (int i = 0; i < kU; ++i) quant_chunk(i);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(1, 3);
#pragma unroll
    for (int j = kPro; j < kDepth; ++j) wh_mx_raw_load(ring[j], wl[j >> 1], sr[j >> 1], j & 1);
    __builtin_amdgcn_sched_barrier(0);
    WH_TL(1, 4);
    WH_TL(1, 5);
    {
        uint32_t dep = wh_opaque_zero(__uint_as_float(*(const uint32_t*)hsb));
        wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const int b = j & 1, kk = j >> 1;
            uint32_t u = wave + 8 * kk;
            u = u < n_units ? u : n_units - 1;
            const uint32_t e = u >> 2, qt = u & 3;
            wh_mx_bop bo;
            wh_mx_bop_load(bo, hc + kCols * e + 512 * qt + 256 * b + dep, hsb + kG * e + 16 * qt + 8 * b + dep, g);
            wh_px_step(acc, ring[j % kDepth], dep, bo, g);
            if (j + kDepth < kJ)
                wh_mx_raw_load(ring[j % kDepth], wl[(j + kDepth) >> 1] + dep, sr[(j + kDepth) >> 1] + dep,
                               (j + kDepth) & 1);
            if (b == 1) {
                asm volatile("" : "+v"(acc));
                if ((L & 15) == 0 && wave + 8 * kk < n_units) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) red[(wave + 8 * kk) * 16 + 4 * g + r] = acc[r];
                }
                acc = wh_v4f{0.0f, 0.0f, 0.0f, 0.0f};
                if (kk < 4) WH_TL(1, 6 + kk);
            }
        }
    }
    __syncthreads();
    WH_TL(1, 10);
    // per-expert outputs (the 4 quarters of each expert), then the ordered
    // routed sum
    if (threadIdx.x < 16) {
        const uint32_t r = threadIdx.x, orow = blockIdx.x * 16 + r;
        float yv[WH_MAX_EXPERTS];
        bool finite = true;
#pragma unroll
        for (uint32_t e = 0; e < WH_MAX_EXPERTS; ++e) {
            if (e < n) {
                const float* p = red + 4 * e * 16 + r;
                const float y = ((p[0] + p[16]) + p[32]) + p[48];
                finite = finite && fabsf(y) <= 3.4028235e38f;
                yv[e] = y;
                a.y[((size_t)tok * n + e) * a.hidden + orow] = y;
            } else {
                yv[e] = 0.0f;
            }
        }
        if (!finite) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        a.out[(size_t)tok * a.hidden + orow] = wh_route_combine(a, yv);
    }
    WH_TL(1, 11);
}
