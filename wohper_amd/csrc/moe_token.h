// Split-K routed-expert kernels for decode tokens (gfx950).
//
// The bit-exact kernels of kernels.h follow the reference's per-lane FMA
// chain (E/deepseek_v4.rs:294-347): one thread walks a whole row for one
// AVX lane, so it reads every x value it needs from LDS and spends about
// 2.6 VALU instructions per FP4 weight.  These kernels compute the same
// matvecs with the summation order freed (outputs within
// 1e-5 * ||w_row||_2 * ||x||_2 of the reference kernel, fp32 accumulation):
//
//   * a wave owns a 2048-column slice of its rows; lane L holds the x values
//     of the 16 bytes it loads from every row (block L/8 of the slice, AVX
//     lane L%8: 8 groups x 4 columns) in registers, as f16 pairs of the
//     act-quant codes (E4M3 values, exact in f16);
//   * the weight nibbles decode to f16 pairs of the reference's base values
//     (two v_perm LUT lookups and the sign bits give the high bytes, two
//     more v_perm per dword place them), multiplied into the codes with
//     v_dot2_f32_f16 (products exact, sums in f32);
//   * per row and group the partial sum takes one FMA with the group's
//     UE8M0 scale times the x block scale (a table in LDS built once per
//     wave);
//   * rows stream through a ring of kDepth 16-byte loads per lane, and the
//     wave's kRows row sums leave through a transposed DPP reduction.
//
// Dequantized weights are the reference's values exactly; only the order
// of the fp32 sums differs from the CPU kernel.
#pragma once
#include "kernels.h"

typedef _Float16 wh_h2 __attribute__((ext_vector_type(2)));

// f16 high bytes of the reference base values |v| of E/deepseek_v4.rs:177-180
// (the low bytes are zero): {0, 0.125, 1, 1.5} and {2, 3, 4, 6}.
#define WH_FP4H_LUT_LO 0x3e3c3000u
#define WH_FP4H_LUT_HI 0x46444240u

// Row stride (floats) of a wave's LDS scale table: 64 groups + 4.
#define WH_SK_SCT_STRIDE 68u

// One resident dword (see wh_fp4_encode_word) -> four f16 pairs:
// (A0, A1), (A2, A3) of its first group and (B0, B1), (B2, B3) of its second.
struct wh_fp4h8 {
    uint32_t a01, a23, b01, b23;
};
__device__ __forceinline__ wh_fp4h8 wh_fp4_decode8_h(uint32_t w) {
    uint32_t fa = __builtin_amdgcn_perm(WH_FP4H_LUT_HI, WH_FP4H_LUT_LO, w & 0x07070707u);
    const uint32_t r = __builtin_amdgcn_alignbit(w, w, 4);  // rotate right by 4
    fa |= r & 0x80808080u;
    uint32_t fb = __builtin_amdgcn_perm(WH_FP4H_LUT_HI, WH_FP4H_LUT_LO, r & 0x07070707u);
    fb |= w & 0x80808080u;
    wh_fp4h8 o;
    o.a01 = __builtin_amdgcn_perm(fa, fa, 0x010c000cu);  // [0, fa.b0, 0, fa.b1]
    o.a23 = __builtin_amdgcn_perm(fa, fa, 0x030c020cu);
    o.b01 = __builtin_amdgcn_perm(fb, fb, 0x010c000cu);
    o.b23 = __builtin_amdgcn_perm(fb, fb, 0x030c020cu);
    return o;
}

__device__ __forceinline__ float wh_dot2h(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(wh_h2, a), __builtin_bit_cast(wh_h2, b), c, false);
}
// The same from a zero sum, in the three-operand encoding (an inline 0
// instead of a register cleared for the accumulating two-operand form).
__device__ __forceinline__ float wh_dot2h0(uint32_t a, uint32_t b) {
    float r;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// One dword of a lane: groups A and B (x pairs xa[0..1], xb[0..1], scales
// sa, sb) folded into acc.
__device__ __forceinline__ float wh_fp4h_dword(uint32_t word, const uint32_t* xa, const uint32_t* xb, float sa,
                                               float sb, float acc) {
    const wh_fp4h8 e = wh_fp4_decode8_h(word);
    float ga = wh_dot2h0(e.a01, xa[0]);
    ga = wh_dot2h(e.a23, xa[1], ga);
    float gb = wh_dot2h0(e.b01, xb[0]);
    gb = wh_dot2h(e.b23, xb[1], gb);
    acc = __builtin_fmaf(ga, sa, acc);
    return __builtin_fmaf(gb, sb, acc);
}

template <int kCtrl>
__device__ __forceinline__ float wh_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// One level of the transposed reduction: v[0..N) -> v[0..N/2).  The lane
// keeps the upper half when `upper`, its partner (which has `upper`
// negated) keeps the other, and each adds the partner's copy of its half.
template <int N, int kCtrl>
__device__ __forceinline__ void wh_fold(float* v, bool upper) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const float keep = upper ? v[i + N / 2] : v[i];
        const float send = upper ? v[i] : v[i + N / 2];
        v[i] = keep + wh_dpp<kCtrl>(send);
    }
}

// Sums v[0..R) (R = 8 or 16) over the 64 lanes of the wave.  The sum of
// row wh_wave_rows_lane_row<R>(L & 15) ends in every lane L.
template <int R>
__device__ __forceinline__ float wh_wave_sum_rows(float* v, uint32_t L) {
    static_assert(R == 4 || R == 8 || R == 16, "4, 8 or 16 rows");
    constexpr int kMirror = 0x141, kXor2 = 0x4e, kXor1 = 0xb1, kRor8 = 0x128;
    wh_fold<R, kMirror>(v, (L >> 2) & 1);  // partner L ^ 7 within 8 lanes
    wh_fold<R / 2, kXor2>(v, (L >> 1) & 1);
    float s;
    if constexpr (R == 4) {
        s = v[0] + wh_dpp<kXor1>(v[0]);
        s += wh_dpp<kRor8>(s);
    } else if constexpr (R == 8) {
        wh_fold<2, kXor1>(v, L & 1);
        s = v[0] + wh_dpp<kRor8>(v[0]);
    } else {
        wh_fold<4, kXor1>(v, L & 1);
        wh_fold<2, kRor8>(v, (L >> 3) & 1);  // partner L ^ 8 within 16 lanes
        s = v[0];
    }
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    return s;
}
template <int R>
__host__ __device__ constexpr uint32_t wh_wave_rows_lane_row(uint32_t l16) {
    return R == 16  ? 8 * ((l16 >> 2) & 1) + 4 * ((l16 >> 1) & 1) + 2 * (l16 & 1) + ((l16 >> 3) & 1)
           : R == 8 ? 4 * ((l16 >> 2) & 1) + 2 * ((l16 >> 1) & 1) + (l16 & 1)
                    : 2 * ((l16 >> 2) & 1) + ((l16 >> 1) & 1);
}

// x of lane L for slice block `blk` (8 groups x 4 columns), as f16 pairs of
// the staged codes.
__device__ __forceinline__ void wh_sk_x_regs(uint32_t (&xr)[8][2], const float* xs, uint32_t blk, uint32_t l) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 q = ((const float4*)xs)[wh_xs_f4(8 * blk + j, l)];
        xr[j][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q.x, q.y));
        xr[j][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q.z, q.w));
    }
}

// A wave's scale table: kRows rows x the 64 groups of its slice, each
// UE8M0 scale times the x block scale of its columns.  The raw bytes are
// loaded early (kRows bytes per lane: row L / (64 / kRows)).
template <int kRows>
struct wh_sk_scales {
    uint32_t v[kRows / 4];
};
template <int kRows>
__device__ __forceinline__ void wh_sk_scales_load(wh_sk_scales<kRows>& st, const uint8_t* sbase, uint32_t G,
                                                  uint32_t L) {
    constexpr uint32_t per_row = 64 / kRows;  // lanes per row
    const uint8_t* p = sbase + (size_t)(L / per_row) * G + kRows * (L % per_row);
    if constexpr (kRows == 16) {
        const uint4 q = *(const uint4*)p;
        st.v[0] = q.x, st.v[1] = q.y, st.v[2] = q.z, st.v[3] = q.w;
    } else if constexpr (kRows == 8) {
        const uint2 q = *(const uint2*)p;
        st.v[0] = q.x, st.v[1] = q.y;
    } else {
        st.v[0] = *(const uint32_t*)p;
    }
}
// The x block scales the lane's scale bytes need (kRows / 2 floats from
// xk_slice, the slice's 32 block scales), loaded early.
template <int kRows>
struct wh_sk_xk {
    float v[kRows / 2];
};
template <int kRows>
__device__ __forceinline__ void wh_sk_xk_load(wh_sk_xk<kRows>& st, const float* xk_slice, uint32_t L) {
    const float* p = xk_slice + (kRows * (L % (64 / kRows))) / 2;
#pragma unroll
    for (int i = 0; i < kRows / 2; i += 2) {
        const float2 q = *(const float2*)(p + i);
        st.v[i] = q.x, st.v[i + 1] = q.y;
    }
}
// xk: the x block scales of the lane's bytes (kRows / 2, two groups each);
// sct: the wave's table.
template <int kRows>
__device__ __forceinline__ void wh_sk_scales_store(const wh_sk_scales<kRows>& st, const float* xk, float* sct,
                                                   uint32_t L) {
    constexpr uint32_t per_row = 64 / kRows;
    const uint32_t g0 = kRows * (L % per_row);  // first group of the lane's bytes
    float* d = sct + (L / per_row) * WH_SK_SCT_STRIDE + g0;
#pragma unroll
    for (int q = 0; q < kRows / 4; ++q) {
        const uint32_t v = st.v[q];
        const float k0 = xk[2 * q], k1 = xk[2 * q + 1];
        ((float4*)d)[q] = make_float4(wh_ue8m0(v) * k0, wh_ue8m0(v >> 8) * k0, wh_ue8m0(v >> 16) * k1,
                                      wh_ue8m0(v >> 24) * k1);
    }
}

// The kRows row sums of one wave over its slice.  wbase: the lane's 16
// bytes of row 0; row r is rstride bytes further.
template <int kRows, int kDepth>
__device__ __forceinline__ void wh_sk_rows(float (&acc)[kRows], const uint8_t* __restrict__ wbase, size_t rstride,
                                           wh_fp4_ring<kDepth>& ring, const uint32_t (&xr)[8][2],
                                           const float* sct_l) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const uint4 w = ring.w[r % kDepth];
        if (r + kDepth < kRows) ring.w[r % kDepth] = *(const uint4*)(wbase + (size_t)(r + kDepth) * rstride);
        const float4 s0 = ((const float4*)(sct_l + r * WH_SK_SCT_STRIDE))[0];
        const float4 s1 = ((const float4*)(sct_l + r * WH_SK_SCT_STRIDE))[1];
        float a = wh_fp4h_dword(w.x, xr[0], xr[1], s0.x, s0.y, 0.0f);
        a = wh_fp4h_dword(w.y, xr[2], xr[3], s0.z, s0.w, a);
        a = wh_fp4h_dword(w.z, xr[4], xr[5], s1.x, s1.y, a);
        acc[r] = wh_fp4h_dword(w.w, xr[6], xr[7], s1.z, s1.w, a);
    }
}

// LDS bytes of the split-K down workgroup: h codes, h block scales, the
// log2f thresholds and 4 waves' scale tables of 8 rows.
__host__ __device__ constexpr size_t wh_moe_down_sk_lds(size_t cols) {
    return sizeof(float) * (wh_xs_floats((uint32_t)cols) + cols / 64 + 256 + 4 * 8 * WH_SK_SCT_STRIDE);
}

// Act-quant of every token's x (block 64, E/compute.rs:2504-2521) for the
// split-K gate/up kernel, hidden = 2048 * kSl: grid (n_tokens), 128 * kSl
// threads of 16 columns.  xq: per token, per 256-column block and AVX lane
// l, the 32 codes the lane multiplies (group j of the block, columns
// l + 8k, k = 0..3 at halves 4j + k) as f16; xk: per token, the block scales.
template <int kSl>
__global__ void __launch_bounds__(128 * kSl) k_moe_xquant(const void* x, uint32_t x_is_bf16, uint32_t* xq, float* xk,
                                                          uint32_t* status) {
    constexpr uint32_t kCols = 2048 * kSl;
    __shared__ uint32_t thr[256];
    const uint32_t tok = blockIdx.x;
    const bool bf16 = x_is_bf16 != 0;
    const void* xt = bf16 ? (const void*)((const uint16_t*)x + (size_t)tok * kCols)
                          : (const void*)((const float*)x + (size_t)tok * kCols);
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_xq_stage xst;
    wh_xq_stage_load(xst, xt, bf16, kCols, threadIdx.x);
    wh_thr_stage_store(ts, thr);
    __syncthreads();
    float q[16], sc;
    if (!wh_xq_quant16(xst, bf16, thr, q, sc)) return;
    const uint32_t c0 = xst.c0, g = c0 >> 5, hh = (c0 >> 4) & 1, b = g >> 3, j = g & 7;
    uint32_t* d = xq + (size_t)tok * (kCols / 2) + b * 128 + 2 * j + hh;  // 2 halves per dword
#pragma unroll
    for (int l = 0; l < 8; ++l)
        d[16 * l] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q[l], q[8 + l]));
    if ((c0 & 63) == 0) xk[(size_t)tok * (kCols / 64) + (c0 >> 6)] = sc;
}

// Gate/up + SwiGLU, hidden = 2048 * kSl, x act-quantized by k_moe_xquant:
// grid (n_experts * inter / kRows, n_tokens), 128 * kSl threads.  Wave
// (m, h) runs slice h of kRows rows of w1 (m = 0) or w3 (m = 1); the
// workgroup's epilogue adds the slices in order and applies SwiGLU
// (E/deepseek_v4.rs:586-594).
template <int kSl, int kRows>
__global__ void __launch_bounds__(128 * kSl) k_moe_gateup_sk(wh_moe_args a) {
    constexpr int kDepth = 8, kWaves = 2 * kSl;
    constexpr uint32_t kCols = 2048 * kSl, G = kCols / 32;
    __shared__ __align__(16) float sct_all[kWaves * kRows * WH_SK_SCT_STRIDE];
    __shared__ float red[kWaves * kRows];
    __shared__ uint64_t exp_tab[WH_EXP_TAB_LEN];
    wh_exp_stage es;
    wh_exp_stage_load(es);
    const uint32_t tok = blockIdx.y;
    wh_moe_clear_arrivals(a, tok);
    const uint32_t per_e = a.inter / kRows;
    const uint32_t e = blockIdx.x / per_e;
    const uint32_t rb = blockIdx.x - e * per_e;
    const uint32_t wave = threadIdx.x >> 6, L = threadIdx.x & 63;
    const uint32_t m = wave / kSl, h = wave - m * kSl;
    const uint32_t row0 = rb * kRows;
    const wh_expert_ptrs ep = a.ex[e];
    const uint8_t* wbase = (m ? ep.w3 : ep.w1) + (size_t)row0 * (kCols / 2) + 1024 * h + 16 * L;
    const uint8_t* sbase = (m ? ep.s3 : ep.s1) + (size_t)row0 * G + 64 * h;
    // the lane's x codes (block 8h + L/8, lane L%8: 64 bytes), the scale
    // bytes and x block scales of its table entries, then the weight ring
    const uint4* xp = (const uint4*)(a.xq + (size_t)tok * (kCols / 2) + (8 * h + (L >> 3)) * 128 + 16 * (L & 7));
    uint4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = xp[i];
    wh_sk_scales<kRows> ss;
    wh_sk_scales_load<kRows>(ss, sbase, G, L);
    wh_sk_xk<kRows> xks;
    wh_sk_xk_load<kRows>(xks, a.xk + (size_t)tok * (kCols / 64) + 32 * h, L);
    wh_fp4_ring<kDepth> ring;
#pragma unroll
    for (int d = 0; d < kDepth; ++d) ring.w[d] = *(const uint4*)(wbase + (size_t)d * (kCols / 2));
    __builtin_amdgcn_sched_barrier(0);
    float* sct = sct_all + wave * kRows * WH_SK_SCT_STRIDE;
    wh_sk_scales_store<kRows>(ss, xks.v, sct, L);
    wh_exp_stage_store(es, exp_tab);
    const uint32_t xr[8][2] = {{xv[0].x, xv[0].y}, {xv[0].z, xv[0].w}, {xv[1].x, xv[1].y}, {xv[1].z, xv[1].w},
                               {xv[2].x, xv[2].y}, {xv[2].z, xv[2].w}, {xv[3].x, xv[3].y}, {xv[3].z, xv[3].w}};
    __syncthreads();
    float acc[kRows];
    wh_sk_rows<kRows, kDepth>(acc, wbase, kCols / 2, ring, xr, sct + 8 * (L >> 3));
    const float s = wh_wave_sum_rows<kRows>(acc, L);
    if (L < 16 && (kRows == 16 || (L & 8) == 0) && (kRows >= 8 || (L & 1) == 0))
        red[wave * kRows + wh_wave_rows_lane_row<kRows>(L)] = s;
    __syncthreads();
    if (threadIdx.x < kRows) {
        const uint32_t r = threadIdx.x;
        float g = red[r], u = red[kSl * kRows + r];
#pragma unroll
        for (int k = 1; k < kSl; ++k) {
            g += red[k * kRows + r];
            u += red[(kSl + k) * kRows + r];
        }
        if (!(fabsf(g) <= 3.4028235e38f) || !(fabsf(u) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        const size_t he = ((size_t)tok * a.n_experts + e) * a.inter;
        a.h[he + row0 + r] = wh_swiglu(g, u, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT);
        if (a.gu) {
            a.gu[2 * he + row0 + r] = g;
            a.gu[2 * he + a.inter + row0 + r] = u;
        }
    }
}

// Down + ordered routed sum, inter = 2048: grid (n_experts * hidden / 32,
// n_tokens), 256 threads = 4 waves x 8 output rows of one expert.  The act-
// quant of h (E/deepseek_v4.rs:595) is recomputed by every workgroup while
// staging it; the last expert to finish a 32-row slice sums the experts in
// route order (E/compute.rs:1948-2012).
__global__ void __launch_bounds__(256) k_moe_down_sk(wh_moe_args a) {
    constexpr int kRows = 8, kDepth = 8;
    constexpr uint32_t kCols = 2048, G = kCols / 32;
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t last;
    float* xs = lds;
    float* xk = xs + wh_xs_floats(kCols);
    uint32_t* thr = (uint32_t*)(xk + kCols / 64);
    float* sct_all = (float*)(thr + 256);
    const uint32_t tok = blockIdx.y;
    const uint32_t per_e = a.hidden >> 5;
    const uint32_t e = blockIdx.x / per_e;
    const uint32_t rb = blockIdx.x - e * per_e;  // 32-row slice of the output
    const uint32_t wave = threadIdx.x >> 6, L = threadIdx.x & 63;
    const uint32_t row0 = rb * 32 + wave * kRows;
    const wh_expert_ptrs ep = a.ex[e];
    const uint8_t* wbase = ep.w2 + (size_t)row0 * (kCols / 2) + 16 * L;
    const uint8_t* sbase = ep.s2 + (size_t)row0 * G;
    const float* hrow = a.h + ((size_t)tok * a.n_experts + e) * kCols;
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_h_stage hst;
    wh_h_stage_load(hst, hrow, kCols, threadIdx.x);  // 8 values per thread: kCols / 8 == 256
    wh_sk_scales<kRows> ss;
    wh_sk_scales_load<kRows>(ss, sbase, G, L);
    wh_fp4_ring<kDepth> ring;
#pragma unroll
    for (int d = 0; d < kDepth; ++d) ring.w[d] = *(const uint4*)(wbase + (size_t)d * (kCols / 2));
    __builtin_amdgcn_sched_barrier(0);
    wh_thr_stage_store(ts, thr);
    __syncthreads();
    wh_h_stage_store<true>(hst, xs, thr, xk);
    __syncthreads();
    float* sct = sct_all + wave * kRows * WH_SK_SCT_STRIDE;
    wh_sk_scales_store<kRows>(ss, xk + (kRows * (L % (64 / kRows))) / 2, sct, L);
    uint32_t xr[8][2];
    wh_sk_x_regs(xr, xs, L >> 3, L & 7);
    __syncthreads();
    float acc[kRows];
    wh_sk_rows<kRows, kDepth>(acc, wbase, kCols / 2, ring, xr, sct + 8 * (L >> 3));
    const float yv = wh_wave_sum_rows<kRows>(acc, L);
    if (L < kRows) {
        const uint32_t row = row0 + wh_wave_rows_lane_row<kRows>(L);
        if (!(fabsf(yv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        wh_store_coherent(a.y + ((size_t)tok * a.n_experts + e) * a.hidden + row, yv);
    }
    wh_moe_routed_sum(a, tok, rb, &last);
}
