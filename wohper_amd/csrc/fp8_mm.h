// Multi-input FP8 GEMV on bf16 MFMA (gfx950): y_t = W x_t for up to 16 inputs
// per workgroup, each weight byte read once from HBM.  This is the
// summation-order-free mode of the multi-input entry points; the reference's
// rows_multi (E/compute.rs:6384-6577) decodes a row once and runs n dots in
// the single-input order.
//
// Numerics.  Every E4M3 weight (the reference's values, +-480 for 0x7F/0xFF
// included) is exact in bf16.  Each input value x splits into three bf16
// pieces, each rounded to nearest: hi = bf16(x), mid = bf16(x - hi),
// lo = bf16(x - hi - mid).  The residuals are exact in f32 and the last one
// has at most 8 significant bits, so hi + mid + lo == x for |x| >= 2^-110
// (below that, the lost bits are < 2^-133 each).  Every MFMA product is
// exact, so the outputs differ from the reference kernel's by fp32
// accumulation order only.
//
// Layout.  The resident FP8 rows keep, per 128-column group, AVX lane l's 16
// bytes together (position p = 16 l + 8 h + c holds column 16 c + 8 h + l).
// The contraction runs in position order: lane group q of
// v_mfma_f32_16x16x32_bf16 m takes positions 32 q + 8 m .. + 7, so a lane
// loads 32 contiguous bytes of its row per group.  The workgroup stages its
// inputs in LDS in the same position order, as bf16 planes
//   xs[hi | mid | lo][group g][m][q][token t][j]   (j = c, the 8 of a slot),
// straight from the f32 inputs: a staging thread (g, t, h, 4-column half)
// loads columns 16 c + 8 h + 4 half + i for c = 0..7, i = 0..3, which are
// the j = 0..7 of slot (m, q) = ((2 l + h) & 3, l / 2), l = 4 half + i.
// Workgroup (row block, k split, token block): 8 waves x 16 rows; the scale
// of a 128 x 128 block multiplies the group's MFMA sum (tiles of 16 rows never
// straddle a scale row).  With more than one k split, each workgroup stores
// its partial tile and the last one of a row block sums the splits in order.
#pragma once
#include "kernels.h"

typedef __bf16 wh_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 wh_bf16x2 __attribute__((ext_vector_type(2)));
typedef float wh_f32x2 __attribute__((ext_vector_type(2)));
typedef float wh_f32x4 __attribute__((ext_vector_type(4)));

#define WH_FP8MM_ROWS 128u  // rows per workgroup: 8 waves x 16
#define WH_FP8MM_TOK 16u    // inputs per token block
#ifndef WH_FP8MM_DEPTH
#define WH_FP8MM_DEPTH 4    // weight groups of a wave in flight
#endif
#ifndef WH_FP8MM_MAX_GROUPS
#define WH_FP8MM_MAX_GROUPS 8u  // 128-column groups per k split
#endif
#ifndef WH_FP8MM_WG_PER_CU
#define WH_FP8MM_WG_PER_CU 2    // launch bound: workgroups per CU the registers allow
#endif

// LDS bytes of a workgroup's staged inputs for a k split of `kc` columns.
__host__ __device__ constexpr size_t wh_fp8mm_lds(size_t kc) { return kc * WH_FP8MM_TOK * 3 * 2; }

struct wh_fp8mm_args {
    const uint8_t* w;     // resident (lane-permuted) rows
    const void* scales;   // [scale_rows][scale_cols], f32 or UE8M0 bytes
    const float* x;       // input t of group g at x + t * x_stride + g * xg_stride
    float* y;             // output t, row r at y + t * y_stride + (r - row_start)
    float* ws;            // partial tiles [token block][row block][split][128][16]
    uint32_t* cnt;        // [token block][row block] arrivals (zero between calls)
    uint32_t* status;
    uint32_t cols, scale_cols, row_group_shift, row_start, row_end;
    uint32_t n, x_stride, y_stride;
    uint32_t xg_shift;    // log2(rows per input group); 31 = one group
    uint32_t xg_stride;
    uint32_t kc, splits, row_blocks;
    // a second tensor on the same inputs (wq_a and wkv): the row blocks from
    // rb_first on run its rows [row_start2, row_end2) into y2 (same width,
    // scale format and rows per scale row); rb_first = row_blocks when there
    // is none
    const uint8_t* w2;
    const void* scales2;
    float* y2;
    uint32_t row_start2, row_end2, y2_stride, rb_first;
};

// Two f32 to two bf16, each rounded to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t wh_bf16x2_rne(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((wh_f32x2){a, b}, wh_bf16x2));
}
__device__ __forceinline__ float wh_bf16_lo_f32(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float wh_bf16_hi_f32(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Splits 8 values into their hi, mid and lo bf16 pieces (8 each).
__device__ __forceinline__ void wh_split3_x8(const float (&v)[8], uint4& hi, uint4& mid, uint4& lo) {
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float a = v[2 * k], b = v[2 * k + 1];
        h[k] = wh_bf16x2_rne(a, b);
        const float ra = a - wh_bf16_lo_f32(h[k]), rb = b - wh_bf16_hi_f32(h[k]);
        m[k] = wh_bf16x2_rne(ra, rb);
        l[k] = wh_bf16x2_rne(ra - wh_bf16_lo_f32(m[k]), rb - wh_bf16_hi_f32(m[k]));
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    mid = make_uint4(m[0], m[1], m[2], m[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// 8 E4M3 bytes (two dwords) -> 8 bf16, the reference's values.
template <bool kSpecial>
__device__ __forceinline__ wh_bf16x8 wh_fp8_bf16x8(uint32_t d0, uint32_t d1) {
    uint32_t o[4];
    const uint32_t d[2] = {d0, d1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (kSpecial) {
            const wh_f2 a = wh_fp8x2<true, false>(d[i]), b = wh_fp8x2<true, true>(d[i]);
            o[2 * i] = __builtin_amdgcn_perm(__float_as_uint(a.y), __float_as_uint(a.x), 0x07060302u);
            o[2 * i + 1] = __builtin_amdgcn_perm(__float_as_uint(b.y), __float_as_uint(b.x), 0x07060302u);
        } else {
            const auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[i], 1.0f, false);
            const auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[i], 1.0f, true);
            o[2 * i] = __builtin_bit_cast(uint32_t, a);
            o[2 * i + 1] = __builtin_bit_cast(uint32_t, b);
        }
    }
    return __builtin_bit_cast(wh_bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
}

template <bool kScaleU8>
__device__ __forceinline__ float wh_fp8mm_scale(const void* s, size_t idx) {
    if constexpr (kScaleU8) return wh_ue8m0(((const uint8_t*)s)[idx]);
    else return ((const float*)s)[idx];
}

// grid (row blocks, splits, token blocks), 512 threads, wh_fp8mm_lds(kc)
// bytes of dynamic LDS; kG = kc / 128 groups per split (2, 4 or 8), a
// compile-time count so that the weight ring is straight-line code whose
// waits cover exactly the loads they need.
template <bool kSpecial, bool kScaleU8, int kG>
__global__ void __launch_bounds__(512, WH_FP8MM_WG_PER_CU) k_fp8_mm(wh_fp8mm_args a) {
    extern __shared__ __align__(16) uint16_t xmm[];  // [hi | mid | lo][G][m][q][t][8]
    const uint32_t rb = blockIdx.x, ks = blockIdx.y, tb = blockIdx.z;
    const uint32_t wave = threadIdx.x >> 6, L = threadIdx.x & 63, q = L >> 4;
    // the row block's tensor
    const bool t2 = rb >= a.rb_first;
    const uint8_t* const W = t2 ? a.w2 : a.w;
    const void* const SC = t2 ? a.scales2 : a.scales;
    float* const Y = t2 ? a.y2 : a.y;
    const uint32_t row_start = t2 ? a.row_start2 : a.row_start, row_end = t2 ? a.row_end2 : a.row_end;
    const uint32_t y_stride = t2 ? a.y2_stride : a.y_stride;
    const uint32_t rbl = t2 ? rb - a.rb_first : rb;  // row block within its tensor
    const uint32_t r0 = row_start + rbl * WH_FP8MM_ROWS;
    const uint32_t grp = a.xg_shift < 31 ? (rbl * WH_FP8MM_ROWS) >> a.xg_shift : 0;
    constexpr uint32_t G = kG;
    const uint32_t g0 = ks * G;
    const uint32_t P = G * 2048;  // bf16 of one plane
    // staging thread (group sg, token st, h, half): 8 float4 of its input row
    const uint32_t sg = threadIdx.x >> 6, st = (L >> 2) & 15, sh = (L >> 1) & 1, shalf = L & 1;
    const uint32_t stg = tb * WH_FP8MM_TOK + st;
    const bool stager = sg < G && stg < a.n;
    float4 xv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) xv[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (stager) {
        const float* xr = a.x + (size_t)stg * a.x_stride + (size_t)grp * a.xg_stride + (g0 + sg) * 128 + 8 * sh +
                          4 * shalf;
#pragma unroll
        for (int c = 0; c < 8; ++c) xv[c] = *(const float4*)(xr + 16 * c);
    }
    // the lane's row (rows past the end load row_start's bytes; not stored)
    const uint32_t row = r0 + 16 * wave + (L & 15);
    const uint32_t rc = row < row_end ? row : row_start;
    const uint8_t* wrow = W + (size_t)rc * a.cols + (size_t)g0 * 128 + 32 * q;
    const uint32_t trow = r0 + 16 * wave < row_end ? r0 + 16 * wave : row_end - 1;  // the tile's scale row
    const size_t srow = (size_t)(trow >> a.row_group_shift) * a.scale_cols + g0;
    // lane j < G holds the tile's scale of group j, loaded with the inputs so
    // that no wait in the weight loop covers a load issued after the ring's
    float sv = 0.0f;
    if (L < G) sv = wh_fp8mm_scale<kScaleU8>(SC, srow + L);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // every wave's input loads go out before any weight load
    __builtin_amdgcn_sched_barrier(0);
    constexpr int kD = kG < WH_FP8MM_DEPTH ? kG : WH_FP8MM_DEPTH;
    uint4 rw[kD][2];
#pragma unroll
    for (int i = 0; i < kD; ++i) {
        rw[i][0] = *(const uint4*)(wrow + 128 * i);
        rw[i][1] = *(const uint4*)(wrow + 128 * i + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (sg < G) {  // tokens past n stage zeros
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v[8] = {xv[0][i], xv[1][i], xv[2][i], xv[3][i], xv[4][i], xv[5][i], xv[6][i], xv[7][i]};
            uint4 hi, mid, lo;
            wh_split3_x8(v, hi, mid, lo);
            const uint32_t l = 4 * shalf + i, m = (2 * l + sh) & 3, lq = l >> 1;
            const uint32_t off = (((sg * 4 + m) * 4 + lq) * 16 + st) * 8;
            *(uint4*)(xmm + off) = hi;
            *(uint4*)(xmm + P + off) = mid;
            *(uint4*)(xmm + 2 * P + off) = lo;
        }
    }
    __syncthreads();
    wh_f32x4 total = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t dep = 0;
#pragma unroll
    for (int gb = 0; gb < kG; gb += kD) {
#pragma unroll
        for (int i = 0; i < kD; ++i) {
            const int gi = gb + i;
            {
                const uint4 lo4 = rw[i][0], hi4 = rw[i][1];
                const uint32_t dw[8] = {lo4.x + dep, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
                wh_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const wh_bf16x8 av = wh_fp8_bf16x8<kSpecial>(dw[2 * m], dw[2 * m + 1]);
                    const uint32_t xo = (((gi * 4 + m) * 4 + q) * 16 + (L & 15)) * 8;
                    const wh_bf16x8 bh = *(const wh_bf16x8*)(xmm + xo);
                    const wh_bf16x8 bm = *(const wh_bf16x8*)(xmm + P + xo);
                    const wh_bf16x8 bl = *(const wh_bf16x8*)(xmm + 2 * P + xo);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bh, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bm, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bl, acc, 0, 0, 0);
                }
                const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), gi));
#pragma unroll
                for (int r = 0; r < 4; ++r) total[r] = __builtin_fmaf(acc[r], s, total[r]);
                dep = wh_opaque_zero(acc[0]);
                // refill: group gi + kD into this slot, after this group's MFMAs
                if (gi + kD < kG) {
                    rw[i][0] = *(const uint4*)(wrow + 128 * (gi + kD) + dep);
                    rw[i][1] = *(const uint4*)(wrow + 128 * (gi + kD) + 16 + dep);
                }
            }
        }
    }
    // every lane's A and B fed the MFMAs; the stores below are per lane
    asm volatile("" : "+v"(total));
    // D[4 (L / 16) + r][L % 16]: row 16 wave + 4 q + r of the block, token L % 16
    const uint32_t t = L & 15, tg = tb * WH_FP8MM_TOK + t;
    if (a.splits == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t orow = r0 + 16 * wave + 4 * q + r;
            if (orow < row_end && tg < a.n) {
                Y[(size_t)tg * y_stride + (orow - row_start)] = total[r];
                if (!(fabsf(total[r]) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            }
        }
        return;
    }
    // partial tile of this split; the last workgroup of the row block sums
    // the splits in order
    const size_t tile = ((size_t)tb * a.row_blocks + rb) * a.splits;
    float* wsp = a.ws + (tile + ks) * (WH_FP8MM_ROWS * 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) wh_store_coherent(wsp + (16 * wave + 4 * q + r) * 16 + t, total[r]);
    wh_stores_done();
    __syncthreads();
    __shared__ uint32_t last;
    if (threadIdx.x == 0) {
        uint32_t* cnt = a.cnt + (size_t)tb * a.row_blocks + rb;
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old + 1 == a.splits;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // element e = threadIdx.x + 512 k of the tile: (row e / 16, token e % 16);
    // eight splits' loads are in flight before their sums
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* wt = a.ws + tile * (WH_FP8MM_ROWS * 16) + threadIdx.x;
    for (uint32_t sp0 = 0; sp0 < a.splits; sp0 += 8) {
        float v[8][4];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                v[j][k] = sp0 + j < a.splits ? wh_load_coherent(wt + (size_t)(sp0 + j) * (WH_FP8MM_ROWS * 16) + 512 * k)
                                             : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (sp0 + j < a.splits) {
#pragma unroll
                for (int k = 0; k < 4; ++k) sum[k] = j == 0 && sp0 == 0 ? v[j][k] : sum[k] + v[j][k];
            }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t e = threadIdx.x + 512 * k;
        const uint32_t orow = r0 + (e >> 4), ttg = tb * WH_FP8MM_TOK + (e & 15);
        if (orow < row_end && ttg < a.n) {
            Y[(size_t)ttg * y_stride + (orow - row_start)] = sum[k];
            if (!(fabsf(sum[k]) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        }
    }
}
