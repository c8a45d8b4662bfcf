// Decode-path kernels for gfx950: FP8 block-scaled GEMV, FP4 E2M1 matvec,
// activation quant-dequant, and the fused routed-expert SwiGLU pipeline.
// Launch helpers and the C ABI live in wohper_hip.hip.
#pragma once
#include "wh_device.h"

#ifndef WH_LIBM_TABLES_INCLUDED
#error "include the generated libm tables before kernels.h"
#endif

// glibc-exact libm tables (generated at build time, see gen_libm_tables.c)
__device__ const uint64_t kExpTab[35] = {WH_EXP2_TAB_INIT};
__device__ const uint32_t kLog2Thr[254] = {WH_LOG2F_THR_INIT};
__device__ const uint32_t kExpfFlip[WH_EXPF_FLIP_COUNT] = {WH_EXPF_FLIP_INIT};

// status word bits, OR-ed by kernels, read by the host after the stream syncs
#define WH_ST_NONFINITE_OUTPUT 1u
#define WH_ST_NONFINITE_INPUT 2u

#define WH_MAX_EXPERTS 16

// ------------------------------------------------------------------ shapes
// FP8 resident layout: per row, per 128-col group, lane l (0..7) owns 16
// contiguous bytes = cols {16c + l} (c = 0..7, the g0 chain) then
// {16c + 8 + l} (the g1 chain).  The x vector is staged in LDS in the same
// order, so one 16-byte global load and four ds_read_b128 feed a lane's group.
__device__ __forceinline__ uint32_t wh_fp8_lds_index(uint32_t col) {
    uint32_t g = col >> 7, w = col & 127, chunk = w >> 4, off = w & 15;
    uint32_t l = off & 7, i = (off >> 3) * 8 + chunk;
    return ((g * 8 + l) << 4) + i;
}

// FP4 resident layout: per row, per 256-col span (8 groups), lane l owns 16
// bytes = 4 dwords, dword d = groups 2d, 2d+1 of the span (see wh_fp4_decode8).
// x staged in LDS as xs[(g*8 + l)*4 + k] = x[32g + l + 8k].
__device__ __forceinline__ uint32_t wh_fp4_lds_index(uint32_t col) {
    uint32_t g = col >> 5, w = col & 31, k = w >> 3, l = w & 7;
    return ((g * 8 + l) << 2) + k;
}

// L1-bypassing load for data written by other workgroups of the same launch
__device__ __forceinline__ float wh_load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------- act-quant
// Standalone E/compute.rs:2504-2521 over n values in place, one workgroup per
// block of `block` values (any block size).  Non-finite values follow the
// reference's f32 semantics: an inf makes the block scale inf.
__global__ void __launch_bounds__(256) k_act_quant_inplace(float* __restrict__ v, uint32_t n,
                                                           uint32_t block) {
    __shared__ float red[4];
    uint32_t b0 = blockIdx.x * block;
    uint32_t b1 = min(b0 + block, n);
    float amax = 0.0f;
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) amax = fmaxf(amax, fabsf(v[i]));
    amax = wh_wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    amax = fmaxf(amax, 1.0e-4f);
    bool inf_scale = !(amax <= 3.4028235e38f);
    int k = inf_scale ? 0 : wh_aq_scale_exp(amax, kLog2Thr);
    float scale = inf_scale ? __uint_as_float(0x7f800000u) : wh_pow2f(k);
    float inv = inf_scale ? 0.0f : wh_pow2f(-k);
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) {
        float x = v[i];
        float t = inf_scale ? x / scale : x * inv;
        float q;
        if (t != t) {
            q = -480.0f;  // partition_point over NaN -> lut[0]
        } else {
            wh_e4m3_nearest(wh_clamp448(t), &q);
        }
        v[i] = q * scale;
    }
}

// Act-quant of a vector into E4M3 codes plus one f32 scale per 64-block
// (block size 64, as every call site of the expert path uses, E/deepseek_v4.rs:587,595).
// code * scale reproduces the reference's dequantized value exactly.
// One wave per block; x is f32 or bf16 (is_bf16).
__global__ void __launch_bounds__(64) k_act_quant_codes(const void* __restrict__ x, int is_bf16,
                                                        uint32_t n, uint8_t* __restrict__ codes,
                                                        float* __restrict__ scales,
                                                        uint32_t* __restrict__ status) {
    uint32_t i = blockIdx.x * 64 + threadIdx.x;
    float v = 0.0f;
    if (i < n) {
        if (is_bf16) v = __uint_as_float((uint32_t)((const uint16_t*)x)[i] << 16);
        else v = ((const float*)x)[i];
    }
    float amax = wh_wave_max(fabsf(v));
    if (!(amax <= 3.4028235e38f)) {  // inf or NaN input: reported, not quantized
        if (threadIdx.x == 0) atomicOr(status, WH_ST_NONFINITE_INPUT);
        amax = 1.0f;
    }
    int k = wh_aq_scale_exp(amax, kLog2Thr);
    float q;
    uint32_t code = wh_e4m3_nearest(wh_clamp448(v * wh_pow2f(-k)), &q);
    if (i < n) codes[i] = (uint8_t)code;
    if (threadIdx.x == 0) scales[blockIdx.x] = wh_pow2f(k);
}

// ------------------------------------------------------------- FP8 GEMV
struct wh_fp8_args {
    const uint8_t* w;       // resident (lane-permuted) bytes, rows x cols
    const void* scales;     // [scale_rows][scale_cols], f32 or UE8M0 bytes
    const float* x;         // cols
    float* y;               // row_end - row_start
    uint32_t* status;
    uint32_t cols, scale_cols, row_group, row_start, row_end;
    uint32_t x_stride, y_stride;  // batch strides (multi-input variant)
};

template <bool kSpecial, bool kScaleU8>
__device__ __forceinline__ float wh_fp8_scale(const void* s, uint32_t idx) {
    if constexpr (kScaleU8) return wh_ue8m0(((const uint8_t*)s)[idx]);
    else return ((const float*)s)[idx];
}

// Fast path: col_group == 128.  One thread = one (row, AVX lane); 256
// threads = 32 rows.  x staged in LDS (cols * 4 bytes).
template <bool kSpecial, bool kScaleU8>
__global__ void __launch_bounds__(256) k_fp8_gemv(wh_fp8_args a) {
    extern __shared__ float xs[];
    const uint32_t batch = blockIdx.y;
    const float* x = a.x + (size_t)batch * a.x_stride;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) xs[wh_fp8_lds_index(c)] = x[c];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 7;
    const uint32_t row = a.row_start + blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool active = row < a.row_end;
    const uint32_t groups = a.cols >> 7;
    float acc = 0.0f;
    if (active) {
        const uint4* wp = (const uint4*)(a.w + (size_t)row * a.cols) + lane;
        const uint32_t srow = (row / a.row_group) * a.scale_cols;
        const float4* xp = (const float4*)xs + lane * 4;
        uint4 wn = wp[0];
#pragma unroll 2
        for (uint32_t g = 0; g < groups; ++g) {
            uint4 wv = wn;
            if (g + 1 < groups) wn = wp[(g + 1) * 8];
            float s = wh_fp8_scale<kSpecial, kScaleU8>(a.scales, srow + g);
            const float4* xg = xp + g * 32;
            float4 x0 = xg[0], x1 = xg[1], x2 = xg[2], x3 = xg[3];
            wh_f2 w0 = wh_fp8x2<kSpecial, false>(wv.x), w1 = wh_fp8x2<kSpecial, true>(wv.x);
            wh_f2 w2 = wh_fp8x2<kSpecial, false>(wv.y), w3 = wh_fp8x2<kSpecial, true>(wv.y);
            wh_f2 w4 = wh_fp8x2<kSpecial, false>(wv.z), w5 = wh_fp8x2<kSpecial, true>(wv.z);
            wh_f2 w6 = wh_fp8x2<kSpecial, false>(wv.w), w7 = wh_fp8x2<kSpecial, true>(wv.w);
            float g0 = __builtin_fmaf(w0.x, x0.x, 0.0f);
            g0 = __builtin_fmaf(w0.y, x0.y, g0);
            g0 = __builtin_fmaf(w1.x, x0.z, g0);
            g0 = __builtin_fmaf(w1.y, x0.w, g0);
            g0 = __builtin_fmaf(w2.x, x1.x, g0);
            g0 = __builtin_fmaf(w2.y, x1.y, g0);
            g0 = __builtin_fmaf(w3.x, x1.z, g0);
            g0 = __builtin_fmaf(w3.y, x1.w, g0);
            float g1 = __builtin_fmaf(w4.x, x2.x, 0.0f);
            g1 = __builtin_fmaf(w4.y, x2.y, g1);
            g1 = __builtin_fmaf(w5.x, x2.z, g1);
            g1 = __builtin_fmaf(w5.y, x2.w, g1);
            g1 = __builtin_fmaf(w6.x, x3.x, g1);
            g1 = __builtin_fmaf(w6.y, x3.y, g1);
            g1 = __builtin_fmaf(w7.x, x3.z, g1);
            g1 = __builtin_fmaf(w7.y, x3.w, g1);
            acc = __builtin_fmaf(g0 + g1, s, acc);
        }
    }
    float sum = wh_hsum8(acc) + 0.0f;  // + tail (0 for col_group % 16 == 0)
    if (active && lane == 0) {
        a.y[(size_t)batch * a.y_stride + (row - a.row_start)] = sum;
        if (!(fabsf(sum) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
    }
}

// Generic path for any col_group: one thread per row emulating the 8 AVX2
// lanes, the scalar tail and `hsum256 + tail` exactly (E/compute.rs:5978-6018).
// Weights are in the original row-major order.
template <bool kScaleU8>
__global__ void __launch_bounds__(64) k_fp8_gemv_generic(wh_fp8_args a, uint32_t col_group) {
    const uint32_t batch = blockIdx.y;
    const float* x = a.x + (size_t)batch * a.x_stride;
    const uint32_t row = a.row_start + blockIdx.x * 64 + threadIdx.x;
    if (row >= a.row_end) return;
    const uint8_t* wr = a.w + (size_t)row * a.cols;
    const uint32_t srow = (row / a.row_group) * a.scale_cols;
    float acc[8];
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    float tail = 0.0f;
    const uint32_t chunks = col_group / 16;
    for (uint32_t g = 0; g < a.scale_cols; ++g) {
        float s = wh_fp8_scale<false, kScaleU8>(a.scales, srow + g);
        const uint8_t* b = wr + g * col_group;
        const float* xc = x + g * col_group;
        float g0[8], g1[8];
        for (int l = 0; l < 8; ++l) g0[l] = g1[l] = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            for (int l = 0; l < 8; ++l) {
                g0[l] = __builtin_fmaf(wh_fp8_exact(b[c * 16 + l]), xc[c * 16 + l], g0[l]);
                g1[l] = __builtin_fmaf(wh_fp8_exact(b[c * 16 + 8 + l]), xc[c * 16 + 8 + l], g1[l]);
            }
        }
        float rem = 0.0f;
        for (uint32_t i = chunks * 16; i < col_group; ++i) {
            float p = wh_fp8_exact(b[i]) * xc[i];
            rem = rem + p;
        }
        for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(g0[l] + g1[l], s, acc[l]);
        float rs = rem * s;
        tail = tail + rs;
    }
    float sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    sum = sum + tail;
    a.y[(size_t)batch * a.y_stride + (row - a.row_start)] = sum;
    if (!(fabsf(sum) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
}

// ------------------------------------------------------------- FP4 matvec
// One lane's contribution over a whole FP4 row in the resident layout: the
// 4-FMA group chain and acc = fma(gacc, scale * 0.125, acc) per group.
// xs: LDS-staged x (wh_fp4_lds_index order).  K = cols, multiple of 256.
__device__ __forceinline__ float wh_fp4_lane_dot(const uint8_t* __restrict__ wrow,
                                                 const uint8_t* __restrict__ srow, uint32_t K,
                                                 uint32_t lane, const float* xs) {
    const uint32_t spans = K >> 8;
    const uint4* wp = (const uint4*)wrow + lane;
    const float4* xp = (const float4*)xs + lane;
    float acc = 0.0f;
    uint4 wn = wp[0];
    for (uint32_t sp = 0; sp < spans; ++sp) {
        uint4 wv = wn;
        if (sp + 1 < spans) wn = wp[(sp + 1) * 8];
        uint2 sv = *(const uint2*)(srow + sp * 8);  // the span's 8 group scales
        uint32_t sw0 = sv.x, sw1 = sv.y;
        uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            wh_fp4x8 e = wh_fp4_decode8(words[d]);
            uint32_t ga = sp * 8 + d * 2;
            uint32_t sword = d < 2 ? sw0 : sw1;
            uint32_t sa = (sword >> ((d & 1) * 16)) & 0xff;
            uint32_t sb = (sword >> ((d & 1) * 16 + 8)) & 0xff;
            float4 xa = xp[ga * 8];
            float4 xb = xp[(ga + 1) * 8];
            float ca = __builtin_fmaf(e.a01.x, xa.x, 0.0f);
            ca = __builtin_fmaf(e.a01.y, xa.y, ca);
            ca = __builtin_fmaf(e.a23.x, xa.z, ca);
            ca = __builtin_fmaf(e.a23.y, xa.w, ca);
            acc = __builtin_fmaf(ca, wh_ue8m0(sa) * 0.125f, acc);
            float cb = __builtin_fmaf(e.b01.x, xb.x, 0.0f);
            cb = __builtin_fmaf(e.b01.y, xb.y, cb);
            cb = __builtin_fmaf(e.b23.x, xb.z, cb);
            cb = __builtin_fmaf(e.b23.y, xb.w, cb);
            acc = __builtin_fmaf(cb, wh_ue8m0(sb) * 0.125f, acc);
        }
    }
    return acc;
}

struct wh_fp4_args {
    const uint8_t* w;  // resident
    const uint8_t* s;  // [rows][cols/32]
    const float* x;
    float* y;
    uint32_t* status;
    uint32_t rows, cols;
};

// Fast path: group_cols == 32, cols % 256 == 0.  256 threads = 32 rows.
__global__ void __launch_bounds__(256) k_fp4_matvec(wh_fp4_args a) {
    extern __shared__ float xs[];
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) xs[wh_fp4_lds_index(c)] = a.x[c];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 7;
    const uint32_t row = blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool active = row < a.rows;
    float acc = 0.0f;
    if (active)
        acc = wh_fp4_lane_dot(a.w + (size_t)row * (a.cols / 2), a.s + (size_t)row * (a.cols / 32),
                              a.cols, lane, xs);
    float sum = wh_hsum8(acc) + 0.0f;
    if (active && lane == 0) {
        a.y[row] = sum;
        if (!(fabsf(sum) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
    }
}

// Generic FP4 path, original packed layout, one thread per row, following
// the reference dispatch (E/deepseek_v4.rs:472-548): the AVX2 lane
// emulation when cols and group_cols are even, else the per-element path.
__global__ void __launch_bounds__(64) k_fp4_matvec_generic(wh_fp4_args a, uint32_t scale_cols) {
    const uint32_t row = blockIdx.x * 64 + threadIdx.x;
    if (row >= a.rows) return;
    const uint32_t row_bytes = (a.cols + 1) / 2;
    const uint32_t group_cols = a.cols / scale_cols;
    const uint8_t* wr = a.w + (size_t)row * row_bytes;
    const uint8_t* sr = a.s + (size_t)row * scale_cols;
    float sum;
    if (a.cols % 2 == 0 && group_cols % 2 == 0) {
        const uint32_t gbytes = group_cols / 2, chunks = gbytes / 16;
        float acc[8];
        for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
        float tail = 0.0f;
        for (uint32_t g = 0; g < scale_cols; ++g) {
            float s = wh_ue8m0(sr[g]);
            const uint8_t* b = wr + g * gbytes;
            const float* xc = a.x + g * group_cols;
            float ga[8];
            for (int l = 0; l < 8; ++l) ga[l] = 0.0f;
            for (uint32_t c = 0; c < chunks; ++c) {
                for (int k = 0; k < 4; ++k) {
                    for (int l = 0; l < 8; ++l) {
                        uint32_t col = k * 8 + l;  // column within the 32-col chunk
                        uint32_t byte = b[c * 16 + col / 2];
                        uint32_t nib = (col & 1) ? byte >> 4 : byte & 15;
                        ga[l] = __builtin_fmaf(wh_fp4_x8(nib), xc[c * 32 + col], ga[l]);
                    }
                }
            }
            float s8 = s * 0.125f;
            for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(ga[l], s8, acc[l]);
            float rem = 0.0f;
            for (uint32_t i = chunks * 16; i < gbytes; ++i) {
                float p0 = wh_fp4_base(b[i] & 15) * xc[2 * i];
                rem = rem + p0;
                float p1 = wh_fp4_base(b[i] >> 4) * xc[2 * i + 1];
                rem = rem + p1;
            }
            float rs = rem * s;
            tail = tail + rs;
        }
        sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
        sum = sum + tail;
    } else {
        sum = 0.0f;
        for (uint32_t col = 0; col < a.cols; ++col) {
            uint32_t byte = wr[col / 2];
            uint32_t nib = (col & 1) ? byte >> 4 : byte & 15;
            float s = wh_ue8m0(sr[col / group_cols]);
            float b = wh_fp4_base(nib);
            float v = b == 0.0f ? 0.0f : b * s;  // decode_fp4_e2m1(nibble, scale)
            float p = v * a.x[col];
            sum = sum + p;
        }
    }
    a.y[row] = sum;
    if (!(fabsf(sum) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
}

// --------------------------------------------------- routed expert pipeline
struct wh_expert_ptrs {
    const uint8_t* w1;
    const uint8_t* s1;
    const uint8_t* w3;
    const uint8_t* s3;
    const uint8_t* w2;
    const uint8_t* s2;
};

struct wh_moe_args {
    wh_expert_ptrs ex[WH_MAX_EXPERTS];
    float route_w[WH_MAX_EXPERTS];
    uint32_t n_experts;
    uint32_t hidden, inter;        // w1/w3: inter x hidden, w2: hidden x inter
    uint32_t n_tokens;             // tokens sharing the same expert list (1 for decode)
    const uint8_t* xq_codes;       // [n_tokens][hidden] act-quant codes of x
    const float* xq_scales;        // [n_tokens][hidden/64]
    float* h;                      // [n_tokens][n_experts][inter] swiglu hidden (pre-quant)
    uint8_t* hq_codes;             // [n_tokens][n_experts][inter]
    float* hq_scales;              // [n_tokens][n_experts][inter/64]
    float* y;                      // [n_tokens][n_experts][hidden] per-expert outputs
    float* out;                    // [n_tokens][hidden] routed sum
    uint32_t* cnt_h;               // [n_tokens][n_experts][inter/64] arrival counters
    uint32_t* cnt_y;               // [n_tokens][hidden/32] arrival counters
    uint32_t* status;
};

// Stage an act-quantized vector (codes + per-64 scales) into LDS in the
// FP4 lane order.
__device__ __forceinline__ void wh_stage_codes_fp4(float* xs, const uint8_t* codes,
                                                   const float* scales, uint32_t n) {
    for (uint32_t c = threadIdx.x; c < n; c += blockDim.x) {
        wh_f2 v = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[c], false);
        xs[wh_fp4_lds_index(c)] = v.x * scales[c >> 6];
    }
}

// Gate/up + SwiGLU + act-quant of the hidden.  Grid: (inter/16, n_experts,
// n_tokens); 128 threads = 16 rows x 8 lanes, each lane running both the w1
// and w3 row (E/deepseek_v4.rs:588-594).  The last of the 4 workgroups that
// complete a 64-row block quantizes it (E/deepseek_v4.rs:595).
__global__ void __launch_bounds__(128) k_moe_gateup(wh_moe_args a) {
    extern __shared__ float xs[];
    __shared__ uint32_t last;
    const uint32_t e = blockIdx.y, tok = blockIdx.z;
    const wh_expert_ptrs ep = a.ex[e];
    wh_stage_codes_fp4(xs, a.xq_codes + (size_t)tok * a.hidden, a.xq_scales + (size_t)tok * (a.hidden / 64),
                       a.hidden);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 7;
    const uint32_t row = blockIdx.x * 16 + (threadIdx.x >> 3);
    const size_t rb = (size_t)row * (a.hidden / 2), sb = (size_t)row * (a.hidden / 32);
    float g = wh_fp4_lane_dot(ep.w1 + rb, ep.s1 + sb, a.hidden, lane, xs);
    float u = wh_fp4_lane_dot(ep.w3 + rb, ep.s3 + sb, a.hidden, lane, xs);
    g = wh_hsum8(g) + 0.0f;
    u = wh_hsum8(u) + 0.0f;
    const size_t hbase = ((size_t)tok * a.n_experts + e) * a.inter;
    if (lane == 0) {
        if (!(fabsf(g) <= 3.4028235e38f) || !(fabsf(u) <= 3.4028235e38f)) {
            atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        }
        a.h[hbase + row] = wh_swiglu(g, u, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT);
    }
    __threadfence();
    __syncthreads();
    const uint32_t blk = row >> 6;
    uint32_t* cnt = a.cnt_h + ((size_t)tok * a.n_experts + e) * (a.inter / 64) + blk;
    if (threadIdx.x == 0) last = atomicAdd(cnt, 1u) == 3u;
    __syncthreads();
    if (!last || threadIdx.x >= 64) return;
    __threadfence();
    float v = wh_load_coherent(a.h + hbase + blk * 64 + threadIdx.x);
    float amax = wh_wave_max(fabsf(v));
    if (!(amax <= 3.4028235e38f)) amax = 1.0f;  // non-finite rows already reported
    int k = wh_aq_scale_exp(amax, kLog2Thr);
    float q;
    uint32_t code = wh_e4m3_nearest(wh_clamp448(v * wh_pow2f(-k)), &q);
    a.hq_codes[hbase + blk * 64 + threadIdx.x] = (uint8_t)code;
    if (threadIdx.x == 0) {
        a.hq_scales[hbase / 64 + blk] = wh_pow2f(k);
        *cnt = 0u;  // ready for the next launch
    }
}

// Down projection + ordered routed sum.  Grid: (hidden/32, n_experts,
// n_tokens); 256 threads = 32 rows x 8 lanes.  The last expert to finish a
// 32-row block combines all experts in route order (E/compute.rs:1948-2012).
__global__ void __launch_bounds__(256) k_moe_down(wh_moe_args a) {
    extern __shared__ float xs[];
    __shared__ uint32_t last;
    const uint32_t e = blockIdx.y, tok = blockIdx.z;
    const wh_expert_ptrs ep = a.ex[e];
    const size_t hbase = ((size_t)tok * a.n_experts + e) * a.inter;
    wh_stage_codes_fp4(xs, a.hq_codes + hbase, a.hq_scales + hbase / 64, a.inter);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 7;
    const uint32_t row = blockIdx.x * 32 + (threadIdx.x >> 3);
    float acc = wh_fp4_lane_dot(ep.w2 + (size_t)row * (a.inter / 2), ep.s2 + (size_t)row * (a.inter / 32),
                                a.inter, lane, xs);
    float yv = wh_hsum8(acc) + 0.0f;
    const size_t ybase = ((size_t)tok * a.n_experts + e) * a.hidden;
    if (lane == 0) {
        if (!(fabsf(yv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        a.y[ybase + row] = yv;
    }
    __threadfence();
    __syncthreads();
    uint32_t* cnt = a.cnt_y + (size_t)tok * (a.hidden / 32) + blockIdx.x;
    if (threadIdx.x == 0) last = atomicAdd(cnt, 1u) == a.n_experts - 1;
    __syncthreads();
    if (!last || threadIdx.x >= 32) return;
    __threadfence();
    const uint32_t r = blockIdx.x * 32 + threadIdx.x;
    const size_t t0 = (size_t)tok * a.n_experts * a.hidden;
    float o;
    if (a.n_experts == 1) {
        o = wh_load_coherent(a.y + t0 + r);
    } else {
        // valid_route_weight_sum (E/compute.rs:2014-2030)
        float sum = 0.0f;
        bool valid = true;
        for (uint32_t i = 0; i < a.n_experts; ++i) {
            float w = a.route_w[i];
            if (!(fabsf(w) <= 3.4028235e38f && w >= 0.0f)) valid = false;
            sum = sum + w;
        }
        if (sum <= 1.1920929e-07f) valid = false;
        float uniform = 1.0f / (float)a.n_experts;
        o = 0.0f;
        for (uint32_t i = 0; i < a.n_experts; ++i) {
            float w = valid ? a.route_w[i] / sum : uniform;
            float p = wh_load_coherent(a.y + t0 + (size_t)i * a.hidden + r) * w;
            o = o + p;
        }
    }
    a.out[(size_t)tok * a.hidden + r] = o;
    if (threadIdx.x == 0) *cnt = 0u;
}

// Bit-exact dequant of a resident FP4 tensor back to reference values
// (decode_fp4_e2m1(nibble, scale), E/deepseek_v4.rs:358-372), through the
// same decode the matvec uses: out = (x8 value) * 0.125 * scale.
__global__ void __launch_bounds__(256) k_fp4_dequant(const uint8_t* __restrict__ w,
                                                     const uint8_t* __restrict__ s, uint32_t rows,
                                                     uint32_t cols, float* __restrict__ out) {
    // one thread per (row, span, lane): 32 values
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t spans = cols >> 8;
    if (t >= (size_t)rows * spans * 8) return;
    const uint32_t lane = t & 7, sp = (t >> 3) % spans, row = (t >> 3) / spans;
    uint4 wv = ((const uint4*)(w + (size_t)row * (cols / 2)))[sp * 8 + lane];
    uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
    for (int d = 0; d < 4; ++d) {
        wh_fp4x8 v = wh_fp4_decode8(words[d]);
        float va[4] = {v.a01.x, v.a01.y, v.a23.x, v.a23.y};
        float vb[4] = {v.b01.x, v.b01.y, v.b23.x, v.b23.y};
        uint32_t ga = sp * 8 + d * 2;
        float sa = wh_ue8m0(s[(size_t)row * (cols / 32) + ga]);
        float sb = wh_ue8m0(s[(size_t)row * (cols / 32) + ga + 1]);
        for (int k = 0; k < 4; ++k) {
            // sign * value * scale with value = x8/8 (exact), zero -> +0
            float a8 = va[k] * 0.125f, b8 = vb[k] * 0.125f;
            out[(size_t)row * cols + ga * 32 + lane + 8 * k] = a8 == 0.0f ? 0.0f : a8 * sa;
            out[(size_t)row * cols + (ga + 1) * 32 + lane + 8 * k] = b8 == 0.0f ? 0.0f : b8 * sb;
        }
    }
}

// Bit-exact dequant of a resident FP8 tensor (base values, no scale):
// decode_fp8_e4m3(byte, 1.0) in original column order.
template <bool kSpecial>
__global__ void __launch_bounds__(256) k_fp8_dequant(const uint8_t* __restrict__ w, uint32_t rows,
                                                     uint32_t cols, float* __restrict__ out) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t groups = cols >> 7;
    if (t >= (size_t)rows * groups * 8) return;
    const uint32_t lane = t & 7, g = (t >> 3) % groups, row = (t >> 3) / groups;
    uint4 wv = ((const uint4*)(w + (size_t)row * cols))[g * 8 + lane];
    uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
    for (int d = 0; d < 4; ++d) {
        wh_f2 lo = wh_fp8x2<kSpecial, false>(words[d]), hi = wh_fp8x2<kSpecial, true>(words[d]);
        float v[4] = {lo.x, lo.y, hi.x, hi.y};
        for (int k = 0; k < 4; ++k) {
            uint32_t i = d * 4 + k;  // position within the lane's 16 bytes
            uint32_t col = g * 128 + (i & 7) * 16 + (i >> 3) * 8 + lane;
            out[(size_t)row * cols + col] = v[k] == 0.0f ? 0.0f : v[k];
        }
    }
}

// Test support: evaluates the device libm emulation on an array.
// fn 0: silu(x), 1: expf(x) (x >= -10), 2: 2^ceil(log2f(max(x,1e-4)/448)).
__global__ void k_debug_eval(int fn, const float* __restrict__ in, float* __restrict__ out, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float x = in[i];
    float r;
    if (fn == 0) r = wh_silu(x, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT);
    else if (fn == 1) r = wh_expf_glibc(x, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT);
    else r = wh_pow2f(wh_aq_scale_exp(x, kLog2Thr));
    out[i] = r;
}
