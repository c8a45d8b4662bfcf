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

// FP4 matvec input order in LDS (the weight layout is described with the FP4
// kernels below): xs[(g*8 + l)*4 + k] = x[32g + l + 8k], so AVX lane l's four
// columns of group g are one float4.
__device__ __forceinline__ uint32_t wh_fp4_lds_index(uint32_t col) {
    uint32_t g = col >> 5, w = col & 31, k = w >> 3, l = w & 7;
    return ((g * 8 + l) << 2) + k;
}

// Cross-workgroup hand-off inside one launch.  The 8 XCDs of an MI355X have
// separate L2s, so an agent-scope fence writes back and invalidates the whole
// L2 - far too costly per workgroup.  Instead the few values that cross
// workgroups are written and read with agent-scope relaxed atomics (coherent
// at the device level), each writer waits for its stores to complete, and an
// agent-scope atomic counter elects the last arriver.
__device__ __forceinline__ float wh_load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wh_store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's stores have completed (no cache maintenance).
__device__ __forceinline__ void wh_stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ uint32_t wh_arrive(uint32_t* cnt) {
    return __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------- LDS staging
// x is staged into LDS in two phases so that a kernel can issue its staging
// loads, then its weight loads, and only then wait for the staging data:
// the weight stream is in flight while x lands in LDS.

// FP4 lane order from f32 x: one 32-col group per thread.
struct wh_stage_f32_fp4 {
    float4 v[8];
    uint32_t g;
    bool on;
};
__device__ __forceinline__ void wh_stage_f32_fp4_load(wh_stage_f32_fp4& st, const float* x, uint32_t n, uint32_t g) {
    st.g = g;
    st.on = g < n / 32;
    if (st.on) {
#pragma unroll
        for (int q = 0; q < 8; ++q) st.v[q] = ((const float4*)x)[8 * g + q];
    }
}
__device__ __forceinline__ float wh_f4_get(const float4& v, int c) {
    return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}
__device__ __forceinline__ void wh_stage_fp4_store_group(float* xs, uint32_t g, const float* v32) {
#pragma unroll
    for (int l = 0; l < 8; ++l)
        ((float4*)xs)[g * 8 + l] = make_float4(v32[l], v32[8 + l], v32[16 + l], v32[24 + l]);
}
__device__ __forceinline__ void wh_stage_f32_fp4_store(const wh_stage_f32_fp4& st, float* xs) {
    if (!st.on) return;
    float v[32];
#pragma unroll
    for (int m = 0; m < 32; ++m) v[m] = wh_f4_get(st.v[m >> 2], m & 3);
    wh_stage_fp4_store_group(xs, st.g, v);
}

// FP4 lane order from act-quant codes (E4M3 bytes + one scale per 64).
struct wh_stage_codes {
    uint4 c0, c1;
    float sc;
    uint32_t g;
    bool on;
};
__device__ __forceinline__ void wh_stage_codes_load(wh_stage_codes& st, const uint8_t* codes, const float* scales,
                                                    uint32_t n, uint32_t g) {
    st.g = g;
    st.on = g < n / 32;
    if (st.on) {
        st.c0 = ((const uint4*)codes)[2 * g];
        st.c1 = ((const uint4*)codes)[2 * g + 1];
        st.sc = scales[g >> 1];
    }
}
__device__ __forceinline__ void wh_stage_codes_store(const wh_stage_codes& st, float* xs) {
    if (!st.on) return;
    const uint32_t words[8] = {st.c0.x, st.c0.y, st.c0.z, st.c0.w, st.c1.x, st.c1.y, st.c1.z, st.c1.w};
    float v[32];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        wh_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[d], false);
        wh_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[d], true);
        v[4 * d + 0] = lo.x * st.sc;
        v[4 * d + 1] = lo.y * st.sc;
        v[4 * d + 2] = hi.x * st.sc;
        v[4 * d + 3] = hi.y * st.sc;
    }
    wh_stage_fp4_store_group(xs, st.g, v);
}
// Whole-vector variants (any n, looping over groups).
__device__ __forceinline__ void wh_stage_codes_all(float* xs, const uint8_t* codes, const float* scales, uint32_t n) {
    for (uint32_t g = threadIdx.x; g < n / 32; g += blockDim.x) {
        wh_stage_codes st;
        wh_stage_codes_load(st, codes, scales, n, g);
        wh_stage_codes_store(st, xs);
    }
}

// FP8 lane order from f32 x: one 16-col chunk per thread.
struct wh_stage_f32_fp8 {
    float4 v[4];
    uint32_t q;
    bool on;
};
__device__ __forceinline__ void wh_stage_f32_fp8_load(wh_stage_f32_fp8& st, const float* x, uint32_t n, uint32_t q) {
    st.q = q;
    st.on = q < n / 16;
    if (st.on) {
#pragma unroll
        for (int i = 0; i < 4; ++i) st.v[i] = ((const float4*)x)[4 * q + i];
    }
}
__device__ __forceinline__ void wh_stage_f32_fp8_store(const wh_stage_f32_fp8& st, float* xs) {
    if (!st.on) return;
    const uint32_t g = st.q >> 3, c = st.q & 7;
#pragma unroll
    for (int o = 0; o < 16; ++o) {
        const uint32_t l = o & 7, i = (o >> 3) * 8 + c;
        xs[((g * 8 + l) << 4) + i] = wh_f4_get(st.v[o >> 2], o & 3);
    }
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

// One 128-col group of one AVX lane: two 8-FMA chains (g0 over cols
// 16c + l, g1 over 16c + 8 + l), then acc = fma(g0 + g1, scale, acc).
template <bool kSpecial>
__device__ __forceinline__ float wh_fp8_lane_group(uint4 wv, const float4* xg, float s, float acc) {
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
    return __builtin_fmaf(g0 + g1, s, acc);
}

// Fast path: col_group == 128.  One thread = one (row, AVX lane); 256
// threads = 32 rows.  x staged in LDS (cols * 4 bytes).  Weights stream in
// blocks of kBlk groups, double-buffered, so every lane keeps up to
// 2 * kBlk 16-byte loads in flight (the path is latency-bound otherwise).
template <bool kSpecial, bool kScaleU8>
__global__ void __launch_bounds__(256) k_fp8_gemv(wh_fp8_args a) {
    constexpr uint32_t kBlk = 8;
    extern __shared__ __align__(16) float xs[];
    const uint32_t batch = blockIdx.y;
    const float* x = a.x + (size_t)batch * a.x_stride;
    const uint32_t lane = threadIdx.x & 7;
    const uint32_t row = a.row_start + blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool active = row < a.row_end;
    const uint32_t groups = a.cols >> 7;
    const uint4* wp = (const uint4*)(a.w + (size_t)(active ? row : a.row_start) * a.cols) + lane;
    const uint32_t srow = ((active ? row : a.row_start) / a.row_group) * a.scale_cols;
    wh_stage_f32_fp8 st;
    wh_stage_f32_fp8_load(st, x, a.cols, threadIdx.x);
    uint4 nxt[kBlk];
    float snxt[kBlk];
#pragma unroll
    for (uint32_t i = 0; i < kBlk; ++i) {
        if (active && i < groups) {
            nxt[i] = wp[i * 8];
            snxt[i] = wh_fp8_scale<kSpecial, kScaleU8>(a.scales, srow + i);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    wh_stage_f32_fp8_store(st, xs);
    for (uint32_t q = threadIdx.x + 256; q < a.cols / 16; q += 256) {  // cols > 4096
        wh_stage_f32_fp8 s2;
        wh_stage_f32_fp8_load(s2, x, a.cols, q);
        wh_stage_f32_fp8_store(s2, xs);
    }
    __syncthreads();
    float acc = 0.0f;
    if (active) {
        const float4* xp = (const float4*)xs + lane * 4;
        for (uint32_t g0 = 0; g0 < groups; g0 += kBlk) {
            uint4 cur[kBlk];
            float scur[kBlk];
#pragma unroll
            for (uint32_t i = 0; i < kBlk; ++i) {
                cur[i] = nxt[i];
                scur[i] = snxt[i];
            }
#pragma unroll
            for (uint32_t i = 0; i < kBlk; ++i) {
                if (g0 + kBlk + i < groups) {
                    nxt[i] = wp[(g0 + kBlk + i) * 8];
                    snxt[i] = wh_fp8_scale<kSpecial, kScaleU8>(a.scales, srow + g0 + kBlk + i);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (uint32_t i = 0; i < kBlk; ++i)
                if (g0 + i < groups) acc = wh_fp8_lane_group<kSpecial>(cur[i], xp + (g0 + i) * 32, scur[i], acc);
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
// Resident FP4 layout (fast path: group_cols == 32, cols % 512 == 0).  A row
// is run by a quad of 4 threads; thread t owns AVX lanes t and t + 4.
//   weights: chunk j = groups 4j..4j+3 (64 bytes of the row); thread t's 16
//            bytes sit at (4j + t) * 16, dword i = group 4j + i, encoded by
//            wh_fp4_encode_word with A = lane t, B = lane t + 4;
//   scales:  thread t owns the UE8M0 bytes of groups t, t+4, t+8, ... stored
//            contiguously: byte t * (G/4) + j is the scale of group 4j + t.
// Each thread decodes one scale per chunk and the quad shares it through a
// DPP broadcast fused into the accumulate FMA.
__host__ __device__ inline uint32_t wh_fp4_encode_word(const uint32_t* a, const uint32_t* b) {
    uint32_t word = 0;
    for (uint32_t k = 0; k < 4; ++k) {
        uint32_t ap = a[(k + 3) & 3];
        uint32_t byte = (a[k] & 7) | ((ap >> 3) << 3) | ((b[k] & 7) << 4) | ((b[k] >> 3) << 7);
        word |= byte << (8 * k);
    }
    return word;
}

template <int kI>
__device__ __forceinline__ float wh_quad_bcast(float v) {  // quad_perm [kI,kI,kI,kI]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kI * 0x55, 0xf, 0xf, false));
}

// Group 4j + kI of one quad thread: two 4-FMA chains (lanes t and t+4) on the
// x8 values, then acc = fma(gacc, scale / 8, acc) per lane.
template <int kI>
__device__ __forceinline__ void wh_fp4_quad_group_x(uint32_t word, float4 xa, float4 xb, float smine,
                                                    float& acc_a, float& acc_b) {
    wh_fp4x8 e = wh_fp4_decode8(word);
    float ga = __builtin_fmaf(e.a01.x, xa.x, 0.0f);
    ga = __builtin_fmaf(e.a01.y, xa.y, ga);
    ga = __builtin_fmaf(e.a23.x, xa.z, ga);
    ga = __builtin_fmaf(e.a23.y, xa.w, ga);
    float gb = __builtin_fmaf(e.b01.x, xb.x, 0.0f);
    gb = __builtin_fmaf(e.b01.y, xb.y, gb);
    gb = __builtin_fmaf(e.b23.x, xb.z, gb);
    gb = __builtin_fmaf(e.b23.y, xb.w, gb);
    float s8 = wh_quad_bcast<kI>(smine);
    acc_a = __builtin_fmaf(ga, s8, acc_a);
    acc_b = __builtin_fmaf(gb, s8, acc_b);
}

template <int kI>
__device__ __forceinline__ void wh_fp4_quad_group(uint32_t word, const float4* xg, uint32_t t,
                                                  float smine, float& acc_a, float& acc_b) {
    wh_fp4x8 e = wh_fp4_decode8(word);
    float4 xa = xg[t], xb = xg[t + 4];
    float ga = __builtin_fmaf(e.a01.x, xa.x, 0.0f);
    ga = __builtin_fmaf(e.a01.y, xa.y, ga);
    ga = __builtin_fmaf(e.a23.x, xa.z, ga);
    ga = __builtin_fmaf(e.a23.y, xa.w, ga);
    float gb = __builtin_fmaf(e.b01.x, xb.x, 0.0f);
    gb = __builtin_fmaf(e.b01.y, xb.y, gb);
    gb = __builtin_fmaf(e.b23.x, xb.z, gb);
    gb = __builtin_fmaf(e.b23.y, xb.w, gb);
    float s8 = wh_quad_bcast<kI>(smine);
    acc_a = __builtin_fmaf(ga, s8, acc_a);
    acc_b = __builtin_fmaf(gb, s8, acc_b);
}

__device__ __forceinline__ void wh_fp4_quad_chunk(uint4 w, uint32_t sbyte, uint32_t j, const float4* xp,
                                                  uint32_t t, float& acc_a, float& acc_b) {
    float smine = wh_ue8m0(sbyte) * 0.125f;
    const float4* xg = xp + j * 32;  // group 4j at float4 index (4j * 8)
    wh_fp4_quad_group<0>(w.x, xg, t, smine, acc_a, acc_b);
    wh_fp4_quad_group<1>(w.y, xg + 8, t, smine, acc_a, acc_b);
    wh_fp4_quad_group<2>(w.z, xg + 16, t, smine, acc_a, acc_b);
    wh_fp4_quad_group<3>(w.w, xg + 24, t, smine, acc_a, acc_b);
}

// A quad thread's whole row in registers (kChunks known at compile time:
// 32 for K = 4096, 16 for K = 2048): every load is issued before any math,
// since one token's matvec is a single latency-bound sweep.
template <int kChunks>
struct wh_fp4_rowbuf {
    uint4 w[kChunks];
    uint32_t sw[kChunks / 4];
};

template <int kChunks>
__device__ __forceinline__ void wh_fp4_rowbuf_load(wh_fp4_rowbuf<kChunks>& b, const uint8_t* __restrict__ wrow,
                                                   const uint8_t* __restrict__ srow, uint32_t t) {
    const uint4* wp = (const uint4*)wrow + t;
    const uint32_t* sp = (const uint32_t*)(srow + t * kChunks);
#pragma unroll
    for (int q = 0; q < kChunks / 4; ++q) b.sw[q] = sp[q];
#pragma unroll
    for (int j = 0; j < kChunks; ++j) b.w[j] = wp[4 * j];
}

// The x values of chunk j + 1 are read from LDS while chunk j computes, so
// the LDS latency is hidden even at one wave per SIMD.
template <int kChunks>
__device__ __forceinline__ void wh_fp4_rowbuf_dot(const wh_fp4_rowbuf<kChunks>& b, const float* xs, uint32_t t,
                                                  float& acc_a, float& acc_b) {
    const float4* xp = (const float4*)xs + t;
    acc_a = 0.0f;
    acc_b = 0.0f;
    float4 xc[8], xn[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xc[2 * i] = xp[i * 8];
        xc[2 * i + 1] = xp[i * 8 + 4];
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
        if (j + 1 < kChunks) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xn[2 * i] = xp[((j + 1) * 4 + i) * 8];
                xn[2 * i + 1] = xp[((j + 1) * 4 + i) * 8 + 4];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        const float smine = wh_ue8m0((b.sw[j >> 2] >> (8 * (j & 3))) & 0xffu) * 0.125f;
        wh_fp4_quad_group_x<0>(b.w[j].x, xc[0], xc[1], smine, acc_a, acc_b);
        wh_fp4_quad_group_x<1>(b.w[j].y, xc[2], xc[3], smine, acc_a, acc_b);
        wh_fp4_quad_group_x<2>(b.w[j].z, xc[4], xc[5], smine, acc_a, acc_b);
        wh_fp4_quad_group_x<3>(b.w[j].w, xc[6], xc[7], smine, acc_a, acc_b);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) xc[i] = xn[i];
    }
}

// Runtime chunk count (multiple of 4), blocks of 4 chunks double-buffered.
__device__ __forceinline__ void wh_fp4_quad_dot_rt(const uint8_t* __restrict__ wrow, const uint8_t* __restrict__ srow,
                                                   uint32_t chunks, uint32_t t, const float* xs, float& acc_a,
                                                   float& acc_b) {
    const uint4* wp = (const uint4*)wrow + t;
    const uint32_t* sp = (const uint32_t*)(srow + t * chunks);
    const float4* xp = (const float4*)xs;
    acc_a = 0.0f;
    acc_b = 0.0f;
    uint4 n0 = wp[0], n1 = wp[4], n2 = wp[8], n3 = wp[12];
    uint32_t ns = sp[0];
    for (uint32_t j = 0; j < chunks; j += 4) {
        uint4 c0 = n0, c1 = n1, c2 = n2, c3 = n3;
        uint32_t cs = ns;
        if (j + 4 < chunks) {
            n0 = wp[4 * (j + 4)];
            n1 = wp[4 * (j + 5)];
            n2 = wp[4 * (j + 6)];
            n3 = wp[4 * (j + 7)];
            ns = sp[(j + 4) >> 2];
        }
        wh_fp4_quad_chunk(c0, cs & 0xffu, j, xp, t, acc_a, acc_b);
        wh_fp4_quad_chunk(c1, (cs >> 8) & 0xffu, j + 1, xp, t, acc_a, acc_b);
        wh_fp4_quad_chunk(c2, (cs >> 16) & 0xffu, j + 2, xp, t, acc_a, acc_b);
        wh_fp4_quad_chunk(c3, cs >> 24, j + 3, xp, t, acc_a, acc_b);
    }
}

// The AVX2 horizontal sum ((l0+l1)+(l2+l3)) + ((l4+l5)+(l6+l7)) over the
// quad's (lane t, lane t+4) accumulators; valid in quad thread 0.
__device__ __forceinline__ float wh_quad_hsum(float acc_a, float acc_b) {
    float p = acc_a + wh_dpp_quad_swap1(acc_a);
    p = p + wh_dpp_quad_swap2(p);
    float q = acc_b + wh_dpp_quad_swap1(acc_b);
    q = q + wh_dpp_quad_swap2(q);
    return p + q;
}

struct wh_fp4_args {
    const uint8_t* w;  // resident
    const uint8_t* s;  // resident scales
    const float* x;
    float* y;
    uint32_t* status;
    uint32_t rows, cols;
};

// Fast path: 256 threads = 64 rows (one quad per row).  kChunks = cols/128
// when it is 16 or 32 (row fully in registers), else 0 (runtime loop).
template <int kChunks>
__global__ void __launch_bounds__(256) k_fp4_matvec(wh_fp4_args a) {
    extern __shared__ __align__(16) float xs[];
    const uint32_t t = threadIdx.x & 3;
    const uint32_t row = blockIdx.x * 64 + (threadIdx.x >> 2);
    const bool active = row < a.rows;
    const uint32_t rr = active ? row : 0;
    const uint8_t* wrow = a.w + (size_t)rr * (a.cols / 2);
    const uint8_t* srow = a.s + (size_t)rr * (a.cols / 32);
    float acc_a = 0.0f, acc_b = 0.0f;
    if constexpr (kChunks > 0) {
        wh_stage_f32_fp4 st;
        wh_stage_f32_fp4_load(st, a.x, a.cols, threadIdx.x);
        wh_fp4_rowbuf<kChunks> b;
        wh_fp4_rowbuf_load<kChunks>(b, wrow, srow, t);
        __builtin_amdgcn_sched_barrier(0);
        wh_stage_f32_fp4_store(st, xs);
        __syncthreads();
        wh_fp4_rowbuf_dot<kChunks>(b, xs, t, acc_a, acc_b);
    } else {
        for (uint32_t g = threadIdx.x; g < a.cols / 32; g += 256) {
            wh_stage_f32_fp4 st;
            wh_stage_f32_fp4_load(st, a.x, a.cols, g);
            wh_stage_f32_fp4_store(st, xs);
        }
        __syncthreads();
        wh_fp4_quad_dot_rt(wrow, srow, a.cols >> 7, t, xs, acc_a, acc_b);
    }
    float sum = wh_quad_hsum(acc_a, acc_b) + 0.0f;  // + tail (0 here)
    if (active && t == 0) {
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

// Gate/up + SwiGLU + act-quant of the hidden.  Grid: (inter/16, n_experts,
// n_tokens); 128 threads = 32 quads = 16 rows x {w1, w3}: quad 2r runs w1
// row r and quad 2r+1 the w3 row r (E/deepseek_v4.rs:588-594).  The last of
// the 4 workgroups that complete a 64-row block quantizes it
// (E/deepseek_v4.rs:595).
template <int kChunks>
__global__ void __launch_bounds__(128) k_moe_gateup(wh_moe_args a) {
    extern __shared__ __align__(16) float xs[];
    __shared__ uint32_t last;
    const uint32_t e = blockIdx.y, tok = blockIdx.z;
    const wh_expert_ptrs ep = a.ex[e];
    const uint32_t t = threadIdx.x & 3, quad = threadIdx.x >> 2;
    const uint32_t row = blockIdx.x * 16 + (quad >> 1);
    const bool up = quad & 1;
    const size_t rb = (size_t)row * (a.hidden / 2), sb = (size_t)row * (a.hidden / 32);
    const uint8_t* wrow = (up ? ep.w3 : ep.w1) + rb;
    const uint8_t* srow = (up ? ep.s3 : ep.s1) + sb;
    const uint8_t* codes = a.xq_codes + (size_t)tok * a.hidden;
    const float* cscales = a.xq_scales + (size_t)tok * (a.hidden / 64);
    float acc_a, acc_b;
    if constexpr (kChunks > 0) {
        wh_stage_codes st;
        wh_stage_codes_load(st, codes, cscales, a.hidden, threadIdx.x);
        wh_fp4_rowbuf<kChunks> b;
        wh_fp4_rowbuf_load<kChunks>(b, wrow, srow, t);
        __builtin_amdgcn_sched_barrier(0);
        wh_stage_codes_store(st, xs);
        __syncthreads();
        wh_fp4_rowbuf_dot<kChunks>(b, xs, t, acc_a, acc_b);
    } else {
        wh_stage_codes_all(xs, codes, cscales, a.hidden);
        __syncthreads();
        wh_fp4_quad_dot_rt(wrow, srow, a.hidden >> 7, t, xs, acc_a, acc_b);
    }
    float v = wh_quad_hsum(acc_a, acc_b) + 0.0f;
    float u = wh_dpp_row_shl4(v);  // lane 8r <- lane 8r + 4 (the w3 quad)
    const size_t hbase = ((size_t)tok * a.n_experts + e) * a.inter;
    if ((threadIdx.x & 7) == 0) {
        if (!(fabsf(v) <= 3.4028235e38f) || !(fabsf(u) <= 3.4028235e38f)) {
            atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        }
        wh_store_coherent(a.h + hbase + row, wh_swiglu(v, u, kExpTab, kExpfFlip, WH_EXPF_FLIP_COUNT));
    }
    wh_stores_done();
    __syncthreads();
    const uint32_t blk = row >> 6;
    uint32_t* cnt = a.cnt_h + ((size_t)tok * a.n_experts + e) * (a.inter / 64) + blk;
    if (threadIdx.x == 0) last = wh_arrive(cnt) == 3u;
    __syncthreads();
    if (!last || threadIdx.x >= 64) return;
    float hv = wh_load_coherent(a.h + hbase + blk * 64 + threadIdx.x);
    float amax = wh_wave_max(fabsf(hv));
    if (!(amax <= 3.4028235e38f)) amax = 1.0f;  // non-finite rows already reported
    int k = wh_aq_scale_exp(amax, kLog2Thr);
    float q;
    uint32_t code = wh_e4m3_nearest(wh_clamp448(hv * wh_pow2f(-k)), &q);
    a.hq_codes[hbase + blk * 64 + threadIdx.x] = (uint8_t)code;
    if (threadIdx.x == 0) {
        a.hq_scales[hbase / 64 + blk] = wh_pow2f(k);
        *cnt = 0u;  // ready for the next launch
    }
}

// Down projection + ordered routed sum.  Grid: (hidden/32, n_experts,
// n_tokens); 128 threads = 32 quads = 32 rows.  The last expert to finish a
// 32-row block combines all experts in route order (E/compute.rs:1948-2012).
template <int kChunks>
__global__ void __launch_bounds__(128) k_moe_down(wh_moe_args a) {
    extern __shared__ __align__(16) float xs[];
    __shared__ uint32_t last;
    const uint32_t e = blockIdx.y, tok = blockIdx.z;
    const wh_expert_ptrs ep = a.ex[e];
    const size_t hbase = ((size_t)tok * a.n_experts + e) * a.inter;
    const uint32_t t = threadIdx.x & 3;
    const uint32_t row = blockIdx.x * 32 + (threadIdx.x >> 2);
    const uint8_t* wrow = ep.w2 + (size_t)row * (a.inter / 2);
    const uint8_t* srow = ep.s2 + (size_t)row * (a.inter / 32);
    float acc_a, acc_b;
    if constexpr (kChunks > 0) {
        wh_stage_codes st;
        wh_stage_codes_load(st, a.hq_codes + hbase, a.hq_scales + hbase / 64, a.inter, threadIdx.x);
        wh_fp4_rowbuf<kChunks> b;
        wh_fp4_rowbuf_load<kChunks>(b, wrow, srow, t);
        __builtin_amdgcn_sched_barrier(0);
        wh_stage_codes_store(st, xs);
        __syncthreads();
        wh_fp4_rowbuf_dot<kChunks>(b, xs, t, acc_a, acc_b);
    } else {
        wh_stage_codes_all(xs, a.hq_codes + hbase, a.hq_scales + hbase / 64, a.inter);
        __syncthreads();
        wh_fp4_quad_dot_rt(wrow, srow, a.inter >> 7, t, xs, acc_a, acc_b);
    }
    float yv = wh_quad_hsum(acc_a, acc_b) + 0.0f;
    const size_t ybase = ((size_t)tok * a.n_experts + e) * a.hidden;
    if (t == 0) {
        if (!(fabsf(yv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        wh_store_coherent(a.y + ybase + row, yv);
    }
    wh_stores_done();
    __syncthreads();
    uint32_t* cnt = a.cnt_y + (size_t)tok * (a.hidden / 32) + blockIdx.x;
    if (threadIdx.x == 0) last = wh_arrive(cnt) == a.n_experts - 1;
    __syncthreads();
    if (!last || threadIdx.x >= 32) return;
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
    // one thread per (row, chunk, quad thread): 4 groups x 8 values
    const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t chunks = cols >> 7, G = cols >> 5;
    if (id >= (size_t)rows * chunks * 4) return;
    const uint32_t t = id & 3, j = (id >> 2) % chunks;
    const size_t row = (id >> 2) / chunks;
    uint4 wv = ((const uint4*)(w + row * (cols / 2)))[4 * j + t];
    uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t g = 4 * j + i;
        wh_fp4x8 v = wh_fp4_decode8(words[i]);
        float va[4] = {v.a01.x, v.a01.y, v.a23.x, v.a23.y};
        float vb[4] = {v.b01.x, v.b01.y, v.b23.x, v.b23.y};
        float sc = wh_ue8m0(s[row * G + (g & 3) * (G / 4) + (g >> 2)]);
        for (uint32_t k = 0; k < 4; ++k) {
            float a8 = va[k] * 0.125f, b8 = vb[k] * 0.125f;
            out[row * cols + g * 32 + t + 8 * k] = a8 == 0.0f ? 0.0f : a8 * sc;
            out[row * cols + g * 32 + t + 4 + 8 * k] = b8 == 0.0f ? 0.0f : b8 * sc;
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

// Plain streaming copy (fn 3 of the debug entry): the known-size kernel that
// calibrates the HBM byte counters against the hot kernels' algorithmic bytes.
__global__ void __launch_bounds__(256) k_copy_f32x4(const float4* __restrict__ in, float4* __restrict__ out, uint32_t n4) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) out[i] = in[i];
}
