// Decode-path kernels for gfx950: FP8 block-scaled GEMV, FP4 E2M1 matvec,
// activation quant-dequant, and the fused routed-expert SwiGLU pipeline.
// Launch helpers and the C ABI live in wohper_hip.hip.
#pragma once
#include "wh_device.h"

#ifndef WH_LIBM_TABLES_INCLUDED
#error "include the generated libm tables before kernels.h"
#endif

// glibc-exact libm tables (generated at build time, see gen_libm_tables.c)
__device__ const uint64_t kExpTab[WH_EXP_TAB_LEN] = {WH_EXP_TAB_INIT};
__device__ const uint32_t kLog2Thr[254] = {WH_LOG2F_THR_INIT};
__device__ const uint32_t kExpfExc[WH_EXPF_EXC_COUNT ? 2 * WH_EXPF_EXC_COUNT : 2] = {WH_EXPF_EXC_INIT};

// status word bits, OR-ed by kernels, read by the host after the stream syncs
#define WH_ST_NONFINITE_OUTPUT 1u
#define WH_ST_NONFINITE_INPUT 2u
#define WH_ST_NOT_RESIDENT 4u

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
// kernels below): AVX lane l's four columns 32g + l + 8k (k = 0..3) of group
// g are one float4, at float4 index g*8 + l plus one float4 of padding per
// two groups, which spreads the staging stores of neighbouring threads over
// all LDS banks (the matvec reads use compile-time offsets either way).
__host__ __device__ constexpr uint32_t wh_xs_f4(uint32_t g, uint32_t l) { return g * 8 + l + (g >> 1); }
// Floats of the staged x for `cols` columns.
__host__ __device__ constexpr uint32_t wh_xs_floats(uint32_t cols) { return cols + (cols >> 4); }

// Cross-workgroup hand-off inside one launch.  The 8 XCDs of an MI355X have
// separate L2s, so an agent-scope fence writes back and invalidates the whole
// L2 - far too costly per workgroup.  Instead the few values that cross
// workgroups are written and read with agent-scope relaxed atomics (coherent
// at the device level), each writer waits for its stores to complete, and an
// agent-scope atomic counter elects the last arriver.
// acc + src[0] + src[1] + ... + src[len - 1], one add at a time in index
// order (the reference's sequential f32 sums), from LDS.  Blocks of 256
// values are straight-line code in which batches of 32 alternate between
// two register sets, so the next batch's reads are in flight while the
// current one is added (in straight-line code the compiler counts the reads
// in flight exactly; across a loop's back edge it waits for all of them).
// src 16-byte aligned.
__device__ __forceinline__ float wh_ordered_sum_lds(const float* src, uint32_t len, float acc) {
    float4 p[2][8];
    auto rd = [&](float4 (&q)[8], const float* a) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = *(const float4*)(a + 4 * i);
    };
    auto add = [&](const float4 (&q)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc = acc + q[i].x;
            acc = acc + q[i].y;
            acc = acc + q[i].z;
            acc = acc + q[i].w;
        }
    };
    uint32_t e = 0;
    for (; e + 256 <= len; e += 256) {
        const float* b = src + e;
        rd(p[0], b);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (k + 1 < 8) rd(p[(k + 1) & 1], b + 32 * (k + 1));
            __builtin_amdgcn_sched_barrier(0);
            add(p[k & 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (; e + 32 <= len; e += 32) {
        rd(p[0], src + e);
        add(p[0]);
    }
    for (; e < len; ++e) acc = acc + src[e];
    return acc;
}

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
        ((float4*)xs)[wh_xs_f4(g, l)] = make_float4(v32[l], v32[8 + l], v32[16 + l], v32[24 + l]);
}
__device__ __forceinline__ void wh_stage_f32_fp4_store(const wh_stage_f32_fp4& st, float* xs) {
    if (!st.on) return;
    float v[32];
#pragma unroll
    for (int m = 0; m < 32; ++m) v[m] = wh_f4_get(st.v[m >> 2], m & 3);
    wh_stage_fp4_store_group(xs, st.g, v);
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
            q = wh_e4m3_round(wh_clamp448(t));
        }
        v[i] = q * scale;
    }
}

// ------------------------------------------------------------- FP8 GEMV
struct wh_fp8_args {
    const uint8_t* w;       // resident (lane-permuted) bytes, rows x cols
    const void* scales;     // [scale_rows][scale_cols], f32 or UE8M0 bytes
    const float* x;         // cols
    float* y;               // row_end - row_start
    uint32_t* status;
    uint32_t cols, scale_cols, row_group, row_start, row_end;
    uint32_t row_group_shift;     // log2(row_group) when it is a power of two (split-K path), else 32
    uint32_t x_stride, y_stride;  // batch strides (multi-input variant)
    // row groups with their own input (wo_a, E/compute.rs:4244-4258): rows
    // row_start + [g*x_group_rows, (g+1)*x_group_rows) read x + g*x_group_stride;
    // 0 = one input for all rows (split-K path only: a power of two, at least
    // WH_FP8_SK_ROWS); x_group_shift = log2(x_group_rows), 32 for one input
    uint32_t x_group_rows, x_group_stride, x_group_shift;
    // a second tensor on the same input in the same launch (split-K path,
    // one input, no row groups): workgroups from blocks1 on run its rows
    // [row_start2, row_end2) into y2; blocks1 = UINT32_MAX for one tensor
    const uint8_t* w2;
    const void* scales2;
    float* y2;
    uint32_t scale_cols2, row_group_shift2, row_start2, row_end2, blocks1;
};

template <bool kSpecial, bool kScaleU8>
__device__ __forceinline__ float wh_fp8_scale(const void* s, uint32_t idx) {
    if constexpr (kScaleU8) return wh_ue8m0(((const uint8_t*)s)[idx]);
    else return ((const float*)s)[idx];
}

// One 128-col group of one AVX lane: two 8-FMA chains (g0 over cols
// 16c + l, g1 over 16c + 8 + l), then acc = fma(g0 + g1, scale, acc).
// g0 + g1 of one 128-col group of one AVX lane: two 8-FMA chains, g0 over
// cols 16c + l and g1 over cols 16c + 8 + l (E/compute.rs:5990-6005).
template <bool kSpecial>
__device__ __forceinline__ float wh_fp8_lane_gsum(uint4 wv, const float4* xg) {
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
    return g0 + g1;
}
template <bool kSpecial>
__device__ __forceinline__ float wh_fp8_lane_group(uint4 wv, const float4* xg, float s, float acc) {
    return __builtin_fmaf(wh_fp8_lane_gsum<kSpecial>(wv, xg), s, acc);
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

// Split-K path (col_group == 128, groups % 8 == 0): 256 threads = 4 waves x
// 8 column segments x 8 AVX lanes; wave w runs rows 2w and 2w + 1 of the
// workgroup's WH_FP8_SK_ROWS, so every x value read from LDS serves two rows.
// Each thread forms g0 + g1 for its segment's groups of both rows into LDS,
// then wave 0 runs the reference's sequential acc = fma(g0 + g1, scale, acc)
// over all groups for the 8 rows x 8 lanes - the same operations in the same
// order as the one-thread row.  kGps = groups per segment when the segment's
// weights fit in registers (4 for 4096 columns), else 0.
#define WH_FP8_SK_ROWS 8u
template <bool kSpecial, bool kScaleU8, int kGps>
__global__ void __launch_bounds__(256) k_fp8_gemv_sk(wh_fp8_args a) {
    constexpr uint32_t kR = WH_FP8_SK_ROWS / 4;  // rows per wave
    extern __shared__ __align__(16) float lds[];
    const uint32_t batch = blockIdx.y;
    // the workgroup's tensor: the first, or the second from blocks1 on
    const bool second = blockIdx.x >= a.blocks1;
    const uint8_t* const aw = second ? a.w2 : a.w;
    const void* const ascales = second ? a.scales2 : a.scales;
    float* const ay = second ? a.y2 : a.y;
    const uint32_t ascale_cols = second ? a.scale_cols2 : a.scale_cols;
    const uint32_t arow_group_shift = second ? a.row_group_shift2 : a.row_group_shift;
    const uint32_t arow_start = second ? a.row_start2 : a.row_start, arow_end = second ? a.row_end2 : a.row_end;
    const uint32_t rb = (second ? blockIdx.x - a.blocks1 : blockIdx.x) * WH_FP8_SK_ROWS;  // relative to row start
    const float* x = a.x + (size_t)batch * a.x_stride +
                     (a.x_group_shift < 32 ? (size_t)(rb >> a.x_group_shift) * a.x_group_stride : 0);
    const uint32_t lane = threadIdx.x & 7, seg = (threadIdx.x >> 3) & 7;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // rows and scale rows stay scalar
    // widths known at compile time for kGps > 0 (cols = 1024 kGps)
    const uint32_t cols = kGps > 0 ? 1024u * kGps : a.cols;
    const uint32_t G = cols >> 7, gps = G >> 3, gbeg = seg * gps;
    float* xs = lds;
    float* gsum = lds + cols;     // [8 rows][8 lanes][G]: g0 + g1 of every group
    float* scl = gsum + 64 * G;   // [8 rows][G]: the group scales
    const float4* xp = (const float4*)xs + lane * 4;  // group g at xp[32 g]
    const uint4* wp[kR];
    uint32_t sbase[kR];
#pragma unroll
    for (uint32_t j = 0; j < kR; ++j) {
        const uint32_t r = arow_start + rb + wv * kR + j;
        const uint32_t rc = r < arow_end ? r : arow_start;  // rows past the end load row_start
        wp[j] = (const uint4*)(aw + (size_t)rc * cols) + lane;  // group g at wp[8 g]
        sbase[j] = (rc >> arow_group_shift) * ascale_cols;
    }
    // staging loads (x chunk, this lane's share of the rows' scales) go out
    // before the weight loads, so waiting for them never waits for weights
    wh_stage_f32_fp8 st;
    wh_stage_f32_fp8_load(st, x, cols, threadIdx.x);
    const uint32_t sg = seg * 8 + lane;  // scales g = sg, sg + 64, ...
    float sv[kR];
#pragma unroll
    for (uint32_t j = 0; j < kR; ++j) sv[j] = sg < G ? wh_fp8_scale<kSpecial, kScaleU8>(ascales, sbase[j] + sg) : 0.0f;
    auto stage_rest = [&]() {
        wh_stage_f32_fp8_store(st, xs);
        for (uint32_t q = threadIdx.x + 256; q < cols / 16; q += 256) {  // cols > 4096
            wh_stage_f32_fp8 s2;
            wh_stage_f32_fp8_load(s2, x, cols, q);
            wh_stage_f32_fp8_store(s2, xs);
        }
#pragma unroll
        for (uint32_t j = 0; j < kR; ++j) {
            float* srow = scl + (wv * kR + j) * G;
            if (sg < G) srow[sg] = sv[j];
            for (uint32_t g = sg + 64; g < G; g += 64) srow[g] = wh_fp8_scale<kSpecial, kScaleU8>(ascales, sbase[j] + g);
        }
    };
    if constexpr (kGps > 0) {
        uint4 w[kR][kGps];
#pragma unroll
        for (uint32_t j = 0; j < kR; ++j)
#pragma unroll
            for (int i = 0; i < kGps; ++i) w[j][i] = wp[j][8 * (gbeg + i)];
        __builtin_amdgcn_sched_barrier(0);
        stage_rest();
        __syncthreads();
        // a thread's kGps sums of one row are adjacent in LDS: computed in
        // registers, then stored as vectors
        float gs[kR][kGps];
#pragma unroll
        for (int i = 0; i < kGps; ++i)
#pragma unroll
            for (uint32_t j = 0; j < kR; ++j) gs[j][i] = wh_fp8_lane_gsum<kSpecial>(w[j][i], xp + 32 * (gbeg + i));
#pragma unroll
        for (uint32_t j = 0; j < kR; ++j) {
            float* dst = gsum + ((wv * kR + j) * 8 + lane) * G + gbeg;
            if constexpr (kGps % 4 == 0) {
#pragma unroll
                for (int i = 0; i < kGps; i += 4) *(float4*)(dst + i) = make_float4(gs[j][i], gs[j][i + 1], gs[j][i + 2], gs[j][i + 3]);
            } else {
#pragma unroll
                for (int i = 0; i < kGps; ++i) dst[i] = gs[j][i];
            }
        }
    } else {
        stage_rest();
        __syncthreads();
        for (uint32_t g = gbeg; g < gbeg + gps; ++g)
#pragma unroll
            for (uint32_t j = 0; j < kR; ++j)
                gsum[((wv * kR + j) * 8 + lane) * G + g] = wh_fp8_lane_gsum<kSpecial>(wp[j][8 * g], xp + 32 * g);
    }
    __syncthreads();
    if (threadIdx.x >= 64) return;  // wave 0: row rl = thread / 8, AVX lane thread % 8
    const uint32_t rl = threadIdx.x >> 3, ln = threadIdx.x & 7;
    const float* gs = gsum + (rl * 8 + ln) * G;
    const float* sc = scl + rl * G;
    float acc = 0.0f;
    if constexpr (kGps > 0) {  // G = 8 kGps known
#pragma unroll
        for (int i = 0; i < 2 * kGps; ++i) {
            const float4 g = ((const float4*)gs)[i], s = ((const float4*)sc)[i];
            acc = __builtin_fmaf(g.x, s.x, acc);
            acc = __builtin_fmaf(g.y, s.y, acc);
            acc = __builtin_fmaf(g.z, s.z, acc);
            acc = __builtin_fmaf(g.w, s.w, acc);
        }
    } else {
        for (uint32_t g = 0; g < G; ++g) acc = __builtin_fmaf(gs[g], sc[g], acc);
    }
    const float sum = wh_hsum8(acc) + 0.0f;  // + tail (0 for col_group % 16 == 0)
    const uint32_t row = arow_start + rb + rl;
    if (row < arow_end && ln == 0) {
        ay[(size_t)batch * a.y_stride + (row - arow_start)] = sum;
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
// Resident FP4 layout (fast path: group_cols == 32, cols % 256 == 0).  A row
// is run by 8 threads, one per AVX lane of E/deepseek_v4.rs:294-347: lane l
// owns columns l, 8+l, 16+l, 24+l of every 32-col group.
//   weights: per block of 8 groups (256 columns = 128 bytes of the row),
//            lane l's 16 bytes sit at block*128 + l*16; dword d holds the
//            lane's 4 values of group 8b+2d (A) and of group 8b+2d+1 (B),
//            packed by wh_fp4_encode_word;
//   scales:  unchanged, [row][cols/32] UE8M0 bytes.
// A workgroup stages x in LDS in lane order (wh_fp4_lds_index) next to a
// table of its rows' group scales, each already multiplied by 1/8 as the
// reference does (`scale * 0.125`, E/deepseek_v4.rs:329).
__host__ __device__ inline uint32_t wh_fp4_encode_word(const uint32_t* a, const uint32_t* b) {
    uint32_t word = 0;
    for (uint32_t k = 0; k < 4; ++k) {
        uint32_t ap = a[(k + 3) & 3];
        uint32_t byte = (a[k] & 7) | ((ap >> 3) << 3) | ((b[k] & 7) << 4) | ((b[k] >> 3) << 7);
        word |= byte << (8 * k);
    }
    return word;
}

// Row stride (floats) of the LDS scale table; the 4 extra floats put
// consecutive rows on different banks.
__host__ __device__ constexpr uint32_t wh_s8_stride(uint32_t groups) { return groups + 4; }

// LDS bytes of a 32-row FP4 workgroup: staged x + the scale table.
__host__ __device__ constexpr size_t wh_fp4_wg_lds(size_t cols) {
    return sizeof(float) * (wh_xs_floats((uint32_t)cols) + 32 * (size_t)wh_s8_stride((uint32_t)(cols / 32)));
}

// One dword of one lane = two groups: a 4-FMA chain from zero per group over
// the x8 integer values, folded in with acc = fma(gacc, scale/8, acc).
__device__ __forceinline__ float wh_fp4_lane_pair(uint32_t word, const float4& xa, const float4& xb, float sa,
                                                  float sb, float acc) {
    wh_fp4x8 e = wh_fp4_decode8(word);
    float ga = __builtin_fmaf(e.a01.x, xa.x, 0.0f);
    ga = __builtin_fmaf(e.a01.y, xa.y, ga);
    ga = __builtin_fmaf(e.a23.x, xa.z, ga);
    ga = __builtin_fmaf(e.a23.y, xa.w, ga);
    acc = __builtin_fmaf(ga, sa, acc);
    float gb = __builtin_fmaf(e.b01.x, xb.x, 0.0f);
    gb = __builtin_fmaf(e.b01.y, xb.y, gb);
    gb = __builtin_fmaf(e.b23.x, xb.z, gb);
    gb = __builtin_fmaf(e.b23.y, xb.w, gb);
    return __builtin_fmaf(gb, sb, acc);
}

// One block (8 groups) of one lane.  xp = (float4*)xs + lane; s8row = the
// row's scale table.
__device__ __forceinline__ float wh_fp4_lane_block(uint4 w, const float4* xp, const float* s8row, uint32_t b,
                                                   float acc) {
    const float4 s0 = ((const float4*)s8row)[2 * b], s1 = ((const float4*)s8row)[2 * b + 1];
    const float4* xg = xp + 68 * b;  // group 8b + j -> xg[wh_xs_f4(j, 0)]
    acc = wh_fp4_lane_pair(w.x, xg[wh_xs_f4(0, 0)], xg[wh_xs_f4(1, 0)], s0.x, s0.y, acc);
    acc = wh_fp4_lane_pair(w.y, xg[wh_xs_f4(2, 0)], xg[wh_xs_f4(3, 0)], s0.z, s0.w, acc);
    acc = wh_fp4_lane_pair(w.z, xg[wh_xs_f4(4, 0)], xg[wh_xs_f4(5, 0)], s1.x, s1.y, acc);
    acc = wh_fp4_lane_pair(w.w, xg[wh_xs_f4(6, 0)], xg[wh_xs_f4(7, 0)], s1.z, s1.w, acc);
    return acc;
}

// A lane's whole row in registers (kBlk = cols / 256 known at compile time),
// loaded before anything waits so the row's bytes are all in flight at once.
template <int kBlk>
struct wh_fp4_lane_row {
    uint4 w[kBlk];
};
template <int kBlk>
__device__ __forceinline__ void wh_fp4_lane_row_load(wh_fp4_lane_row<kBlk>& r, const uint8_t* __restrict__ wrow,
                                                     uint32_t lane) {
    const uint4* p = (const uint4*)wrow + lane;
#pragma unroll
    for (int b = 0; b < kBlk; ++b) r.w[b] = p[8 * b];
}
// LDS operands of one block of one lane: x of its 8 groups and their scales.
struct wh_fp4_blk_lds {
    float4 x[8];
    float4 s0, s1;
};
// `dep` is an opaque zero tied to the running sum: block reads indexed with
// it cannot be hoisted above the blocks before them, which would keep every
// block's operands live at once.
__device__ __forceinline__ void wh_fp4_blk_lds_read(wh_fp4_blk_lds& o, const float4* xp, const float* s8row,
                                                    uint32_t b, uint32_t dep) {
    const float4* xg = xp + 68 * b + dep;  // group 8b + j -> xg[wh_xs_f4(j, 0)]
#pragma unroll
    for (int j = 0; j < 8; ++j) o.x[j] = xg[wh_xs_f4(j, 0)];
    const float4* sp = (const float4*)s8row + 2 * b + dep;
    o.s0 = sp[0];
    o.s1 = sp[1];
}
__device__ __forceinline__ uint32_t wh_opaque_zero(float after) {
    uint32_t z = 0;
    asm volatile("" : "+v"(z) : "v"(after));
    return z;
}
__device__ __forceinline__ float wh_fp4_blk_compute(uint4 w, const wh_fp4_blk_lds& o, float acc) {
    acc = wh_fp4_lane_pair(w.x, o.x[0], o.x[1], o.s0.x, o.s0.y, acc);
    acc = wh_fp4_lane_pair(w.y, o.x[2], o.x[3], o.s0.z, o.s0.w, acc);
    acc = wh_fp4_lane_pair(w.z, o.x[4], o.x[5], o.s1.x, o.s1.y, acc);
    acc = wh_fp4_lane_pair(w.w, o.x[6], o.x[7], o.s1.z, o.s1.w, acc);
    return acc;
}

// The LDS reads of block b + 1 are issued before block b computes, so their
// latency hides behind that block's arithmetic (kBlk even; two named
// buffers, alternated by hand, stay in registers).
template <int kBlk>
__device__ __forceinline__ float wh_fp4_lane_row_dot(const wh_fp4_lane_row<kBlk>& r, const float* xs,
                                                     const float* s8row, uint32_t lane) {
    static_assert(kBlk % 2 == 0, "blocks are processed in pairs");
    const float4* xp = (const float4*)xs + lane;
    wh_fp4_blk_lds ba, bb;
    float acc = 0.0f;
    wh_fp4_blk_lds_read(ba, xp, s8row, 0, 0);
#pragma unroll
    for (int b = 0; b < kBlk; b += 2) {
        wh_fp4_blk_lds_read(bb, xp, s8row, b + 1, wh_opaque_zero(acc));
        __builtin_amdgcn_sched_barrier(0);
        acc = wh_fp4_blk_compute(r.w[b], ba, acc);
        if (b + 2 < kBlk) wh_fp4_blk_lds_read(ba, xp, s8row, b + 2, wh_opaque_zero(acc));
        __builtin_amdgcn_sched_barrier(0);
        acc = wh_fp4_blk_compute(r.w[b + 1], bb, acc);
    }
    return acc;
}
// A lane's row streamed through a ring of kDepth blocks: the prologue issues
// blocks 0..kDepth-1, the dot issues block b + kDepth once block b is
// consumed.  Issuing a whole row at once stalls the wave behind the memory
// system's back-pressure (loads issue in order, and nothing after them runs
// until they have issued); kDepth blocks per wave are enough in flight to
// keep HBM busy.
template <int kDepth>
struct wh_fp4_ring {
    uint4 w[kDepth];
};
template <int kDepth>
__device__ __forceinline__ void wh_fp4_ring_prologue(wh_fp4_ring<kDepth>& r, const uint8_t* __restrict__ wrow,
                                                     uint32_t lane) {
    const uint4* p = (const uint4*)wrow + lane;
#pragma unroll
    for (int b = 0; b < kDepth; ++b) r.w[b] = p[8 * b];
}
template <int kBlk, int kDepth>
__device__ __forceinline__ float wh_fp4_ring_dot(wh_fp4_ring<kDepth>& r, const uint8_t* __restrict__ wrow,
                                                 const float* xs, const float* s8row, uint32_t lane) {
    static_assert(kBlk % 2 == 0 && kDepth % 2 == 0 && kDepth <= kBlk, "blocks are processed in pairs");
    const uint4* p = (const uint4*)wrow + lane;
    const float4* xp = (const float4*)xs + lane;
    wh_fp4_blk_lds ba, bb;
    float acc = 0.0f;
    wh_fp4_blk_lds_read(ba, xp, s8row, 0, 0);
#pragma unroll
    for (int b = 0; b < kBlk; b += 2) {
        wh_fp4_blk_lds_read(bb, xp, s8row, b + 1, wh_opaque_zero(acc));
        __builtin_amdgcn_sched_barrier(0);
        acc = wh_fp4_blk_compute(r.w[b % kDepth], ba, acc);
        if (b + kDepth < kBlk) r.w[b % kDepth] = p[8 * (b + kDepth)];
        if (b + 2 < kBlk) wh_fp4_blk_lds_read(ba, xp, s8row, b + 2, wh_opaque_zero(acc));
        __builtin_amdgcn_sched_barrier(0);
        acc = wh_fp4_blk_compute(r.w[(b + 1) % kDepth], bb, acc);
        if (b + 1 + kDepth < kBlk) r.w[(b + 1) % kDepth] = p[8 * (b + 1 + kDepth)];
    }
    return acc;
}

// Runtime block count: weights streamed one block ahead.
__device__ __forceinline__ float wh_fp4_lane_dot_rt(const uint8_t* __restrict__ wrow, uint32_t blocks,
                                                    const float* xs, const float* s8row, uint32_t lane) {
    const uint4* p = (const uint4*)wrow + lane;
    const float4* xp = (const float4*)xs + lane;
    float acc = 0.0f;
    uint4 nxt = p[0];
    for (uint32_t b = 0; b < blocks; ++b) {
        uint4 cur = nxt;
        if (b + 1 < blocks) nxt = p[8 * (b + 1)];
        acc = wh_fp4_lane_block(cur, xp, s8row, b, acc);
    }
    return acc;
}

// A row's UE8M0 bytes staged as scale/8 floats: lane l takes the kBlk bytes
// [l*kBlk, (l+1)*kBlk) of the row (kBlk = groups / 8, a multiple of 4).
template <int kBlk>
struct wh_s8_stage {
    uint32_t v[kBlk / 4];
};
template <int kBlk>
__device__ __forceinline__ void wh_s8_stage_load(wh_s8_stage<kBlk>& st, const uint8_t* srow, uint32_t lane) {
    const uint32_t* p = (const uint32_t*)(srow + lane * kBlk);
#pragma unroll
    for (int i = 0; i < kBlk / 4; ++i) st.v[i] = p[i];
}
template <int kBlk>
__device__ __forceinline__ void wh_s8_stage_store(const wh_s8_stage<kBlk>& st, float* s8row, uint32_t lane) {
    float4* d = (float4*)(s8row + lane * kBlk);
#pragma unroll
    for (int i = 0; i < kBlk / 4; ++i) {
        const uint32_t v = st.v[i];
        d[i] = make_float4(wh_ue8m0(v) * 0.125f, wh_ue8m0(v >> 8) * 0.125f, wh_ue8m0(v >> 16) * 0.125f,
                           wh_ue8m0(v >> 24) * 0.125f);
    }
}
__device__ __forceinline__ void wh_s8_stage_rt(const uint8_t* srow, uint32_t groups, float* s8row, uint32_t lane) {
    for (uint32_t g = lane; g < groups; g += 8) s8row[g] = wh_ue8m0(srow[g]) * 0.125f;
}

struct wh_fp4_args {
    const uint8_t* w;  // resident
    const uint8_t* s;  // scales
    const float* x;
    float* y;
    uint32_t* status;
    uint32_t rows, cols;
};

// Fast path: 256 threads = 32 rows (8 lanes each).  kBlk = cols/256 when
// it is 8 or 16 (row fully in registers), else 0 (runtime loop).
template <int kBlk>
__global__ void __launch_bounds__(256) k_fp4_matvec(wh_fp4_args a) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t G = a.cols >> 5;
    const uint32_t lane = threadIdx.x & 7, oct = threadIdx.x >> 3;
    const uint32_t row = blockIdx.x * 32 + oct;
    const bool active = row < a.rows;
    const uint32_t rr = active ? row : 0;
    const uint8_t* wrow = a.w + (size_t)rr * (a.cols / 2);
    const uint8_t* srow = a.s + (size_t)rr * G;
    float* xs = lds;
    float* s8row = lds + wh_xs_floats(a.cols) + oct * wh_s8_stride(G);
    float acc;
    if constexpr (kBlk > 0) {
        wh_stage_f32_fp4 st;
        wh_stage_f32_fp4_load(st, a.x, a.cols, threadIdx.x);
        wh_s8_stage<kBlk> ss;
        wh_s8_stage_load<kBlk>(ss, srow, lane);
        wh_fp4_lane_row<kBlk> r;
        wh_fp4_lane_row_load<kBlk>(r, wrow, lane);
        __builtin_amdgcn_sched_barrier(0);
        wh_stage_f32_fp4_store(st, xs);
        wh_s8_stage_store<kBlk>(ss, s8row, lane);
        __syncthreads();
        acc = wh_fp4_lane_row_dot<kBlk>(r, xs, s8row, lane);
    } else {
        for (uint32_t g = threadIdx.x; g < G; g += 256) {
            wh_stage_f32_fp4 st;
            wh_stage_f32_fp4_load(st, a.x, a.cols, g);
            wh_stage_f32_fp4_store(st, xs);
        }
        wh_s8_stage_rt(srow, G, s8row, lane);
        __syncthreads();
        acc = wh_fp4_lane_dot_rt(wrow, G >> 3, xs, s8row, lane);
    }
    float sum = wh_hsum8(acc) + 0.0f;  // + tail (0 here)
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
// Two launches per decode step run the routed-expert FFN of
// E/compute.rs:1948-2012 for every token of the step:
//   k_moe_gateup: gate/up matvecs + SwiGLU (E/deepseek_v4.rs:586-594), with
//                 the act-quant of x recomputed by every workgroup from the
//                 input (a 4096-vector, cheaper than another launch);
//   k_moe_down:   act-quant of the hidden (E/deepseek_v4.rs:595) recomputed
//                 per workgroup while staging it, the down matvec
//                 (E/deepseek_v4.rs:596-599) and the ordered weighted sum.
// The launch boundary is the only hand-off between the two; the routed sum
// is the one value that crosses workgroups inside a launch.
struct wh_expert_ptrs {
    const uint8_t* w1;
    const uint8_t* s1;
    const uint8_t* w3;
    const uint8_t* s3;
    const uint8_t* w2;
    const uint8_t* s2;
};

// A token's route list in device memory (the router's output resolved
// against the layer's expert table by k_moe_resolve): slots [0, n_routed)
// are the routes in route order; the slots after them up to the shared slot
// hold copies of a resident expert, computed and never summed.
struct wh_moe_dyn {
    wh_expert_ptrs ex[WH_MAX_EXPERTS];
    float route_w[WH_MAX_EXPERTS];
    uint32_t n_routed;
};

struct wh_moe_args {
    wh_expert_ptrs ex[WH_MAX_EXPERTS];
    float route_w[WH_MAX_EXPERTS];
    uint32_t n_experts;            // expert slots: routed ones, plus the shared one (the last) when has_shared
    uint32_t has_shared;           // the last expert slot is the shared expert
    const wh_moe_dyn* dyn;         // null: ex / route_w above; else the slots' experts and weights live there
    uint32_t hidden, inter;        // w1/w3: inter x hidden, w2: hidden x inter
    uint32_t n_tokens;             // tokens sharing the same expert list
    const void* x;                 // [n_tokens][hidden], f32 or bf16
    uint32_t x_is_bf16;
    float* h;                      // [n_tokens][n_experts][inter] SwiGLU output
    float* y;                      // [n_tokens][n_experts][hidden] per-expert outputs
    float* out;                    // [n_tokens][hidden] routed sum
    uint32_t* cnt_y;               // [n_tokens][hidden/16] arrivals per 16- or 32-row slice
    uint32_t* status;
    float* gu;                     // null, or [n_tokens][n_experts][2][inter]: gate and up captured
};

// Slot e's expert, route weight i and the number of routed slots summed, from
// the kernel arguments or the device route list.  The device list is read
// through the constant address space: with a wave-uniform index these are
// scalar loads, which leave the vector-memory counters of the kernels that
// count their own loads untouched.
typedef __attribute__((address_space(4))) const wh_moe_dyn wh_moe_dyn_k;
__device__ __forceinline__ wh_expert_ptrs wh_moe_ex(const wh_moe_args& a, uint32_t e) {
    if (a.dyn) {
        wh_moe_dyn_k* d = (wh_moe_dyn_k*)a.dyn;
        wh_expert_ptrs r;
        r.w1 = d->ex[e].w1;
        r.s1 = d->ex[e].s1;
        r.w3 = d->ex[e].w3;
        r.s3 = d->ex[e].s3;
        r.w2 = d->ex[e].w2;
        r.s2 = d->ex[e].s2;
        return r;
    }
    return a.ex[e];
}
__device__ __forceinline__ float wh_moe_w(const wh_moe_args& a, uint32_t i) {
    if (a.dyn) return ((wh_moe_dyn_k*)a.dyn)->route_w[i];
    return a.route_w[i];
}
__device__ __forceinline__ uint32_t wh_moe_nr(const wh_moe_args& a) {
    if (a.dyn) return ((wh_moe_dyn_k*)a.dyn)->n_routed;
    return a.n_experts - a.has_shared;
}

// Resolves a token's route list in device memory (ids, route weights and
// count as the router writes them) against a layer's expert table
// (table_n entries, null where nothing is resident) into *out: slots
// [0, n_routed) are the routes in order, n_routed = min(count, n_slots);
// the later routed slots, and ids with no resident expert (reported as
// NotResident), get a resident expert's pointers - the first resolved
// route, else the shared expert, else the table's first resident entry -
// computed and never summed; the shared expert goes to slot n_slots.  One
// wave; the host checks that some expert is resident.
// The resolve of one wave (k_moe_resolve, or the router's last arriver):
// lane L < cnt holds route L's expert id and weight; slots [0, cnt) get
// their experts, the slots after them up to n_slots a resident stand-in
// (computed, never summed), slot n_slots the shared expert when there is
// one.  got: 64 entries of workgroup memory.
__device__ __forceinline__ void wh_moe_resolve_wave(uint32_t id, float wt, uint32_t cnt,
                                                    const wh_expert_ptrs* __restrict__ table, uint32_t table_n,
                                                    const wh_expert_ptrs& shared, uint32_t has_shared,
                                                    uint32_t n_slots, wh_moe_dyn* __restrict__ out, uint32_t* status,
                                                    wh_expert_ptrs* got) {
    const uint32_t L = threadIdx.x & 63;
    bool ok = false;
    wh_expert_ptrs p = {};
    if (L < cnt) {
        if (id < table_n) {
            p = table[id];
            ok = p.w1 != nullptr;
        }
        if (!ok) atomicOr(status, WH_ST_NOT_RESIDENT);
    }
    got[L] = p;
    const uint64_t okm = __ballot(ok);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    wh_expert_ptrs fb = shared;
    if (okm) {
        fb = got[__ffsll((long long)okm) - 1];
    } else if (!has_shared) {
        for (uint32_t base = 0; base < table_n; base += 64) {
            const uint32_t j = base + L;
            const bool r = j < table_n && table[j].w1 != nullptr;
            const uint64_t m = __ballot(r);
            if (m) {
                fb = table[base + __ffsll((long long)m) - 1];
                break;
            }
        }
    }
    // field by field: a select of whole structs goes through scratch memory
    auto put = [&](uint32_t slot, const wh_expert_ptrs& e) {
        out->ex[slot].w1 = e.w1;
        out->ex[slot].s1 = e.s1;
        out->ex[slot].w3 = e.w3;
        out->ex[slot].s3 = e.s3;
        out->ex[slot].w2 = e.w2;
        out->ex[slot].s2 = e.s2;
    };
    if (L < n_slots) {
        if (ok) put(L, p);
        else put(L, fb);
        out->route_w[L] = L < cnt ? wt : 0.0f;
    }
    if (L == n_slots && has_shared) put(L, shared);
    if (L == 0) out->n_routed = cnt;
}

__global__ void __launch_bounds__(64) k_moe_resolve(const uint32_t* __restrict__ ids, const float* __restrict__ w,
                                                    const uint32_t* __restrict__ count,
                                                    const wh_expert_ptrs* __restrict__ table, uint32_t table_n,
                                                    wh_expert_ptrs shared, uint32_t has_shared, uint32_t n_slots,
                                                    wh_moe_dyn* __restrict__ out, uint32_t* status) {
    __shared__ wh_expert_ptrs got[64];
    const uint32_t L = threadIdx.x;
    const uint32_t cnt = min(*count, n_slots);
    const uint32_t id = L < cnt ? ids[L] : 0u;
    const float wt = L < cnt ? w[L] : 0.0f;
    wh_moe_resolve_wave(id, wt, cnt, table, table_n, shared, has_shared, n_slots, out, status, got);
}

// The ordered routed sum of one output row from the per-slot outputs yv
// (E/compute.rs:1929-2030): route-weighted in route order with the weight
// rules of valid_route_weight_sum (E/compute.rs:2014-2030), then shared +
// routed (E/compute.rs:1929-1941); the shared expert is the last slot.
// yv is indexed with compile-time indices only (unrolled, guarded loops), so
// it stays in registers.
__device__ __forceinline__ float wh_route_combine(const wh_moe_args& a, const float (&yv)[WH_MAX_EXPERTS]) {
    const uint32_t nr = wh_moe_nr(a);
    float o = 0.0f;
    if (nr == 1) {
        o = yv[0];
    } else if (nr > 1) {
        float sum = 0.0f;
        bool valid = true;
        for (uint32_t i = 0; i < nr; ++i) {
            const float w = wh_moe_w(a, i);
            if (!(fabsf(w) <= 3.4028235e38f && w >= 0.0f)) valid = false;
            sum = sum + w;
        }
        if (sum <= 1.1920929e-07f) valid = false;
        const float uniform = 1.0f / (float)nr;
#pragma unroll
        for (uint32_t i = 0; i < WH_MAX_EXPERTS; ++i) {
            if (i < nr) {
                const float w = valid ? wh_moe_w(a, i) / sum : uniform;
                const float p = yv[i] * w;
                o = o + p;
            }
        }
    }
    if (a.has_shared) {
        float sh = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < WH_MAX_EXPERTS; ++i)
            if (i + 1 == a.n_experts) sh = yv[i];
        o = nr == 0 ? sh : sh + o;
    }
    return o;
}

// The per-binade log2f thresholds of the act-quant scale, staged in LDS: a
// table lookup in global memory after the weight loads would make the wave
// wait for all of them (memory loads complete in issue order).
struct wh_thr_stage {
    uint32_t v;
};
__device__ __forceinline__ void wh_thr_stage_load(wh_thr_stage& st) {
    st.v = threadIdx.x < 254 ? kLog2Thr[threadIdx.x] : 0u;
}
__device__ __forceinline__ void wh_thr_stage_store(const wh_thr_stage& st, uint32_t* thr) {
    if (threadIdx.x < 254) thr[threadIdx.x] = st.v;
}

// The expf table staged in LDS the same way (needs >= 74 threads), so the
// SwiGLU epilogue reads no global memory behind the weight stream.
struct wh_exp_stage {
    uint32_t v;
};
__device__ __forceinline__ void wh_exp_stage_load(wh_exp_stage& st) {
    st.v = threadIdx.x < 2 * WH_EXP_TAB_LEN ? reinterpret_cast<const uint32_t*>(kExpTab)[threadIdx.x] : 0u;
}
__device__ __forceinline__ void wh_exp_stage_store(const wh_exp_stage& st, uint64_t* tab) {
    if (threadIdx.x < 2 * WH_EXP_TAB_LEN) reinterpret_cast<uint32_t*>(tab)[threadIdx.x] = st.v;
}
// LDS bytes of a routed-expert workgroup over `cols` input columns.
__host__ __device__ constexpr size_t wh_moe_wg_lds(size_t cols) {
    return wh_fp4_wg_lds(cols) + (256 + 2 + 2 * WH_EXP_TAB_LEN) * sizeof(uint32_t);
}
// The staged expf table of a workgroup whose log2f thresholds sit at thr
// (256 words), 8-byte aligned.
__device__ __forceinline__ uint64_t* wh_exp_tab_after(uint32_t* thr) {
    return reinterpret_cast<uint64_t*>((reinterpret_cast<uintptr_t>(thr + 256) + 7) & ~uintptr_t(7));
}

// 16 consecutive x values of one thread (bf16 or f32), loaded early.
struct wh_xq_stage {
    uint4 raw[4];
    uint32_t c0;
    bool on;
};
__device__ __forceinline__ void wh_xq_stage_load(wh_xq_stage& st, const void* x, bool bf16, uint32_t n,
                                                 uint32_t idx) {
    st.c0 = 16 * idx;
    st.on = st.c0 < n;
    if (!st.on) {
        for (int i = 0; i < 4; ++i) st.raw[i] = make_uint4(0, 0, 0, 0);
        return;
    }
    if (bf16) {
        const uint4* p = (const uint4*)((const uint16_t*)x + st.c0);
        st.raw[0] = p[0];
        st.raw[1] = p[1];
    } else {
        const uint4* p = (const uint4*)((const float*)x + st.c0);
#pragma unroll
        for (int i = 0; i < 4; ++i) st.raw[i] = p[i];
    }
}
// Act-quant of the 64-block the thread's quad covers (E/compute.rs:2504-2521,
// block 64): q = the E4M3 values before the block scale sc.  All lanes take
// part in the block's amax; returns false for a thread without columns.
// Non-finite inputs keep the reference's f32 semantics: the amax skips NaN
// (f32::max), a NaN quantizes to the lowest sorted-LUT entry, -480
// (partition_point over NaN is 0), and an infinite amax makes the scale
// infinite, so every value of that block dequantizes to a non-finite value
// and the matvecs downstream report NonFiniteOutput.  *nonfinite is set when
// the block held an inf or NaN (the batch path keeps such inputs off MFMA).
__device__ __forceinline__ bool wh_xq_quant16(const wh_xq_stage& st, bool bf16, const uint32_t* log2_thr,
                                              float (&q)[16], float& sc, bool* nonfinite = nullptr) {
    float v[16];
    if (bf16) {
        const uint32_t w[8] = {st.raw[0].x, st.raw[0].y, st.raw[0].z, st.raw[0].w,
                               st.raw[1].x, st.raw[1].y, st.raw[1].z, st.raw[1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[4 * i] = __uint_as_float(st.raw[i].x);
            v[4 * i + 1] = __uint_as_float(st.raw[i].y);
            v[4 * i + 2] = __uint_as_float(st.raw[i].z);
            v[4 * i + 3] = __uint_as_float(st.raw[i].w);
        }
    }
    float amax = 0.0f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float m = fabsf(v[i]);
        bad |= !(m <= 3.4028235e38f);
        amax = fmaxf(amax, m);  // a NaN operand is skipped
    }
    amax = fmaxf(amax, wh_dpp_quad_swap1(amax));  // the quad holds one 64-block
    amax = fmaxf(amax, wh_dpp_quad_swap2(amax));
    if (!st.on) return false;
    if (nonfinite) *nonfinite = bad;
    const bool inf_scale = !(amax <= 3.4028235e38f);
    const int k = inf_scale ? 0 : wh_aq_scale_exp(amax, log2_thr);
    // v / inf is v * 0 for every v: +-0 for finite v, NaN for +-inf
    const float inv = inf_scale ? 0.0f : wh_pow2f(-k);
    sc = inf_scale ? __uint_as_float(0x7f800000u) : wh_pow2f(k);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float t = v[i] * inv;
        q[i] = t != t ? -480.0f : wh_e4m3_round(wh_clamp448_finite(t));
    }
    return true;
}
// The same, result written to LDS in FP4 lane order (scaled values).
__device__ __forceinline__ void wh_xq_stage_store(const wh_xq_stage& st, bool bf16, float* xs,
                                                  const uint32_t* log2_thr) {
    float q[16], sc;
    if (!wh_xq_quant16(st, bf16, log2_thr, q, sc)) return;
    // columns c0 + j: group c0/32, lane j % 8, k = 2*((c0/16) & 1) + j/8
    const uint32_t g = st.c0 >> 5, h = (st.c0 >> 4) & 1;
#pragma unroll
    for (int l = 0; l < 8; ++l) ((float2*)xs)[wh_xs_f4(g, l) * 2 + h] = make_float2(q[l] * sc, q[8 + l] * sc);
}

__device__ __forceinline__ float wh_dpp_row_shl8(float v) {  // lane i <- lane i+8 (within 16)
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x108, 0xf, 0xf, false));
}

// The first gate/up workgroup of a token clears the token's routed-sum
// arrival counters, which the down launch after it counts with: whatever
// the counters' memory held before, every call starts from zero.
// The token's arrival counters: hidden / 16 of them (one per 16-row output
// slice; the exact kernels' 32-row slices use the first half).
__device__ __forceinline__ void wh_moe_clear_arrivals(const wh_moe_args& a, uint32_t tok) {
    if (blockIdx.x != 0) return;
    uint32_t* cnt = a.cnt_y + (size_t)tok * (a.hidden >> 4);
    for (uint32_t i = threadIdx.x; i < (a.hidden >> 4); i += blockDim.x)
        __hip_atomic_store(cnt + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Gate/up: grid (n_experts * inter / 16, n_tokens), 256 threads = 32 rows =
// 16 hidden rows x {w1, w3}; octet 2r runs w1 row r, octet 2r+1 the w3 row r.
// kBlk = hidden / 256 when the rows fit in registers, else 0.
template <int kBlk, int kRing = (kBlk < 4 ? 2 : 4)>
__global__ void __launch_bounds__(256) k_moe_gateup(wh_moe_args a) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t tok = blockIdx.y;
    const uint32_t per_e = a.inter >> 4;
    const uint32_t e = blockIdx.x / per_e;
    const uint32_t rb = blockIdx.x - e * per_e;  // 16-row block of the hidden
    const uint32_t lane = threadIdx.x & 7, oct = threadIdx.x >> 3;
    const uint32_t row = rb * 16 + (oct >> 1);
    const bool up = oct & 1;
    const uint32_t G = a.hidden >> 5;
    const wh_expert_ptrs ep = wh_moe_ex(a, e);
    const uint8_t* wrow = (up ? ep.w3 : ep.w1) + (size_t)row * (a.hidden >> 1);
    const uint8_t* srow = (up ? ep.s3 : ep.s1) + (size_t)row * G;
    float* xs = lds;
    float* s8row = lds + wh_xs_floats(a.hidden) + oct * wh_s8_stride(G);
    uint32_t* thr = (uint32_t*)(lds + wh_fp4_wg_lds(a.hidden) / sizeof(float));
    uint64_t* exp_tab = wh_exp_tab_after(thr);
    const bool bf16 = a.x_is_bf16 != 0;
    const void* xt = bf16 ? (const void*)((const uint16_t*)a.x + (size_t)tok * a.hidden)
                          : (const void*)((const float*)a.x + (size_t)tok * a.hidden);
    wh_moe_clear_arrivals(a, tok);
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    wh_exp_stage es;
    wh_exp_stage_load(es);
    float acc;
    if constexpr (kBlk > 0) {
        // staging loads first, then the weight row; the staging waits below
        // therefore never wait for weight bytes
        wh_xq_stage xst;
        wh_xq_stage_load(xst, xt, bf16, a.hidden, threadIdx.x);
        wh_s8_stage<kBlk> ss;
        wh_s8_stage_load<kBlk>(ss, srow, lane);
        wh_fp4_ring<kRing> r;
        wh_fp4_ring_prologue<kRing>(r, wrow, lane);
        __builtin_amdgcn_sched_barrier(0);
        wh_thr_stage_store(ts, thr);
        wh_exp_stage_store(es, exp_tab);
        __syncthreads();
        wh_xq_stage_store(xst, bf16, xs, thr);
        wh_s8_stage_store<kBlk>(ss, s8row, lane);
        __syncthreads();
        acc = wh_fp4_ring_dot<kBlk, kRing>(r, wrow, xs, s8row, lane);
    } else {
        wh_thr_stage_store(ts, thr);
        wh_exp_stage_store(es, exp_tab);
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < (a.hidden >> 4); i += 256) {
            wh_xq_stage xst;
            wh_xq_stage_load(xst, xt, bf16, a.hidden, i);
            wh_xq_stage_store(xst, bf16, xs, thr);
        }
        wh_s8_stage_rt(srow, G, s8row, lane);
        __syncthreads();
        acc = wh_fp4_lane_dot_rt(wrow, G >> 3, xs, s8row, lane);
    }
    const float v = wh_hsum8(acc) + 0.0f;
    const float u = wh_dpp_row_shl8(v);  // lane 16k <- lane 16k + 8: the w3 row
    if ((threadIdx.x & 15) == 0) {
        if (!(fabsf(v) <= 3.4028235e38f) || !(fabsf(u) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        a.h[((size_t)tok * a.n_experts + e) * a.inter + row] = wh_swiglu(v, u, exp_tab, kExpfExc, WH_EXPF_EXC_COUNT);
        if (a.gu) {
            float* gu = a.gu + ((size_t)tok * a.n_experts + e) * 2 * a.inter;
            gu[row] = v;
            gu[a.inter + row] = u;
        }
    }
}

// Act-quant (block 64) of the hidden while staging it: thread t takes the 8
// values [8t, 8t+8), so 8 consecutive threads hold one 64-block; the result
// goes to LDS in FP4 lane order.  Loaded early, stored after the weight
// loads are issued.
struct wh_h_stage {
    float4 p, q;
    uint32_t t;
    bool on;
};
__device__ __forceinline__ void wh_h_stage_load(wh_h_stage& st, const float* __restrict__ h, uint32_t n, uint32_t t) {
    st.t = t;
    st.on = t < n / 8;
    if (st.on) {
        st.p = ((const float4*)h)[2 * t];
        st.q = ((const float4*)h)[2 * t + 1];
    } else {
        st.p = st.q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}
template <bool kCodes = false>
__device__ __forceinline__ void wh_h_stage_store(const wh_h_stage& st, float* xs, const uint32_t* log2_thr,
                                                 float* xk = nullptr) {
    const float v[8] = {st.p.x, st.p.y, st.p.z, st.p.w, st.q.x, st.q.y, st.q.z, st.q.w};
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, wh_dpp_quad_swap1(amax));
    amax = fmaxf(amax, wh_dpp_quad_swap2(amax));
    const float lo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x104, 0xf, 0xf, false));
    const float hi = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x114, 0xf, 0xf, false));
    amax = fmaxf(amax, (threadIdx.x & 4) ? hi : lo);  // the other quad of the 64-block
    if (!st.on) return;
    if (!(amax <= 3.4028235e38f)) amax = 1.0f;        // non-finite rows already reported
    const int k = wh_aq_scale_exp(amax, log2_thr);
    const float inv = wh_pow2f(-k), sc = wh_pow2f(k);
    const uint32_t g = st.t >> 2, kk = st.t & 3;  // columns 32g + 8kk + j: lane j, slot kk
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float q = wh_e4m3_round(wh_clamp448_finite(v[j] * inv));
        xs[wh_xs_f4(g, j) * 4 + kk] = kCodes ? q : q * sc;
    }
    if constexpr (kCodes) {
        if ((st.t & 7) == 0) xk[st.t >> 3] = sc;
    }
}

// After this workgroup's y stores of 32-row slice rb: the last expert
// workgroup of the slice to arrive sums all experts' rows in route order
// (E/compute.rs:1948-2012).  All threads of the workgroup call it.
__device__ __forceinline__ void wh_moe_routed_sum(const wh_moe_args& a, uint32_t tok, uint32_t rb, uint32_t* last) {
    wh_stores_done();
    __syncthreads();
    uint32_t* cnt = a.cnt_y + (size_t)tok * (a.hidden >> 4) + rb;
    if (threadIdx.x == 0) *last = wh_arrive(cnt) == a.n_experts - 1;
    __syncthreads();
    if (!*last || threadIdx.x >= 32) return;
    const uint32_t r_out = rb * 32 + threadIdx.x;
    const size_t t0 = (size_t)tok * a.n_experts * a.hidden;
    // every expert's row is requested before any is used: one round trip
    // to the coherent level instead of one per expert
    float yv[WH_MAX_EXPERTS];
#pragma unroll
    for (uint32_t i = 0; i < WH_MAX_EXPERTS; ++i)
        yv[i] = i < a.n_experts ? wh_load_coherent(a.y + t0 + (size_t)i * a.hidden + r_out) : 0.0f;
    a.out[(size_t)tok * a.hidden + r_out] = wh_route_combine(a, yv);
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Down + ordered routed sum: grid (n_experts * hidden / 32, n_tokens), 256
// threads = 32 output rows of one expert.  The last expert to finish a
// 32-row slice sums all experts in route order (E/compute.rs:1948-2012).
template <int kBlk, int kRing = (kBlk < 4 ? 2 : 4)>
__global__ void __launch_bounds__(256) k_moe_down(wh_moe_args a) {
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t last;
    const uint32_t tok = blockIdx.y;
    const uint32_t per_e = a.hidden >> 5;
    const uint32_t e = blockIdx.x / per_e;
    const uint32_t rb = blockIdx.x - e * per_e;  // 32-row slice of the output
    const uint32_t lane = threadIdx.x & 7, oct = threadIdx.x >> 3;
    const uint32_t row = rb * 32 + oct;
    const uint32_t G = a.inter >> 5;
    const wh_expert_ptrs ep = wh_moe_ex(a, e);
    const uint8_t* wrow = ep.w2 + (size_t)row * (a.inter >> 1);
    const uint8_t* srow = ep.s2 + (size_t)row * G;
    float* xs = lds;
    float* s8row = lds + wh_xs_floats(a.inter) + oct * wh_s8_stride(G);
    uint32_t* thr = (uint32_t*)(lds + wh_fp4_wg_lds(a.inter) / sizeof(float));
    const float* hrow = a.h + ((size_t)tok * a.n_experts + e) * a.inter;
    wh_thr_stage ts;
    wh_thr_stage_load(ts);
    float acc;
    if constexpr (kBlk > 0) {
        wh_h_stage hst;
        wh_h_stage_load(hst, hrow, a.inter, threadIdx.x);  // inter == 2048: one pass
        wh_s8_stage<kBlk> ss;
        wh_s8_stage_load<kBlk>(ss, srow, lane);
        wh_fp4_ring<kRing> r;
        wh_fp4_ring_prologue<kRing>(r, wrow, lane);
        __builtin_amdgcn_sched_barrier(0);
        wh_thr_stage_store(ts, thr);
        __syncthreads();
        wh_h_stage_store(hst, xs, thr);
        wh_s8_stage_store<kBlk>(ss, s8row, lane);
        __syncthreads();
        acc = wh_fp4_ring_dot<kBlk, kRing>(r, wrow, xs, s8row, lane);
    } else {
        wh_thr_stage_store(ts, thr);
        __syncthreads();
        for (uint32_t t = threadIdx.x; t < a.inter / 8; t += 256) {
            wh_h_stage hst;
            wh_h_stage_load(hst, hrow, a.inter, t);
            wh_h_stage_store(hst, xs, thr);
        }
        wh_s8_stage_rt(srow, G, s8row, lane);
        __syncthreads();
        acc = wh_fp4_lane_dot_rt(wrow, G >> 3, xs, s8row, lane);
    }
    const float yv = wh_hsum8(acc) + 0.0f;
    const size_t yb = ((size_t)tok * a.n_experts + e) * a.hidden;
    if (lane == 0) {
        if (!(fabsf(yv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        wh_store_coherent(a.y + yb + row, yv);
    }
    wh_moe_routed_sum(a, tok, rb, &last);
}

// Bit-exact dequant of a resident FP4 tensor back to reference values
// (decode_fp4_e2m1(nibble, scale), E/deepseek_v4.rs:358-372), through the
// same decode the matvec uses: out = (x8 value) * 0.125 * scale.
__global__ void __launch_bounds__(256) k_fp4_dequant(const uint8_t* __restrict__ w,
                                                     const uint8_t* __restrict__ s, uint32_t rows,
                                                     uint32_t cols, float* __restrict__ out) {
    // one thread per (row, block, lane): 8 groups x 4 values
    const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t blocks = cols >> 8, G = cols >> 5;
    if (id >= (size_t)rows * blocks * 8) return;
    const uint32_t lane = id & 7, b = (id >> 3) % blocks;
    const size_t row = (id >> 3) / blocks;
    const uint4 wv = ((const uint4*)(w + row * (cols / 2)))[8 * b + lane];
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
    for (uint32_t d = 0; d < 4; ++d) {
        const wh_fp4x8 v = wh_fp4_decode8(words[d]);
        const float va[4] = {v.a01.x, v.a01.y, v.a23.x, v.a23.y};
        const float vb[4] = {v.b01.x, v.b01.y, v.b23.x, v.b23.y};
        const uint32_t ga = 8 * b + 2 * d;
        const float sa = wh_ue8m0(s[row * G + ga]), sb = wh_ue8m0(s[row * G + ga + 1]);
        for (uint32_t k = 0; k < 4; ++k) {
            const float a8 = va[k] * 0.125f, b8 = vb[k] * 0.125f;
            out[row * cols + ga * 32 + lane + 8 * k] = a8 == 0.0f ? 0.0f : a8 * sa;
            out[row * cols + (ga + 1) * 32 + lane + 8 * k] = b8 == 0.0f ? 0.0f : b8 * sb;
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
// fn 0: silu(x), 1: expf(x), 2: 2^ceil(log2f(max(x,1e-4)/448)).
__global__ void k_debug_eval(int fn, const float* __restrict__ in, float* __restrict__ out, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float x = in[i];
    float r;
    if (fn == 0) r = wh_silu(x, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
    else if (fn == 1) r = wh_expf_glibc(x, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
    else r = wh_pow2f(wh_aq_scale_exp(x, kLog2Thr));
    out[i] = r;
}

// Plain streaming copy (fn 3 of the debug entry): the known-size kernel that
// calibrates the HBM byte counters against the hot kernels' algorithmic bytes.
__global__ void __launch_bounds__(256) k_copy_f32x4(const float4* __restrict__ in, float4* __restrict__ out, uint32_t n4) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) out[i] = in[i];
}
