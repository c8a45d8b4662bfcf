// Multi-input FP8 GEMV in the reference's order, each weight byte decoded
// once for all the inputs: gemv_fp8_e4m3_ue8m0_rows_multi (E/compute.rs:
// 6384-6577) decodes a weight row to f32 once, then runs every input's dot
// on the decoded row with the single-input kernel's reduction order
// (fp8_ue8m0_dot_row, E/compute.rs:5978-6018): per AVX lane l, per 128-col
// group, g0 and g1 chains of 8 FMAs (cols 16c + l and 16c + 8 + l), acc =
// fma(g0 + g1, scale, acc) over the groups in order, then the pairwise
// horizontal sum.  Bit-identical to the single-input kernels for every
// input.
//
// Thread (rows p and p + 16 with p = t / 8, AVX lane t % 8) of a 32-row
// workgroup holds 2 kN accumulators, one per row and input, and walks the
// groups in order; each group's 16 weight bytes of the lane are decoded once
// and dotted with the kN inputs' x values (one LDS read of a lane's x
// serves both rows), which stream through LDS in chunks of groups (the
// lane's 16 values of a group contiguous, as the single-input kernels stage
// them), double-buffered, with the next chunk's weights and x loads in
// flight during the current chunk's arithmetic.
#pragma once
#include "kernels.h"

#define WH_FP8_MULTI_ROWS 32u  // rows per workgroup (128 threads, two rows each)

// 128-column groups per staged chunk for kN inputs: 2 (a chunk of 16
// inputs' x and the next chunk's loads leave room for two waves per SIMD),
// more for fewer inputs so that every thread stages at least one 16-value
// unit.  cols must be a multiple of 128 times this.
#ifndef WH_FP8_MULTI_KC
#define WH_FP8_MULTI_KC 2
#endif
__host__ __device__ constexpr int wh_fp8_multi_groups(int n) {
    return WH_FP8_MULTI_KC * n >= 16 ? WH_FP8_MULTI_KC : 16 / n;
}

// Grid (row blocks [+ the second tensor's], ceil(n_in / kN)), 128 threads,
// kN in {2, 4, 8, 16}.  cols % (128 wh_fp8_multi_groups(kN)) == 0; a workgroup's rows lie in one input's
// row group.  The host takes the largest kN that still gives a few hundred
// workgroups (small matrices re-read their weights from cache once per
// input block).
template <int kN, bool kSpecial, bool kScaleU8>
__global__ void __launch_bounds__(128) k_fp8_gemv_multi(wh_fp8_args a, uint32_t n_in) {
    constexpr int kT = 128;                          // threads
    constexpr int kC = wh_fp8_multi_groups(kN);
    constexpr int kChunk = kC * 128;                 // columns per chunk
    constexpr int kUnits = kN * kChunk / 16 / kT;    // 16-value staging units per thread per chunk
    static_assert(kUnits >= 1 && kN * kChunk % (16 * kT) == 0, "staging units");
    __shared__ __align__(16) float xs[2][kN][kChunk];
    const uint32_t t = threadIdx.x, p = t >> 3, l = t & 7;
    // which tensor: blocks from blocks1 on run the second one
    const bool two = blockIdx.x >= a.blocks1;
    const uint8_t* w = two ? a.w2 : a.w;
    const void* sc = two ? a.scales2 : a.scales;
    const uint32_t scale_cols = two ? a.scale_cols2 : a.scale_cols;
    const uint32_t rg_shift = two ? a.row_group_shift2 : a.row_group_shift;
    const uint32_t r_lo = two ? a.row_start2 : a.row_start, r_hi = two ? a.row_end2 : a.row_end;
    float* yb = two ? a.y2 : a.y;
    const uint32_t blk = two ? blockIdx.x - a.blocks1 : blockIdx.x;
    const uint32_t row0 = r_lo + blk * WH_FP8_MULTI_ROWS;
    const uint32_t cols = a.cols, n_chunks = cols / kChunk;
    const uint32_t i0 = blockIdx.y * kN;
    const uint32_t n_here = min((uint32_t)kN, n_in - i0);
    const uint32_t grp = a.x_group_shift < 32 ? (row0 - a.row_start) >> a.x_group_shift : 0u;
    const float* xbase = a.x + (size_t)i0 * a.x_stride + (size_t)grp * a.x_group_stride;
    const uint4* wrow[2];
    uint32_t srow[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t row = row0 + p + 16 * h;
        row = row < r_hi ? row : r_hi - 1;  // rows past the end repeat the last one; not stored
        wrow[h] = (const uint4*)(w + (size_t)row * cols) + l;  // group g at wrow[h][8 g]
        srow[h] = (row >> rg_shift) * scale_cols;
    }

    // staging unit u = t + kT k: input u / (kChunk / 16), 16 columns
    // 16 (u % (kChunk / 16)) .. of the chunk
    float4 xr[kUnits][4];
    auto load_x = [&](uint32_t chunk) {
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const uint32_t u = t + kT * k, i = u / (kChunk / 16), q = u % (kChunk / 16);
            const float4* src = (const float4*)(xbase + (size_t)i * a.x_stride + (size_t)chunk * kChunk + 16 * q);
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[k][j] = i < n_here ? src[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const uint32_t u = t + kT * k, i = u / (kChunk / 16), q = u % (kChunk / 16);
            const uint32_t g = q >> 3, c = q & 7;
            float* dst = xs[buf][i];
#pragma unroll
            for (int o = 0; o < 16; ++o) {
                const uint32_t lo = o & 7, idx = (o >> 3) * 8 + c;
                dst[((g * 8 + lo) << 4) + idx] = wh_f4_get(xr[k][o >> 2], o & 3);
            }
        }
    };
    uint4 wv[2][kC], wn[2][kC];
    float sv[2][kC], sn[2][kC];
    auto load_w = [&](uint32_t chunk, uint4 (&wd)[2][kC], float (&sd)[2][kC]) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int g = 0; g < kC; ++g) {
                const uint32_t gi = chunk * kC + g;
                wd[h][g] = wrow[h][8 * gi];
                sd[h][g] = wh_fp8_scale<kSpecial, kScaleU8>(sc, srow[h] + gi);
            }
    };
    float acc[2][kN];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < kN; ++i) acc[h][i] = 0.0f;

    load_x(0);
    load_w(0, wv, sv);
    store_x(0);
    __syncthreads();
    for (uint32_t k = 0; k < n_chunks; ++k) {
        const int buf = k & 1;
        const bool more = k + 1 < n_chunks;
        if (more) {
            load_x(k + 1);
            load_w(k + 1, wn, sn);
        }
#pragma unroll
        for (int g = 0; g < kC; ++g) {
            // the lane's 16 weights of group g of both rows, decoded once
            float wd[2][16];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t d[4] = {wv[h][g].x, wv[h][g].y, wv[h][g].z, wv[h][g].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const wh_f2 lo = wh_fp8x2<kSpecial, false>(d[q]), hi = wh_fp8x2<kSpecial, true>(d[q]);
                    wd[h][4 * q] = lo.x;
                    wd[h][4 * q + 1] = lo.y;
                    wd[h][4 * q + 2] = hi.x;
                    wd[h][4 * q + 3] = hi.y;
                }
            }
#pragma unroll
            for (int i = 0; i < kN; ++i) {
                if ((uint32_t)i < n_here) {
                    const float4* xp = (const float4*)(xs[buf][i] + ((g * 8 + l) << 4));
                    const float4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float* v = wd[h];
                        float g0 = __builtin_fmaf(v[0], x0.x, 0.0f);
                        g0 = __builtin_fmaf(v[1], x0.y, g0);
                        g0 = __builtin_fmaf(v[2], x0.z, g0);
                        g0 = __builtin_fmaf(v[3], x0.w, g0);
                        g0 = __builtin_fmaf(v[4], x1.x, g0);
                        g0 = __builtin_fmaf(v[5], x1.y, g0);
                        g0 = __builtin_fmaf(v[6], x1.z, g0);
                        g0 = __builtin_fmaf(v[7], x1.w, g0);
                        float g1 = __builtin_fmaf(v[8], x2.x, 0.0f);
                        g1 = __builtin_fmaf(v[9], x2.y, g1);
                        g1 = __builtin_fmaf(v[10], x2.z, g1);
                        g1 = __builtin_fmaf(v[11], x2.w, g1);
                        g1 = __builtin_fmaf(v[12], x3.x, g1);
                        g1 = __builtin_fmaf(v[13], x3.y, g1);
                        g1 = __builtin_fmaf(v[14], x3.z, g1);
                        g1 = __builtin_fmaf(v[15], x3.w, g1);
                        acc[h][i] = __builtin_fmaf(g0 + g1, sv[h][g], acc[h][i]);
                    }
                }
            }
        }
        if (more) {
            store_x(buf ^ 1);
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int g = 0; g < kC; ++g) {
                    wv[h][g] = wn[h][g];
                    sv[h][g] = sn[h][g];
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t out_row = row0 + p + 16 * h;
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const float s = wh_hsum8(acc[h][i]) + 0.0f;  // + tail (0 for col_group % 16 == 0)
            if ((uint32_t)i < n_here && l == 0 && out_row < r_hi) {
                yb[(size_t)(i0 + i) * a.y_stride + (out_row - r_lo)] = s;
                if (!(fabsf(s) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            }
        }
    }
}
