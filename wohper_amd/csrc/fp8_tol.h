// FP8 E4M3 dequant GEMV with the summation order freed (exact numerics off):
// gemv_fp8_e4m3_ue8m0_tensorwise / _rows (E/compute.rs:6174-6321) for one
// input, within max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2 of the reference's
// AVX2 kernel.  The exact kernel (k_fp8_gemv_sk) reproduces the reference's
// per-lane FMA chain and hands every row's partial sums to one wave for the
// ordered scale FMAs; this one reads like the HBM read-floor kernel instead:
// small workgroups, every weight load of a thread issued before any
// arithmetic, no LDS staging of x and no ordered hand-off.
//
// Resident layout (fp8_permute_row): in each 128-col group, 16-byte chunk l
// holds the columns l + 16 j (bytes 0..7) and l + 8 + 16 j (bytes 8..15),
// j = 0..7.  Lane L of a wave takes chunk L % 8 of group L / 8 of a 1024-col
// slice, so a wave reads 1 KB of a row contiguously and each lane needs the
// same 16 x values for every row of the slice: loaded once, kept in
// registers.  Bytes decode with v_cvt_pk_f32_fp8, exact for every code but
// 0x7F / 0xFF (the reference's +-480); tensors holding those keep the exact
// kernel.
#pragma once
#include "kernels.h"

// Grid (blocks of kR rows [+ the second tensor's blocks], n_batch), 256
// threads.  Work items are (row, 1024-col slice) pairs, kS slices a row;
// wave w runs pairs w, w + 4, ... of the block's kR * kS (a multiple of 4),
// so a wave keeps one slice when kS <= 4 and two when kS = 8.
template <int kR, int kS, bool kScaleU8>
__global__ void __launch_bounds__(256) k_fp8_gemv_tol(wh_fp8_args a) {
    static_assert((kR * kS) % 4 == 0 && (kS == 1 || kS == 2 || kS == 4 || kS == 8), "pairs per wave");
    constexpr int kP = kR * kS / 4;           // pairs per wave
    constexpr int kX = kS == 8 ? 2 : 1;        // x slices per wave
    __shared__ float red[kR][kS];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), L = threadIdx.x & 63;
    const uint32_t gi = L >> 3, l = L & 7;
    // which tensor: blocks from blocks1 on run the second one
    const bool two = blockIdx.x >= a.blocks1;
    const uint8_t* w = two ? a.w2 : a.w;
    const void* sc = two ? a.scales2 : a.scales;
    const uint32_t scale_cols = two ? a.scale_cols2 : a.scale_cols;
    const uint32_t rg_shift = two ? a.row_group_shift2 : a.row_group_shift;
    const uint32_t r_lo = two ? a.row_start2 : a.row_start, r_hi = two ? a.row_end2 : a.row_end;
    float* yb = two ? a.y2 : a.y;
    const uint32_t blk = two ? blockIdx.x - a.blocks1 : blockIdx.x;
    const uint32_t row0 = r_lo + blk * kR;
    const uint32_t cols = a.cols;
    // this block's input (row groups with their own input share one block)
    const uint32_t grp = a.x_group_shift < 32 ? (row0 - a.row_start) >> a.x_group_shift : 0u;
    const float* x = a.x + (size_t)blockIdx.y * a.x_stride + (size_t)grp * a.x_group_stride;
    // weight chunks of the wave's pairs (rows past r_hi repeat the last row;
    // their sums are not stored)
    uint4 wv[kP];
    float s[kP];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
        const uint32_t item = wave + 4 * p, r = item / kS, sl = item % kS;
        uint32_t row = row0 + r;
        row = row < r_hi ? row : r_hi - 1;
        const uint32_t col = sl * 1024 + gi * 128;
        wv[p] = *(const uint4*)(w + (size_t)row * cols + col + 16 * l);
        s[p] = wh_fp8_scale<false, kScaleU8>(sc, (row >> rg_shift) * scale_cols + (col >> 7));
    }
    float xa[kX][8], xb[kX][8];
#pragma unroll
    for (int k = 0; k < kX; ++k) {
        const uint32_t sl = (wave + 4 * k) % kS;
        const float* xs = x + sl * 1024 + gi * 128 + l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xa[k][j] = xs[16 * j];
            xb[k][j] = xs[16 * j + 8];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any arithmetic
    float acc[kP];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
        const int k = kX == 2 ? (p & 1) : 0;  // pairs alternate between the two slices when kS = 8
        const uint32_t d[4] = {wv[p].x, wv[p].y, wv[p].z, wv[p].w};
        float g = 0.0f;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            // bytes 4q .. 4q + 3: columns 16 (2q + {0, 1, 2, 3}) + l; bytes
            // 8 + 4q ..: the same + 8
            const auto a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[q], false);
            const auto a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[q], true);
            const auto b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[2 + q], false);
            const auto b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[2 + q], true);
            g = __builtin_fmaf(a0[0], xa[k][4 * q], g);
            g = __builtin_fmaf(a0[1], xa[k][4 * q + 1], g);
            g = __builtin_fmaf(a1[0], xa[k][4 * q + 2], g);
            g = __builtin_fmaf(a1[1], xa[k][4 * q + 3], g);
            g = __builtin_fmaf(b0[0], xb[k][4 * q], g);
            g = __builtin_fmaf(b0[1], xb[k][4 * q + 1], g);
            g = __builtin_fmaf(b1[0], xb[k][4 * q + 2], g);
            g = __builtin_fmaf(b1[1], xb[k][4 * q + 3], g);
        }
        acc[p] = g * s[p];
    }
    // sum each pair over the wave's 64 lanes: halving exchanges while there
    // are several sums per lane, then a tree on the last one
    float v[kP];
#pragma unroll
    for (int p = 0; p < kP; ++p) v[p] = acc[p];
    int n = kP, stride = 32;
#pragma unroll
    for (int step = 0; step < 6; ++step) {
        if (n > 1) {
            // lanes with bit `stride` clear keep the first half of the sums,
            // the others the second half; each adds its partner's copy
            const bool up = (L & stride) != 0;
#pragma unroll
            for (int p = 0; p < kP / 2; ++p) {
                if (p < n / 2) {
                    const float send = up ? v[p] : v[p + n / 2];
                    const float keep = up ? v[p + n / 2] : v[p];
                    v[p] = keep + __shfl_xor(send, stride, 64);
                }
            }
            n /= 2;
        } else {
            v[0] += __shfl_xor(v[0], stride, 64);
        }
        stride >>= 1;
    }
    // after the halvings, sum p lives in the lanes whose bits (32, 16, ...)
    // spell p, most significant first
    if ((L & ((64 / kP) - 1)) == 0) {
        const uint32_t p = L / (64 / kP);
        const uint32_t item = wave + 4 * p;
        red[item / kS][item % kS] = v[0];
    }
    __syncthreads();
    if (threadIdx.x < kR) {
        const uint32_t r = threadIdx.x, row = row0 + r;
        float y = red[r][0];
#pragma unroll
        for (int sl = 1; sl < kS; ++sl) y += red[r][sl];
        if (row < r_hi) {
            if (!(fabsf(y) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            yb[(size_t)blockIdx.y * a.y_stride + (row - r_lo)] = y;
        }
    }
}
