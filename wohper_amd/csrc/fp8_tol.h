// FP8 E4M3 dequant GEMV with the summation order freed (exact numerics off):
// gemv_fp8_e4m3_ue8m0_tensorwise / _rows (E/compute.rs:6174-6321) for one
// input, within max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2 of the reference's
// AVX2 kernel.  The exact kernel (k_fp8_gemv_sk) reproduces the reference's
// per-lane FMA chain and hands every row's partial sums to one wave for the
// ordered scale FMAs; this one reads like the HBM read-floor kernel instead:
// every load of a thread issued before any arithmetic, no ordered hand-off,
// cross-lane sums on the DPP / permlane-swap paths rather than through LDS.
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

template <int kCtrl>
__device__ __forceinline__ float wh_dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, false));
}

// One halving step of a wave sum over lane bit kB (32, 16, 8, 4, 2, 1):
// every lane holds kN partial sums v[0..kN); lanes with bit kB clear keep
// sums [0, kN/2), the others [kN/2, kN), each adding the copy of a partner
// lane with the same higher bits and the opposite bit kB.  kN = 1 adds the
// partner's single value.  Partners: v_permlane32_swap (lanes L <-> L ^ 32),
// v_permlane16_swap (L <-> L ^ 16), DPP row_ror:8 (L ^ 8), row_half_mirror
// (L <-> L ^ 7 inside 8 lanes: bit 2 flips), quad_perm (L ^ 2, L ^ 1).
template <int kB, int kN, int kCap>
__device__ __forceinline__ void wh_wave_halve(float (&v)[kCap], uint32_t L) {
    if constexpr (kB == 32 || kB == 16) {
        // the swap exchanges the upper half of its first operand's pairs of
        // lanes with the lower half of its second: lanes with bit kB clear
        // then hold (own A, partner A), the others (partner B, own B)
#pragma unroll
        for (int p = 0; p < (kN > 1 ? kN / 2 : 1); ++p) {
            const float A = v[p], B = kN > 1 ? v[p + kN / 2] : v[p];
            const auto r = kB == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(A), __float_as_uint(B), false, false)
                                    : __builtin_amdgcn_permlane16_swap(__float_as_uint(A), __float_as_uint(B), false, false);
            v[p] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
    } else {
        constexpr int kCtrl = kB == 8 ? 0x128 : kB == 4 ? 0x141 : kB == 2 ? 0x4E : 0xB1;
        const bool up = (L & kB) != 0;
#pragma unroll
        for (int p = 0; p < (kN > 1 ? kN / 2 : 1); ++p) {
            if constexpr (kN > 1) {
                const float A = v[p], B = v[p + kN / 2];
                v[p] = (up ? B : A) + wh_dpp_f<kCtrl>(up ? A : B);
            } else {
                v[p] = v[p] + wh_dpp_f<kCtrl>(v[p]);
            }
        }
    }
}

// Sums kP values per lane over the wave: afterwards sum p sits in the lanes
// L with L % (64 / kP) == 0, p = L / (64 / kP).
template <int kP>
__device__ __forceinline__ void wh_wave_sums(float (&v)[kP], uint32_t L) {
    wh_wave_halve<32, (kP >= 2 ? kP : 1)>(v, L);
    wh_wave_halve<16, (kP >= 4 ? kP / 2 : 1)>(v, L);
    wh_wave_halve<8, (kP >= 8 ? kP / 4 : 1)>(v, L);
    wh_wave_halve<4, (kP >= 16 ? kP / 8 : 1)>(v, L);
    wh_wave_halve<2, (kP >= 32 ? kP / 16 : 1)>(v, L);
    wh_wave_halve<1, (kP >= 64 ? kP / 32 : 1)>(v, L);
}

// Grid (blocks [+ the second tensor's blocks], n_batch), 64 kW threads.
// Wave w takes the 1024-col slice w % kS of kP rows: rows row0 + w / kS +
// (kW / kS) p, p < kP, so a block covers kR = kP kW / kS rows and every wave
// reuses its 16 x values kP times.  kOneSR: every block's rows lie in one
// scale row (the host checks rows per scale row % kR == 0 and row starts %
// kR == 0), so a lane loads one scale for all its pairs.
template <int kW, int kS, int kP, bool kScaleU8, bool kOneSR>
__global__ void __launch_bounds__(64 * kW) k_fp8_gemv_tol(wh_fp8_args a) {
    static_assert(kW % kS == 0 && (kS == 1 || kS == 2 || kS == 4 || kS == 8), "slices per block");
    static_assert(kP == 1 || kP == 2 || kP == 4 || kP == 8 || kP == 16, "pairs per wave");
    constexpr int kRw = kW / kS;  // waves per slice
    constexpr int kR = kP * kRw;  // rows per block
    __shared__ float red[kR][kS];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), L = threadIdx.x & 63;
    const uint32_t gi = L >> 3, l = L & 7;
    const uint32_t sl = wave % kS, rw = wave / kS;
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
    const uint32_t col = sl * 1024 + gi * 128;
    // this block's input (row groups with their own input share one block)
    const uint32_t grp = a.x_group_shift < 32 ? (row0 - a.row_start) >> a.x_group_shift : 0u;
    const float* xs = a.x + (size_t)blockIdx.y * a.x_stride + (size_t)grp * a.x_group_stride + col + l;
    // x first: the first pair's arithmetic waits for x and its own weights
    // only
    float xa[8], xb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        xa[j] = xs[16 * j];
        xb[j] = xs[16 * j + 8];
    }
    // weight chunks of the wave's pairs (rows past r_hi repeat the last row;
    // their sums are not stored)
    uint4 wv[kP];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
        uint32_t row = row0 + rw + kRw * p;
        row = row < r_hi ? row : r_hi - 1;
        wv[p] = *(const uint4*)(w + (size_t)row * cols + col + 16 * l);
    }
    constexpr int kSc = kOneSR ? 1 : kP;
    float s[kSc];
#pragma unroll
    for (int p = 0; p < kSc; ++p) {
        uint32_t row = row0 + rw + kRw * p;
        row = row < r_hi ? row : r_hi - 1;
        s[p] = wh_fp8_scale<false, kScaleU8>(sc, (row >> rg_shift) * scale_cols + (col >> 7));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any arithmetic
    float v[kP];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
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
            g = __builtin_fmaf(a0[0], xa[4 * q], g);
            g = __builtin_fmaf(a0[1], xa[4 * q + 1], g);
            g = __builtin_fmaf(a1[0], xa[4 * q + 2], g);
            g = __builtin_fmaf(a1[1], xa[4 * q + 3], g);
            g = __builtin_fmaf(b0[0], xb[4 * q], g);
            g = __builtin_fmaf(b0[1], xb[4 * q + 1], g);
            g = __builtin_fmaf(b1[0], xb[4 * q + 2], g);
            g = __builtin_fmaf(b1[1], xb[4 * q + 3], g);
        }
        v[p] = g * s[kOneSR ? 0 : p];
    }
    wh_wave_sums<kP>(v, L);
    const bool holder = (L & ((64 / kP) - 1)) == 0;
    const uint32_t p = L / (64 / kP);
    const uint32_t r = rw + kRw * p;  // the block row of sum p
    if constexpr (kS == 1) {
        const uint32_t row = row0 + r;
        if (holder && row < r_hi) {
            if (!(fabsf(v[0]) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            yb[(size_t)blockIdx.y * a.y_stride + (row - r_lo)] = v[0];
        }
    } else {
        if (holder) red[r][sl] = v[0];
        __syncthreads();
        if (threadIdx.x < kR) {
            const uint32_t rr = threadIdx.x, row = row0 + rr;
            float y = red[rr][0];
#pragma unroll
            for (int k = 1; k < kS; ++k) y += red[rr][k];
            if (row < r_hi) {
                if (!(fabsf(y) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
                yb[(size_t)blockIdx.y * a.y_stride + (row - r_lo)] = y;
            }
        }
    }
}
