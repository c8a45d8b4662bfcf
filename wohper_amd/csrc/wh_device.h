// Device-side building blocks shared by the decode-path kernels (gfx950).
//
// Numerics follow the reference CPU kernels operation for operation:
//   FP8 row dot  E/compute.rs:5978-6018  (8 lanes, g0/g1 chains of 8 FMAs per
//                128-col group, acc = fma(g0 + g1, scale, acc), pairwise hsum)
//   FP4 row dot  E/deepseek_v4.rs:294-347 (8 lanes, 4 FMAs per 32-col group on
//                the x8 integer LUT values, acc = fma(gacc, scale/8, acc))
// One AVX lane maps to one GPU thread; the horizontal sum is a DPP tree with
// the same ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)) shape.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "libm_emul.h"

typedef float wh_f2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- FP8 codes
// gfx950 converts OCP E4M3 (bias 7) in hardware.  Codes 0x7F/0xFF are NaN
// there but +-480 in the reference (E/deepseek_v4.rs:151-164); tensors that
// contain them take the kSpecial path.  0x80 decodes to -0 instead of +0,
// which never changes a sum that starts from +0.
template <bool kSpecial, bool kHi>
__device__ __forceinline__ wh_f2 wh_fp8x2(uint32_t w) {
    wh_f2 v = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, kHi);
    if constexpr (kSpecial) {
        uint32_t b0 = kHi ? (w >> 16) & 0xff : w & 0xff;
        uint32_t b1 = kHi ? (w >> 24) & 0xff : (w >> 8) & 0xff;
        if ((b0 & 0x7f) == 0x7f) v.x = (b0 & 0x80) ? -480.0f : 480.0f;
        if ((b1 & 0x7f) == 0x7f) v.y = (b1 & 0x80) ? -480.0f : 480.0f;
    }
    return v;
}

// Reference-exact scalar decode of one FP8 byte (all 256 codes).
__device__ __forceinline__ float wh_fp8_exact(uint32_t b) {
    b &= 0xff;
    uint32_t e = (b >> 3) & 0xf, m = b & 7;
    if (e == 0 && m == 0) return 0.0f;
    float v = e == 0 ? (float)m * 0.001953125f /* m/8 * 2^-6 */
                     : (1.0f + (float)m * 0.125f) * wh_pow2f((int)e - 7);
    return (b & 0x80) ? -v : v;
}

// ---------------------------------------------------------------- FP4 codes
// Resident FP4 encoding (written by fp4_encode_row and k_synth_fp4): one dword
// holds the 8 elements that one lane consumes from two consecutive 32-col
// groups, byte k = [sB_k | mB_k(3) | sA_(k-1 mod 4) | mA_k(3)], where A_k / B_k
// are column l + 8k of the first / second group and m/s are the E2M1
// magnitude index and sign bit of the original nibble.  A v_perm LUT maps 4
// magnitudes to the E4M3 codes of the reference's x8 integer values
// {0, 1, 8, 12, 16, 24, 32, 48} (E/deepseek_v4.rs:285-287), the sign bits
// are OR-ed in, and v_cvt_pk_f32_fp8 produces exact f32 values.
#define WH_FP4_LUT_LO 0x54503800u  // 0, 1, 8, 12  as E4M3
#define WH_FP4_LUT_HI 0x64605c58u  // 16, 24, 32, 48 as E4M3

struct wh_fp4x8 {
    wh_f2 a01, a23, b01, b23;
};

__device__ __forceinline__ wh_fp4x8 wh_fp4_decode8(uint32_t w, uint32_t lut_hi = WH_FP4_LUT_HI,
                                                   uint32_t lut_lo = WH_FP4_LUT_LO) {
    uint32_t sel_a = w & 0x07070707u;
    uint32_t fa = __builtin_amdgcn_perm(lut_hi, lut_lo, sel_a);
    uint32_t r = __builtin_amdgcn_alignbit(w, w, 4);  // rotate right by 4
    fa |= r & 0x80808080u;
    uint32_t sel_b = r & 0x07070707u;
    uint32_t fb = __builtin_amdgcn_perm(lut_hi, lut_lo, sel_b);
    fb |= w & 0x80808080u;
    wh_fp4x8 o;
    o.a01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)fa, false);
    o.a23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)fa, true);
    o.b01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)fb, false);
    o.b23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)fb, true);
    return o;
}

// Reference-exact x8 base value of one original nibble.
__device__ __forceinline__ float wh_fp4_x8(uint32_t nib) {
    const float mags[8] = {0.0f, 1.0f, 8.0f, 12.0f, 16.0f, 24.0f, 32.0f, 48.0f};
    float v = mags[nib & 7];
    return (nib & 8) ? -v : v;
}

// Reference base value (E/deepseek_v4.rs:177-180) of one original nibble.
__device__ __forceinline__ float wh_fp4_base(uint32_t nib) {
    const float mags[8] = {0.0f, 0.125f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = mags[nib & 7];
    return ((nib & 8) && (nib & 7)) ? -v : v;
}

// UE8M0 byte -> f32 2^(b-127); 0 -> 0.0, 255 -> +inf (E/deepseek_v4.rs:166-172)
__device__ __forceinline__ float wh_ue8m0(uint32_t b) { return __uint_as_float((b & 0xffu) << 23); }

// ------------------------------------------------------- cross-lane sums
__device__ __forceinline__ float wh_dpp_quad_swap1(float v) {  // quad_perm [1,0,3,2]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
}
__device__ __forceinline__ float wh_dpp_quad_swap2(float v) {  // quad_perm [2,3,0,1]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
}
__device__ __forceinline__ float wh_dpp_row_shl4(float v) {  // lane i <- lane i+4 (within 16)
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x104, 0xf, 0xf, false));
}

// Pairwise sum over each aligned group of 8 lanes in the AVX2 hsum order;
// the result is valid in lane 0 of the group (lanes 0 and 8 of each row).
__device__ __forceinline__ float wh_hsum8(float v) {
    float p1 = v + wh_dpp_quad_swap1(v);
    float p2 = p1 + wh_dpp_quad_swap2(p1);
    return p2 + wh_dpp_row_shl4(p2);
}

__device__ __forceinline__ float wh_wave_max(float v) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// ------------------------------------------------------------ act-quant
// Block scale of act-quant: exp2f(ceilf(log2f(max(amax,1e-4)/448)))
__device__ __forceinline__ int wh_aq_scale_exp(float amax, const uint32_t* log2_thr) {
    amax = fmaxf(amax, 1.0e-4f);
    float r = amax / 448.0f;
    return wh_ceil_log2f(r, log2_thr);
}

// f32::clamp(-448, 448)
__device__ __forceinline__ float wh_clamp448(float v) {
    return v < -448.0f ? -448.0f : (v > 448.0f ? 448.0f : v);
}
// The same clamp for finite v as one min/max pair; NaN maps to -448 (the
// staging paths that use it report non-finite inputs as errors).
__device__ __forceinline__ float wh_clamp448_finite(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }

// DeepSeek-V4 SwiGLU on one gate/up pair (E/deepseek_v4.rs:590-594)
__device__ __forceinline__ float wh_swiglu(float g, float u, const uint64_t* exp_tab,
                                           const uint32_t* exc, uint32_t n_exc) {
    float gated = fminf(g, 10.0f);
    float upped = u < -10.0f ? -10.0f : (u > 10.0f ? 10.0f : u);
    return wh_silu(gated, exp_tab, exc, n_exc) * upped;
}
