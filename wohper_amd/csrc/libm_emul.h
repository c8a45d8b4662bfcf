// glibc-exact float libm pieces used on the decode path, shared by the HIP
// device code and by the host-side table generator (gen_libm_tables.c).
//
// The reference engine calls the platform libm through Rust's f32 methods:
//   silu(x) = x / (1 + expf(-x))                 E/deepseek_v4.rs:551-554
//   act-quant block scale exp2f(ceilf(log2f(r)))  E/compute.rs:2514
// glibc's expf is not correctly rounded (it misrounds roughly 7e-5 of the
// inputs in [-10, 89]), so matching it bit for bit needs more than an
// accurate exp.  The scheme here:
//   1. wh_exp_double(y): exp(y) in double, relative error below 1e-15
//      (Cody-Waite reduction by ln2/32, 32-entry 2^(j/32) table, degree-6
//      Taylor polynomial), built only from IEEE add/mul/fma/rint, so host
//      and device evaluate it to the same bits.
//   2. Round to float.  If the double result lies within
//      WH_EXPF_WINDOW ulp of a float rounding midpoint, look the input up in
//      a sorted table of inputs where glibc's result is the other neighbour
//      of that midpoint, and flip.  The generator builds that table by
//      comparing this exact code with the host glibc expf over every float
//      input of the silu domain [-10, +inf), and then re-verifies the whole
//      domain.
//   3. ceil(log2f(r)) for normal r is e + (mantissa > T[e]), where the
//      per-binade thresholds T[] are found by scanning the host log2f and
//      verified over every mantissa of every binade.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define WH_HD __host__ __device__ inline
#else
#define WH_HD static inline
#endif

#define WH_EXPF_WINDOW 0.003  // in float ulps; must exceed glibc's error beyond 0.5 ulp

WH_HD double wh_bits_to_double(uint64_t b) {
    union { uint64_t u; double d; } v;
    v.u = b;
    return v.d;
}
WH_HD uint64_t wh_double_to_bits(double d) {
    union { uint64_t u; double d; } v;
    v.d = d;
    return v.u;
}
WH_HD float wh_bits_to_float(uint32_t b) {
    union { uint32_t u; float f; } v;
    v.u = b;
    return v.f;
}
WH_HD uint32_t wh_float_to_bits(float f) {
    union { uint32_t u; float f; } v;
    v.f = f;
    return v.u;
}

// exp(y) for finite y with |y| < 104 (callers clamp).  exp2_tab holds, as
// double bit patterns, 2^(j/32) for j = 0..31, then 32/ln2, then ln2/32 split
// into a 32-significant-bit head (so n*head is exact) and a tail; the
// generator derives them from long double arithmetic.
WH_HD double wh_exp_double(float yf, const uint64_t* exp2_tab) {
    const double inv_l = wh_bits_to_double(exp2_tab[32]);
    const double l_hi = wh_bits_to_double(exp2_tab[33]);
    const double l_lo = wh_bits_to_double(exp2_tab[34]);
    double x = (double)yf;
    double nd = __builtin_rint(x * inv_l);
    double r = __builtin_fma(-nd, l_hi, x);
    r = __builtin_fma(-nd, l_lo, r);
    // Taylor polynomial of exp(r) on |r| <= ln2/64, Horner with fma
    double p = 1.0 / 720.0;
    p = __builtin_fma(p, r, 1.0 / 120.0);
    p = __builtin_fma(p, r, 1.0 / 24.0);
    p = __builtin_fma(p, r, 1.0 / 6.0);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    int64_t n = (int64_t)nd;
    int64_t j = n & 31;
    int64_t k = (n - j) / 32;  // exact floor division
    double t = wh_bits_to_double(exp2_tab[j]);
    double s = wh_bits_to_double((uint64_t)(k + 1023) << 52);  // 2^k, |k| < 160 here
    return (t * p) * s;
}

// Returns 1 if the double result `d` (positive, finite) is within the window
// of the rounding midpoint between float(d) and its neighbour on d's side.
WH_HD int wh_expf_near_midpoint(double d, float f) {
    double fd = (double)f;
    double diff = d - fd;
    uint32_t fb = wh_float_to_bits(f);
    int ex = (int)((fb >> 23) & 0xff);
    if (ex == 0 || ex == 0xff) return 1;  // subnormal / inf: always consult the table
    double ulp = wh_bits_to_double((uint64_t)(ex - 127 - 23 + 1023) << 52);
    // below a power of two the neighbour spacing halves
    double ulp_side = (diff < 0.0 && (fb & 0x7fffff) == 0) ? ulp * 0.5 : ulp;
    double dist = 0.5 * ulp_side - (diff < 0.0 ? -diff : diff);
    return dist < WH_EXPF_WINDOW * ulp_side;
}

WH_HD int wh_table_contains(const uint32_t* tab, uint32_t n, uint32_t key) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        uint32_t mid = (lo + hi) >> 1;
        uint32_t v = tab[mid];
        if (v == key) return 1;
        if (v < key) lo = mid + 1;
        else hi = mid;
    }
    return 0;
}

// glibc-exact expf(y) for every non-NaN float y (the silu domain is
// [-10, +inf); the router's sqrt-softplus also takes y < -10, where results
// go subnormal and then zero).  `flip` lists (sorted) the inputs whose glibc result is the other
// neighbour of the nearby rounding midpoint.
WH_HD float wh_expf_glibc(float y, const uint64_t* exp2_tab, const uint32_t* flip, uint32_t nflip) {
    if (y > 89.0f) return wh_bits_to_float(0x7f800000u);
    if (y < -104.0f) return 0.0f;  // below half the least subnormal
    double d = wh_exp_double(y, exp2_tab);
    float f = (float)d;
    if (wh_expf_near_midpoint(d, f) && wh_table_contains(flip, nflip, wh_float_to_bits(y))) {
        uint32_t fb = wh_float_to_bits(f);
        double diff = d - (double)f;
        if ((fb & 0x7fffffffu) == 0x7f800000u) {
            f = wh_bits_to_float(0x7f7fffffu);  // inf -> FLT_MAX
        } else {
            f = wh_bits_to_float(diff > 0.0 ? fb + 1 : fb - 1);  // positive f: +1 bit = next up
        }
    }
    return f;
}

// silu exactly as the reference computes it in f32: x / (1 + expf(-x)).
WH_HD float wh_silu(float x, const uint64_t* exp2_tab, const uint32_t* flip, uint32_t nflip) {
    float e = wh_expf_glibc(-x, exp2_tab, flip, nflip);
    float den = 1.0f + e;
    return x / den;
}

// ceil(log2f(r)) for a positive normal float r, glibc-exact given the
// per-binade thresholds thr[e + 126] (e = unbiased exponent, -126..127).
WH_HD int wh_ceil_log2f(float r, const uint32_t* thr) {
    uint32_t b = wh_float_to_bits(r);
    int e = (int)((b >> 23) & 0xff) - 127;
    uint32_t m = b & 0x7fffff;
    if (m == 0) return e;
    return m > thr[e + 126] ? e + 1 : e;
}

// glibc-exact log1pf(x) for x >= 0 (Rust's f32::ln_1p): the float form of
// the published fdlibm log1p method (Sun Microsystems; s_log1pf.c as carried
// by FreeBSD msun and glibc's sysdeps/ieee754/flt-32), evaluated in float
// with every operation rounded on its own (no contraction), which host and
// device do alike.  With k and f such that 1+x = 2^k (1+f), sqrt(2)/2 <=
// 1+f < sqrt(2), and c the rounding error of 1+x:
//   log1p(x) = k ln2_hi + (f - (hfsq - (s (hfsq + R(s^2)) + (k ln2_lo + c))))
// where hfsq = f^2/2, s = f/(2+f) and R is a degree-7 polynomial in s^2 for
// log((1+s)/(1-s)) - 2s.  The generator compares it with the host glibc on
// every non-negative float.
WH_HD float wh_log1pf(float x) {
    const float ln2_hi = wh_bits_to_float(0x3f317180u), ln2_lo = wh_bits_to_float(0x3717f7d1u);
    const float lp1 = wh_bits_to_float(0x3f2aaaabu), lp2 = wh_bits_to_float(0x3ecccccdu),
                lp3 = wh_bits_to_float(0x3e924925u), lp4 = wh_bits_to_float(0x3e638e29u),
                lp5 = wh_bits_to_float(0x3e3a3325u), lp6 = wh_bits_to_float(0x3e1cd04fu),
                lp7 = wh_bits_to_float(0x3e178897u);
    const int32_t hx = (int32_t)wh_float_to_bits(x);
    const int32_t ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    float f = 0.0f, c = 0.0f;
    if (hx < 0x3ed413d7) {                         // x < 0.41422
        if (ax >= 0x3f800000) return wh_bits_to_float(0x7fc00000u);  // x <= -1: not on this path
        if (ax < 0x31000000) {                     // |x| < 2^-29
            if (ax < 0x24800000) return x;         // |x| < 2^-54
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { // -0.2929 < x < 0.41422
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;                              // +inf, NaN
    }
    if (k != 0) {
        float u;
        if (hx < 0x5a000000) {                     // 1+x is inexact below 2^53
            u = 1.0f + x;
            hu = (int32_t)wh_float_to_bits(u);
            k = (hu >> 23) - 127;
            c = k > 0 ? 1.0f - (u - x) : x - (u - 1.0f);
            c /= u;
        } else {
            u = x;
            hu = (int32_t)wh_float_to_bits(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {                       // mantissa below sqrt(2): u in [1, sqrt(2))
            u = wh_bits_to_float((uint32_t)hu | 0x3f800000u);
        } else {                                   // halve: u in [sqrt(2)/2, 1)
            k += 1;
            u = wh_bits_to_float((uint32_t)hu | 0x3f000000u);
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    const float kf = (float)k;
    if (hu == 0) {                                 // |f| < 2^-20
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += kf * ln2_lo;
            return kf * ln2_hi + c;
        }
        const float r = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - r;
        return kf * ln2_hi - ((r - (kf * ln2_lo + c)) - f);
    }
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float r = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + r));
    return kf * ln2_hi - ((hfsq - (s * (hfsq + r) + (kf * ln2_lo + c))) - f);
}

// 2^k as float for -126 <= k <= 127 (exp2f of an integral float is exact there).
WH_HD float wh_pow2f(int k) { return wh_bits_to_float((uint32_t)(k + 127) << 23); }

// Nearest E4M3 value to t in [-448, 448] (the act-quant grid, E/compute.rs:
// 2537-2545): ties go to the lower value (toward -inf) and a zero result is
// +0.  For |t| >= 2^-6 the grid has 3 mantissa bits at t's own exponent, so
// rounding is an integer add on the f32 bits: 0x7ffff below the dropped
// half for positive t (ties stay low), 0x80000 for negative t (ties move the
// magnitude up, i.e. toward -inf).  Below 2^-6 the grid is n * 2^-9: |t| *
// 2^33 as an integer holds every bit of |t| down to 2^-33 (all that can
// decide a rounding there), and the same integer add rounds it to a multiple
// of 2^24.  Both results are formed and one is selected, so a wave never
// diverges.  The generator checks this against a brute-force nearest over
// every float in [-448, 448].
WH_HD float wh_e4m3_round(float t) {
    const uint32_t b = wh_float_to_bits(t);
    const uint32_t s = b & 0x80000000u, a = b & 0x7fffffffu, up = s >> 31;
    const uint32_t normal = ((a + 0x7ffffu + up) & 0xfff00000u) | s;
    const float at = wh_bits_to_float(a < 0x3c800000u ? a : 0x3c800000u);  // min(|t|, 2^-6)
    const uint32_t u = (uint32_t)(at * 8589934592.0f);                        // * 2^33, < 2^28
    const uint32_t n = (u + 0x7fffffu + up) >> 24;
    const uint32_t sub = wh_float_to_bits((float)n * 0.001953125f) | (n ? s : 0u);
    return wh_bits_to_float(a >= 0x3c800000u ? normal : sub);
}
