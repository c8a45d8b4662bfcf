// glibc-exact float libm pieces used on the decode path, shared by the HIP
// device code and by the host-side table generator (gen_libm_tables.c).
//
// The reference engine calls the platform libm through Rust's f32 methods:
//   silu(x) = x / (1 + expf(-x))                 E/deepseek_v4.rs:551-554
//   act-quant block scale exp2f(ceilf(log2f(r)))  E/compute.rs:2514
//   router sqrt(log1pf(expf(v)))                  E/compute.rs:2238-2249
// glibc's expf and log1pf are not correctly rounded, so a correctly rounded
// device function would not match them.  Instead:
//   1. expf restates glibc's own method (the exp of ARM's optimized-routines
//      by Szabolcs Nagy, glibc's sysdeps/ieee754/flt-32/e_expf.c since 2.27):
//      x*32/ln2 = k + r, 2^(k/32) from a 32-entry table, a cubic in r, all
//      in IEEE double with each operation rounded on its own, which host and
//      device evaluate alike.  The generator compares it with the host
//      glibc on every float and lists the few inputs where the two still
//      differ (different contraction of the polynomial in the host build)
//      with glibc's result; the device checks that short sorted list.
//   2. log1pf restates fdlibm's float log1p (see wh_log1pf), which matches
//      glibc on every non-negative float.
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

// Layout of the expf table (doubles as bit patterns): entries 0..31 are
// asuint64(2^(i/32)) - (i << 47), then 32/ln2, 1.5 * 2^52 (the rounding
// shift) and the cubic's coefficients for r in units of 1/32 (c0 r^3 +
// c1 r^2 + c2 r + 1).
#define WH_EXP_TAB_LEN 37

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

// glibc's expf(x) for every float x.  `exc` holds n_exc (input bits, glibc
// result bits) pairs sorted by input: the inputs where this restatement and
// the host glibc differ.
WH_HD float wh_expf_glibc(float x, const uint64_t* tab, const uint32_t* exc, uint32_t n_exc) {
    const uint32_t ux = wh_float_to_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                                 // |x| >= 88 (top 12 bits of 88.0f)
        if (ux == 0xff800000u) return 0.0f;                // -inf
        if (abstop >= 0x7f8) return x + x;                 // +inf, NaN
        if (x > wh_bits_to_float(0x42b17217u)) return wh_bits_to_float(0x7f800000u);  // > log(2^128)
        if (x < wh_bits_to_float(0xc2cff1b4u)) return 0.0f;                            // < log(2^-150)
    }
    const double xd = (double)x;
    const double z = wh_bits_to_double(tab[32]) * xd;
    double kd = z + wh_bits_to_double(tab[33]);            // round to the nearest integer
    const uint64_t ki = wh_double_to_bits(kd);
    kd -= wh_bits_to_double(tab[33]);
    const double r = z - kd;
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = wh_bits_to_double(t);                 // 2^(k/32)
    const double zz = wh_bits_to_double(tab[34]) * r + wh_bits_to_double(tab[35]);
    const double r2 = r * r;
    double y = wh_bits_to_double(tab[36]) * r + 1.0;
    y = zz * r2 + y;
    y = y * s;
    float f = (float)y;
    if (n_exc <= 32) {
        // a short list: uniform loads the compiler keeps in scalar registers
        for (uint32_t i = 0; i < n_exc; ++i)
            if (exc[2 * i] == ux) return wh_bits_to_float(exc[2 * i + 1]);
    } else {
        uint32_t lo = 0, hi = n_exc;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            const uint32_t k = exc[2 * mid];
            if (k == ux) return wh_bits_to_float(exc[2 * mid + 1]);
            if (k < ux) lo = mid + 1;
            else hi = mid;
        }
    }
    return f;
}

// silu exactly as the reference computes it in f32: x / (1 + expf(-x)).
WH_HD float wh_silu(float x, const uint64_t* exp_tab, const uint32_t* exc, uint32_t n_exc) {
    float e = wh_expf_glibc(-x, exp_tab, exc, n_exc);
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

// The same thresholds in closed form.  log2f(2^e (1 + m 2^-23)) is e plus
// about 1.44 m 2^-23, and it rounds back to e while that is under half an
// ulp of the result; the result's binade is that of |e| for e >= 0 and of
// |e| - 1 for e < 0 (the result lies just above e), so the threshold
// depends only on the bit length of e >= 0 ? e : -e - 1 (0..7):
// {0, 0, 0, 1, 2, 5, 11, 22}.  The table generator checks this against the
// table it derives from the host glibc, binade by binade, and fails the
// build on any difference.
WH_HD uint32_t wh_log2f_thr(int e) {
    const uint32_t u = (uint32_t)(e ^ (e >> 31));  // e >= 0 ? e : -e - 1
    uint32_t bl = 0;
    while ((u >> bl) != 0u) ++bl;
    return (uint32_t)((0x160B050201000000ull >> (8 * bl)) & 0xffu);
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

// glibc-exact sinf / cosf (Rust's f32::sin / f32::cos, which f32::sin_cos
// calls one after the other; the RoPE angle of E/compute.rs:2623-2649).
// This restates glibc's method (the sinf/cosf of ARM's optimized-routines by
// Szabolcs Nagy, glibc's sysdeps/ieee754/flt-32/s_sinf.c, s_cosf.c and
// s_sincosf.h since 2.28): the float argument is reduced in IEEE double to
// r in [-pi/4, pi/4] and a quadrant n, then
//   sin(r) ~ (r + s1 r^3) + r^5 (s2 + s3 r^2),
//   cos(r) ~ ((c0 + c1 r^2) + c2 r^4) + r^6 (c3 + c4 r^2),
// with the published minimax coefficients in IEEE double, then rounded to
// float once.  On CPUs with FMA (every AVX2 machine the reference runs on)
// glibc selects a build of these functions compiled with FMA contraction, so
// every a + b*c form below (the reduction x - n pi/2 included) is one fused
// multiply-add, as there; products stand alone.  Reduction: |x| < 120 multiplies by
// 2/pi in double (n = nearest integer, r = x - n pi/2); larger |x| takes the
// exact fixed-point product of the 24-bit mantissa with a 96-bit window of
// the bits of 2/pi (an integer Payne-Hanek step) to a 2.62 fixed-point
// fraction.  Odd quadrants swap the two polynomials; quadrants 2 and 3
// negate them.  The generator compares both with the host glibc on every
// float in [0, 2^24) and a stride sample of all other floats.
#define WH_SC_HPI_INV 0x1.45F306DC9C883p+23  /* 2/pi * 2^24 */
#define WH_SC_HPI 0x1.921FB54442D18p0        /* pi/2 */
#define WH_SC_PI63 0x1.921FB54442D18p-62     /* pi/2 * 2^-61: one unit of the 2.62 fraction */

// Bits [start, start + 32) of the fraction of 2/pi (zero before bit 0),
// from its first 224 bits.
WH_HD uint32_t wh_two_over_pi_bits(int start) {
    const uint32_t w[7] = {0xA2F9836Eu, 0x4E441529u, 0xFC2757D1u, 0xF534DDC0u,
                           0xDB629599u, 0x3C439041u, 0xFE5163ABu};
    if (start <= -32) return 0u;
    if (start < 0) return w[0] >> (uint32_t)(-start);
    const int i = start >> 5, s = start & 31;
    return s == 0 ? w[i] : (w[i] << s) | (w[i + 1] >> (32 - s));
}

// The two polynomials for reduced r (x2 = r^2): odd n gives the cosine one.
// neg = 1 negates the coefficients (quadrants 2 and 3).
WH_HD float wh_sincos_poly(double x, double x2, int n, int neg) {
    const double sg = neg ? -1.0 : 1.0;
    if ((n & 1) == 0) {
        const double s1c = -0x1.555545995a603p-3, s2c = 0x1.1107605230bc4p-7, s3c = -0x1.994eb3774cf24p-13;
        const double x3 = x * x2;
        const double s1 = __builtin_fma(x2, s3c, s2c);
        const double x7 = x3 * x2;
        const double s = __builtin_fma(x3, s1c, x);
        return (float)__builtin_fma(x7, s1, s);
    }
    const double c0 = sg * 0x1p0, c1 = sg * -0x1.ffffffd0c621cp-2, c2 = sg * 0x1.55553e1068f19p-5,
                 c3 = sg * -0x1.6c087e89a359dp-10, c4 = sg * 0x1.99343027bf8c3p-16;
    const double x4 = x2 * x2;
    const double c2p = __builtin_fma(x2, c4, c3);
    const double c1p = __builtin_fma(x2, c1, c0);
    const double x6 = x4 * x2;
    const double c = __builtin_fma(x4, c2, c1p);
    return (float)__builtin_fma(x6, c2p, c);
}

// Large-argument reduction (|x| >= 120, finite): r in double and the
// quadrant n (mod 4) of the float with bits xi (sign ignored).
WH_HD double wh_sincos_reduce_large(uint32_t xi, int* np) {
    const int i0 = (int)((xi >> 26) & 15), shift = (int)((xi >> 23) & 7);
    const uint32_t a0 = wh_two_over_pi_bits(8 * i0 - 24), a4 = wh_two_over_pi_bits(8 * i0 + 8),
                   a8 = wh_two_over_pi_bits(8 * i0 + 40);
    uint32_t m = ((xi & 0xffffffu) | 0x800000u) << shift;
    uint64_t res0 = (uint64_t)(uint32_t)(m * a0);
    const uint64_t res1 = (uint64_t)m * a4, res2 = (uint64_t)m * a8;
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    const uint64_t n = (res0 + (1ull << 61)) >> 62;
    res0 -= n << 62;
    *np = (int)n;
    return (double)(int64_t)res0 * WH_SC_PI63;
}

// cosine = 0: sinf(y); cosine = 1: cosf(y).
WH_HD float wh_sincosf_glibc(float y, int cosine) {
    const uint32_t top = (wh_float_to_bits(y) >> 20) & 0x7ff;
    double x = (double)y;
    int n;
    if (top < 0x3f4) {                                   // |y| < pi/4
        if (top < 0x398) return cosine ? 1.0f : y;        // |y| < 2^-12
        return wh_sincos_poly(x, x * x, cosine, 0);
    }
    if (top < 0x42f) {                                   // |y| < 120
        const double r = x * WH_SC_HPI_INV;
        n = ((int32_t)r + 0x800000) >> 24;
        x = __builtin_fma(-(double)n, WH_SC_HPI, x);
        const double s = ((n + 1) & 2) ? -1.0 : 1.0;     // quadrant signs 1, -1, -1, 1
        return wh_sincos_poly(x * s, x * x, n ^ cosine, (n & 2) != 0);
    }
    if (top < 0x7f8) {                                   // finite
        const uint32_t xi = wh_float_to_bits(y);
        const int sign = (int)(xi >> 31);
        x = wh_sincos_reduce_large(xi, &n);
        const int q = n + sign;
        const double s = ((q + 1) & 2) ? -1.0 : 1.0;
        return wh_sincos_poly(x * s, x * x, n ^ cosine, (q & 2) != 0);
    }
    return y - y;                                        // inf, NaN
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

// The E4M3 code of t = h / 2^k under the act-quant rounding (nearest, ties
// toward -inf, E/compute.rs:2537-2545), from h's own bits, for |t| <= 448.
// For |t| >= 2^-6 the grid keeps 3 mantissa bits and dividing by 2^k only
// moves the exponent, so the rounded magnitude is ((|h| bits + 0x7ffff +
// sign) >> 20) - (960 + 8 k): wh_e4m3_round's integer rounding, shifted.
// Below 2^-6 the grid is n 2^-9 and wh_e4m3_round's second branch applies.
// A zero result keeps the sign (0x80 for -0; the MFMA takes it as 0).  The
// table generator compares it with wh_e4m3_round for every float h with
// |h / 2^k| <= 448 at several k.
WH_HD uint32_t wh_e4m3_code_scaled(float h, int k) {
    const uint32_t b = wh_float_to_bits(h), a = b & 0x7fffffffu, sg = b >> 31;
    uint32_t mag = ((a + 0x7ffffu + sg) >> 20) - (uint32_t)(960 + 8 * k);
    if (a < ((uint32_t)(121 + k) << 23)) {
        float at = wh_bits_to_float(a) * wh_pow2f(-k);  // |h / 2^k|, exact
        at = at < 0.015625f ? at : 0.015625f;
        mag = ((uint32_t)(at * 8589934592.0f) + 0x7fffffu + sg) >> 24;
    }
    return (mag < 0x7eu ? mag : 0x7eu) | (sg << 7);  // (the clamp only ever meets non-finite h)
}

// The same code as the token kernels form it, for finite v with
// |v / 2^k| <= 448 (no clamp): the normal-range magnitude ((|v| bits +
// 0x7ffff + sign) >> 20) - (960 + 8 k), folded into one add; below 2^-6 the
// grid is n 2^-9 with n = (|v| 2^(33 - k) + 0x7fffff + sign) >> 24 (the
// power-of-two scaling is exact, |v| 2^(33 - k) < 2^27 there).  The table
// generator compares it with wh_e4m3_round for every float t = v / 2^k in
// [-448, 448] at several k.
WH_HD uint32_t wh_e4m3_code_pow2(float v, int k) {
    const uint32_t b = wh_float_to_bits(v), a = b & 0x7fffffffu, sg = b >> 31;
    const uint32_t K = 0x7ffffu - ((uint32_t)(960 + 8 * k) << 20), lim = (uint32_t)(121 + k) << 23;
    const uint32_t nrm = (a + K + sg) >> 20;
    float at = wh_bits_to_float(a) * wh_pow2f(33 - k);
    at = at < 134217728.0f ? at : 134217728.0f;
    const uint32_t sub = ((uint32_t)at + 0x7fffffu + sg) >> 24;
    return (a < lim ? sub : nrm) | (sg << 7);
}

// a / 448.0f, correctly rounded, for finite a >= 1e-4 (the act-quant's
// amax / 448, E/compute.rs:2511-2514) without a float division: a / 7 is
// never a midpoint between two floats (a 24-bit a would need 27 significant
// bits), its distance to the nearest one is at least 2^-27.8 of its value,
// and the double product a * (1 / 7) is within 2^-52 of it, so rounding
// that product to float gives a / 7 correctly rounded; dividing by 64 is
// exact above 1e-4 / 448.  The table generator compares it with the float
// division for every float in [1e-4, FLT_MAX].
WH_HD float wh_div448(float a) { return (float)((double)a * (1.0 / 7.0)) * 0.015625f; }

#ifdef __HIPCC__
// Device form: the bit length from the count of leading zeros.
__device__ __forceinline__ uint32_t wh_log2f_thr_dev(int e) {
    const uint32_t u = (uint32_t)(e ^ (e >> 31));
    const uint32_t bl = 32u - (uint32_t)__clz((int)u);
    return __builtin_amdgcn_perm(0x160B0502u, 0x01000000u, bl) & 0xffu;
}
// ceil(log2f(max(amax, 1e-4) / 448)): the act-quant scale exponent
// (E/compute.rs:2511-2514) without the threshold table.
__device__ __forceinline__ int wh_aq_scale_exp_fast(float amax) {
    const float r = wh_div448(fmaxf(amax, 1.0e-4f));
    const uint32_t b = wh_float_to_bits(r);
    const int e = (int)((b >> 23) & 0xff) - 127;
    const uint32_t m = b & 0x7fffff;
    return m > wh_log2f_thr_dev(e) ? e + 1 : e;  // (m > threshold implies m != 0)
}
#endif
