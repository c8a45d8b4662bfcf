// Build-time generator for the glibc-exact libm tables used by the device
// code (see libm_emul.h).  It runs the exact same emulation code on the host
// and compares it with the host glibc over every float input of each domain:
//   expf : every non-NaN float; the few inputs where the restated method
//          still differs are listed with glibc's result (at most 4096)
//   log1pf: every non-negative float     (log1p(expf(v)) of the router)
//   log2f: every normal float            (ceil(log2f(r)) for r = amax / 448)
//   exp2f: every integral k in [-126, 127]
// and aborts if any other input disagrees, so a written table is a verified
// one.
//
// Usage: gen_libm_tables <out.inc>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "libm_emul.h"

static uint64_t g_tab[WH_EXP_TAB_LEN];

// The constants of glibc's expf method: 2^(i/32) from long double (then
// less i << 47, so that adding k << 47 scales by 2^(k/32)), 32/ln2, the
// rounding shift 1.5 * 2^52 and the published cubic, scaled for r in units
// of 1/32.
static void build_exp_constants(void) {
    for (int i = 0; i < 32; ++i)
        g_tab[i] = wh_double_to_bits((double)exp2l((long double)i / 32.0L)) - ((uint64_t)i << 47);
    const double n = 32.0;
    g_tab[32] = wh_double_to_bits(0x1.71547652b82fep+0 * n);
    g_tab[33] = wh_double_to_bits(0x1.8p+52);
    g_tab[34] = wh_double_to_bits(0x1.c6af84b912394p-5 / n / n / n);
    g_tab[35] = wh_double_to_bits(0x1.ebfce50fac4f3p-3 / n / n);
    g_tab[36] = wh_double_to_bits(0x1.62e42ff0c52d6p-1 / n);
}

enum { EXC_MAX = 4096 };

typedef struct {
    uint64_t lo, hi;  // float bit range [lo, hi)
    uint32_t exc[2 * EXC_MAX];
    size_t nexc;
    long over;
} exp_job;

static void* exp_scan(void* p) {
    exp_job* j = (exp_job*)p;
    for (uint64_t b = j->lo; b < j->hi; ++b) {
        const uint32_t u = (uint32_t)b;
        if ((u & 0x7fffffffu) > 0x7f800000u) continue;  // NaN
        const float y = wh_bits_to_float(u);
        const uint32_t g = wh_float_to_bits(expf(y));
        if (wh_float_to_bits(wh_expf_glibc(y, g_tab, NULL, 0)) == g) continue;
        if (j->nexc == EXC_MAX) {
            j->over++;
            continue;
        }
        j->exc[2 * j->nexc] = u;
        j->exc[2 * j->nexc + 1] = g;
        j->nexc++;
    }
    return NULL;
}

static int cmp_u32(const void* a, const void* b) {
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return (x > y) - (x < y);
}

typedef struct {
    uint64_t lo, hi;
    long bad;
} log1p_job;

static void* log1p_verify(void* p) {
    log1p_job* j = (log1p_job*)p;
    for (uint64_t b = j->lo; b < j->hi; ++b) {
        float x = wh_bits_to_float((uint32_t)b);
        if (wh_float_to_bits(wh_log1pf(x)) != wh_float_to_bits(log1pf(x))) {
            if (j->bad < 5) fprintf(stderr, "log1pf: mismatch x=%a glibc=%a emul=%a\n", x, log1pf(x), wh_log1pf(x));
            j->bad++;
        }
    }
    return NULL;
}

typedef struct {
    int e0, e1;
    const uint32_t* thr;
    long bad;
} log_job;

static void* log_verify(void* p) {
    log_job* j = (log_job*)p;
    for (int e = j->e0; e < j->e1; ++e) {
        for (uint32_t m = 0; m < (1u << 23); ++m) {
            uint32_t b = ((uint32_t)(e + 127) << 23) | m;
            float r = wh_bits_to_float(b);
            float want = ceilf(log2f(r));
            int got = wh_ceil_log2f(r, j->thr);
            if ((float)got != want) {
                if (j->bad < 5) fprintf(stderr, "log2f: mismatch r=%a glibc=%g emul=%d\n", r, want, got);
                j->bad++;
            }
        }
    }
    return NULL;
}

typedef struct {
    uint64_t lo, hi, step;
    long bad;
} sincos_job;

static void* sincos_verify(void* p) {
    sincos_job* j = (sincos_job*)p;
    for (uint64_t b = j->lo; b < j->hi; b += j->step) {
        const float y = wh_bits_to_float((uint32_t)b);
        if ((((uint32_t)b) & 0x7fffffffu) > 0x7f800000u) continue;  // NaN
        const uint32_t gs = wh_float_to_bits(sinf(y)), gc = wh_float_to_bits(cosf(y));
        if (wh_float_to_bits(wh_sincosf_glibc(y, 0)) != gs || wh_float_to_bits(wh_sincosf_glibc(y, 1)) != gc) {
            if (j->bad < 5)
                fprintf(stderr, "sinf/cosf: mismatch y=%a glibc=%a/%a emul=%a/%a\n", y, sinf(y), cosf(y),
                        wh_sincosf_glibc(y, 0), wh_sincosf_glibc(y, 1));
            j->bad++;
        }
    }
    return NULL;
}

// sinf and cosf: every float in [+0, 2^24) (every RoPE angle position x
// inverse frequency of a position below 2^24 with frequencies <= 1), and
// every 101st float of the rest (negative, large, inf).
static int check_sincos(void) {
    enum { T = 8 };
    sincos_job js[2 * T];
    pthread_t ts[2 * T];
    const uint64_t dense = 0x4b800000ull;  // 2^24
    for (int i = 0; i < T; ++i) {
        js[i].lo = dense * i / T;
        js[i].hi = dense * (i + 1) / T;
        js[i].step = 1;
        js[T + i].lo = dense + (0x100000000ull - dense) * i / T;
        js[T + i].hi = dense + (0x100000000ull - dense) * (i + 1) / T;
        js[T + i].step = 101;
        js[i].bad = js[T + i].bad = 0;
    }
    for (int i = 0; i < 2 * T; ++i) pthread_create(&ts[i], NULL, sincos_verify, &js[i]);
    long bad = 0;
    for (int i = 0; i < 2 * T; ++i) {
        pthread_join(ts[i], NULL);
        bad += js[i].bad;
    }
    if (bad) fprintf(stderr, "sinf/cosf: %ld mismatches\n", bad);
    else fprintf(stderr, "sinf/cosf: every float in [0, 2^24) and the sample of the rest match the host glibc\n");
    return bad != 0;
}

// wh_div448 against the float division for every float in [1e-4, FLT_MAX].
typedef struct {
    uint32_t b0, b1;
    long bad;
} div_job;
static void* div_verify(void* p) {
    div_job* j = (div_job*)p;
    for (uint32_t b = j->b0; b < j->b1; ++b) {
        const float a = wh_bits_to_float(b);
        const volatile float want = a / 448.0f;
        if (wh_float_to_bits(wh_div448(a)) != wh_float_to_bits(want) && j->bad++ < 5)
            fprintf(stderr, "div448 mismatch: a=%a got %a want %a\n", a, wh_div448(a), (float)want);
    }
    return NULL;
}
static int check_div448(void) {
    enum { T = 8 };
    div_job js[T];
    pthread_t ts[T];
    const uint32_t lo = wh_float_to_bits(1.0e-4f), hi = 0x7f800000u;  // [1e-4, FLT_MAX]
    for (int i = 0; i < T; ++i) {
        js[i].b0 = lo + (uint32_t)((uint64_t)(hi - lo) * i / T);
        js[i].b1 = lo + (uint32_t)((uint64_t)(hi - lo) * (i + 1) / T);
        js[i].bad = 0;
        pthread_create(&ts[i], NULL, div_verify, &js[i]);
    }
    long bad = 0;
    for (int i = 0; i < T; ++i) {
        pthread_join(ts[i], NULL);
        bad += js[i].bad;
    }
    if (bad) fprintf(stderr, "div448: %ld mismatches\n", bad);
    else fprintf(stderr, "div448: every float in [1e-4, FLT_MAX] matches the float division\n");
    return bad != 0;
}

// wh_e4m3_code_scaled(h, k) and wh_e4m3_code_pow2(h, k) against the code of wh_e4m3_round(h / 2^k) for
// t = h / 2^k over every float in [0, 448] (both signs; every 11th float
// for the other k), with h = t 2^k exactly representable.
typedef struct {
    uint32_t b0, b1;
    long bad;
} code_job;
static uint32_t e4m3_code_of(float q) {  // q on the E4M3 grid, |q| <= 448
    const uint32_t b = wh_float_to_bits(q), a = b & 0x7fffffffu;
    const uint32_t mag = a >= 0x3c800000u ? (a >> 20) - 960u : (uint32_t)(wh_bits_to_float(a) * 512.0f);
    return mag | ((b >> 31) << 7);
}
static void* code_verify(void* p) {
    code_job* j = (code_job*)p;
    static const int ks[5] = {-3, -23, -9, 0, 5};
    for (uint32_t b = j->b0; b < j->b1; ++b) {
        const float t = wh_bits_to_float(b);
        for (int ki = 0; ki < 5; ++ki) {
            if (ki > 0 && b % 11u) continue;
            const int k = ks[ki];
            const float h = t * wh_pow2f(k);
            if (h * wh_pow2f(-k) != t) continue;  // t 2^k not exact (underflow)
            for (int sg = 0; sg < 2; ++sg) {
                const float hs = sg ? -h : h, ts = sg ? -t : t;
                uint32_t want = e4m3_code_of(wh_e4m3_round(ts)), got = wh_e4m3_code_scaled(hs, k);
                if ((want & 0x7f) == 0 && (got & 0x7f) == 0) want = got;  // zero: either sign
                if (want != got && j->bad++ < 5)
                    fprintf(stderr, "e4m3 code mismatch: h=%a k=%d got %02x want %02x\n", hs, k, got, want);
                const uint32_t got2 = wh_e4m3_code_pow2(hs, k);
                if ((want & 0x7f) == 0 && (got2 & 0x7f) == 0) want = got2;
                if (want != got2 && j->bad++ < 5)
                    fprintf(stderr, "e4m3 pow2 code mismatch: h=%a k=%d got %02x want %02x\n", hs, k, got2, want);
            }
        }
    }
    return NULL;
}
static int check_e4m3_code_scaled(void) {
    enum { T = 8 };
    code_job js[T];
    pthread_t ts[T];
    const uint32_t end = 0x43e00001u;  // +0 .. 448
    for (int i = 0; i < T; ++i) {
        js[i].b0 = (uint32_t)((uint64_t)end * i / T);
        js[i].b1 = (uint32_t)((uint64_t)end * (i + 1) / T);
        js[i].bad = 0;
        pthread_create(&ts[i], NULL, code_verify, &js[i]);
    }
    long bad = 0;
    for (int i = 0; i < T; ++i) {
        pthread_join(ts[i], NULL);
        bad += js[i].bad;
    }
    if (bad) fprintf(stderr, "e4m3 code: %ld mismatches\n", bad);
    else fprintf(stderr, "e4m3 code: every scaled float matches wh_e4m3_round\n");
    return bad != 0;
}

// Every float t in [-448, 448] against the brute-force nearest E4M3 value
// (ties to the lower value, +0 for zero), walking the positive grid upward.
static int check_e4m3_round(void) {
    float grid[127];
    int n = 0;
    for (int code = 0; code < 0x7f; ++code) {  // +0 .. 448, ascending
        int e = (code >> 3) & 15, m = code & 7;
        grid[n++] = e == 0 ? (float)m * 0.001953125f : ldexpf(1.0f + (float)m / 8.0f, e - 7);
    }
    long bad = 0;
    int i = 0;
    for (uint32_t b = 0; b <= 0x43e00000u; ++b) {  // +0 .. 448
        float a = wh_bits_to_float(b);
        while (i + 1 < n && grid[i + 1] <= a) ++i;
        float lo = grid[i], hi = i + 1 < n ? grid[i + 1] : grid[i];
        float dlo = a - lo, dhi = hi - a;
        float pos = dhi < dlo ? hi : lo;   // positive t: ties to lo
        float neg = dlo < dhi ? lo : hi;   // negative t: ties to the larger magnitude
        float want_p = pos, want_n = neg == 0.0f ? 0.0f : -neg;
        float got_p = wh_e4m3_round(a), got_n = wh_e4m3_round(-a);
        if (wh_float_to_bits(got_p) != wh_float_to_bits(want_p) ||
            wh_float_to_bits(got_n) != wh_float_to_bits(want_n)) {
            if (bad++ < 5) fprintf(stderr, "e4m3 round mismatch at %a: %a/%a want %a/%a\n", a, got_p, got_n, want_p, want_n);
        }
    }
    if (bad) fprintf(stderr, "e4m3 round: %ld mismatches\n", bad);
    else fprintf(stderr, "e4m3 round: every float in [-448, 448] matches the brute-force nearest\n");
    return bad != 0;
}

int main(int argc, char** argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s out.inc\n", argv[0]);
        return 2;
    }
    enum { T = 8 };
    build_exp_constants();

    // expf over every float: the restated method, and the inputs where it
    // still differs from the host glibc
    static exp_job js[T];
    pthread_t ts[T];
    uint32_t* exc = NULL;
    size_t nexc = 0;
    long bad = 0;
    for (int i = 0; i < T; ++i) {
        js[i].lo = (0x100000000ull * i) / T;
        js[i].hi = (0x100000000ull * (i + 1)) / T;
        js[i].nexc = 0;
        js[i].over = 0;
        pthread_create(&ts[i], NULL, exp_scan, &js[i]);
    }
    for (int i = 0; i < T; ++i) {
        pthread_join(ts[i], NULL);
        bad += js[i].over;
        exc = (uint32_t*)realloc(exc, (nexc + js[i].nexc + 1) * 2 * sizeof(uint32_t));
        memcpy(exc + 2 * nexc, js[i].exc, js[i].nexc * 2 * sizeof(uint32_t));
        nexc += js[i].nexc;
    }
    if (bad || nexc > EXC_MAX) {
        fprintf(stderr, "expf: more than %d inputs differ from the host glibc\n", EXC_MAX);
        return 1;
    }
    // sort the (input, result) pairs by input (ranges above were ascending
    // in bit order per thread; the sign bit splits them, so sort anyway)
    for (size_t a = 1; a < nexc; ++a)
        for (size_t b2 = a; b2 > 0 && exc[2 * (b2 - 1)] > exc[2 * b2]; --b2) {
            uint32_t k = exc[2 * b2], v = exc[2 * b2 + 1];
            exc[2 * b2] = exc[2 * (b2 - 1)];
            exc[2 * b2 + 1] = exc[2 * (b2 - 1) + 1];
            exc[2 * (b2 - 1)] = k;
            exc[2 * (b2 - 1) + 1] = v;
        }
    // verify the table-driven function on every listed input and on a
    // stride sample of the rest (the scan above covered every input)
    for (size_t i = 0; i < nexc; ++i) {
        float y = wh_bits_to_float(exc[2 * i]);
        if (wh_float_to_bits(wh_expf_glibc(y, g_tab, exc, (uint32_t)nexc)) != wh_float_to_bits(expf(y))) {
            fprintf(stderr, "expf: verification failed at %a\n", y);
            return 1;
        }
    }
    for (uint64_t b = 0; b < 0x100000000ull; b += 997) {
        if (((uint32_t)b & 0x7fffffffu) > 0x7f800000u) continue;
        float y = wh_bits_to_float((uint32_t)b);
        if (wh_float_to_bits(wh_expf_glibc(y, g_tab, exc, (uint32_t)nexc)) != wh_float_to_bits(expf(y))) {
            fprintf(stderr, "expf: verification failed at %a\n", y);
            return 1;
        }
    }
    fprintf(stderr, "expf: every float matches the host glibc (%zu listed exceptions)\n", nexc);

    // log2f thresholds per binade: largest mantissa for which log2f(r) == e
    static uint32_t thr[254];
    for (int e = -126; e <= 127; ++e) {
        uint32_t t = 0;
        for (uint32_t m = 1; m < (1u << 23); ++m) {
            float r = wh_bits_to_float(((uint32_t)(e + 127) << 23) | m);
            if (log2f(r) == (float)e) t = m;
            else break;
        }
        thr[e + 126] = t;
    }
    {
        log_job js[T];
        pthread_t ts[T];
        for (int i = 0; i < T; ++i) {
            js[i].e0 = -126 + 254 * i / T;
            js[i].e1 = -126 + 254 * (i + 1) / T;
            js[i].thr = thr;
            js[i].bad = 0;
            pthread_create(&ts[i], NULL, log_verify, &js[i]);
        }
        for (int i = 0; i < T; ++i) {
            pthread_join(ts[i], NULL);
            bad += js[i].bad;
        }
    }
    if (bad) {
        fprintf(stderr, "log2f: %ld mismatches\n", bad);
        return 1;
    }
    for (int e = -126; e <= 127; ++e) {
        if (wh_log2f_thr(e) != thr[e + 126]) {
            fprintf(stderr, "log2f: closed-form threshold of binade %d is %u, the table's %u\n", e, wh_log2f_thr(e),
                    thr[e + 126]);
            return 1;
        }
    }
    for (int k = -126; k <= 127; ++k) {
        if (wh_float_to_bits(exp2f((float)k)) != wh_float_to_bits(wh_pow2f(k))) {
            fprintf(stderr, "exp2f(%d) is not 2^%d\n", k, k);
            return 1;
        }
    }

    if (check_e4m3_round()) return 1;
    if (check_e4m3_code_scaled()) return 1;
    if (check_div448()) return 1;
    if (check_sincos()) return 1;

    // log1pf over [+0, +inf]
    {
        log1p_job js[T];
        pthread_t ts[T];
        const uint64_t n = 0x7f800001ull;
        for (int i = 0; i < T; ++i) {
            js[i].lo = n * i / T;
            js[i].hi = n * (i + 1) / T;
            js[i].bad = 0;
            pthread_create(&ts[i], NULL, log1p_verify, &js[i]);
        }
        for (int i = 0; i < T; ++i) {
            pthread_join(ts[i], NULL);
            bad += js[i].bad;
        }
        if (bad) {
            fprintf(stderr, "log1pf: %ld mismatches\n", bad);
            return 1;
        }
        fprintf(stderr, "log1pf: every non-negative float matches the host glibc\n");
    }

    FILE* out = fopen(argv[1], "w");
    if (!out) {
        perror("open");
        return 1;
    }
    fprintf(out, "// Generated by gen_libm_tables.c from the host glibc; verified exhaustively.\n");
    fprintf(out, "#define WH_EXP_TAB_INIT \\\n");
    for (int j = 0; j < WH_EXP_TAB_LEN; ++j)
        fprintf(out, "  0x%016llxull%s\n", (unsigned long long)g_tab[j], j < WH_EXP_TAB_LEN - 1 ? ", \\" : "");
    fprintf(out, "#define WH_LOG2F_THR_INIT \\\n");
    for (int i = 0; i < 254; ++i) fprintf(out, "  %uu%s\n", thr[i], i < 253 ? ", \\" : "");
    fprintf(out, "#define WH_EXPF_EXC_COUNT %zuu\n", nexc);
    fprintf(out, "#define WH_EXPF_EXC_INIT");
    if (nexc == 0) fprintf(out, " 0u, 0u");  // placeholder pair, never read
    for (size_t i = 0; i < nexc; ++i) fprintf(out, "%s 0x%08xu, 0x%08xu", i ? "," : "", exc[2 * i], exc[2 * i + 1]);
    fprintf(out, "\n");
    fclose(out);
    fprintf(stderr, "libm tables: %zu expf exceptions, log2f thresholds written to %s\n", nexc, argv[1]);
    free(exc);
    return 0;
}
