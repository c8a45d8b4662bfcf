// Build-time generator for the glibc-exact libm tables used by the device
// code (see libm_emul.h).  It runs the exact same emulation code on the host
// and compares it with the host glibc over every float input of each domain:
//   expf : every non-NaN float (silu's argument after min(g, 10) lies in
//          [-10, +inf); the router's sqrt-softplus takes any value <= 20)
//   log1pf: every non-negative float     (log1p(expf(v)) of the router)
//   log2f: every normal float            (ceil(log2f(r)) for r = amax / 448)
//   exp2f: every integral k in [-126, 127]
// and aborts if any input disagrees, so a written table is a verified one.
//
// Usage: gen_libm_tables <out.inc>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "libm_emul.h"

static uint64_t g_tab[35];

static void build_exp_constants(void) {
    for (int j = 0; j < 32; ++j) g_tab[j] = wh_double_to_bits((double)exp2l((long double)j / 32.0L));
    long double ln2 = logl(2.0L);
    g_tab[32] = wh_double_to_bits((double)(32.0L / ln2));
    long double l = ln2 / 32.0L;
    // head: l rounded to 32 significant bits, so n * head is exact for |n| < 2^21
    int ex;
    long double m = frexpl(l, &ex);
    long double head = ldexpl(roundl(ldexpl(m, 32)), ex - 32);
    g_tab[33] = wh_double_to_bits((double)head);
    g_tab[34] = wh_double_to_bits((double)(l - head));
}

typedef struct {
    uint64_t lo, hi;  // float bit range [lo, hi)
    uint32_t* flips;
    size_t nflips, cap;
    long bad;
} exp_job;

static void* exp_scan(void* p) {
    exp_job* j = (exp_job*)p;
    for (uint64_t b = j->lo; b < j->hi; ++b) {
        float y = wh_bits_to_float((uint32_t)b);
        float g = expf(y);
        float f;
        double d = 0.0;
        if (y > 89.0f) {
            f = wh_bits_to_float(0x7f800000u);
        } else if (y < -104.0f) {
            f = 0.0f;
        } else {
            d = wh_exp_double(y, g_tab);
            f = (float)d;
        }
        if (wh_float_to_bits(g) == wh_float_to_bits(f)) continue;
        // a mismatch must be a flip across a nearby midpoint
        uint32_t fb = wh_float_to_bits(f);
        double diff = d - (double)f;
        uint32_t want;
        if ((fb & 0x7fffffffu) == 0x7f800000u) want = 0x7f7fffffu;
        else want = diff > 0.0 ? fb + 1 : fb - 1;
        if (y > 89.0f || y < -104.0f || !wh_expf_near_midpoint(d, f) || want != wh_float_to_bits(g)) {
            if (j->bad < 5)
                fprintf(stderr, "expf: unrepresentable mismatch y=%a glibc=%a emul=%a d=%a\n", y, g, f, d);
            j->bad++;
            continue;
        }
        if (j->nflips == j->cap) {
            j->cap = j->cap ? j->cap * 2 : 4096;
            j->flips = (uint32_t*)realloc(j->flips, j->cap * sizeof(uint32_t));
        }
        j->flips[j->nflips++] = (uint32_t)b;
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

    // expf over [-inf, -0] and [+0, +inf]
    uint64_t ranges[2][2] = {{0x80000000ull, 0xff800001ull}, {0x00000000ull, 0x7f800001ull}};
    uint32_t* flips = NULL;
    size_t nflips = 0;
    long bad = 0;
    for (int r = 0; r < 2; ++r) {
        exp_job js[T];
        pthread_t ts[T];
        uint64_t lo = ranges[r][0], n = ranges[r][1] - ranges[r][0];
        for (int i = 0; i < T; ++i) {
            memset(&js[i], 0, sizeof js[i]);
            js[i].lo = lo + n * i / T;
            js[i].hi = lo + n * (i + 1) / T;
            pthread_create(&ts[i], NULL, exp_scan, &js[i]);
        }
        for (int i = 0; i < T; ++i) {
            pthread_join(ts[i], NULL);
            bad += js[i].bad;
            flips = (uint32_t*)realloc(flips, (nflips + js[i].nflips + 1) * sizeof(uint32_t));
            memcpy(flips + nflips, js[i].flips, js[i].nflips * sizeof(uint32_t));
            nflips += js[i].nflips;
            free(js[i].flips);
        }
    }
    if (bad) {
        fprintf(stderr, "expf: %ld inputs not representable by the flip scheme\n", bad);
        return 1;
    }
    qsort(flips, nflips, sizeof(uint32_t), cmp_u32);
    // re-check the table-driven function on every flipped input and on a
    // stride sample of the rest (the scan above already covered every input)
    for (size_t i = 0; i < nflips; ++i) {
        float y = wh_bits_to_float(flips[i]);
        if (wh_float_to_bits(wh_expf_glibc(y, g_tab, flips, (uint32_t)nflips)) != wh_float_to_bits(expf(y))) {
            fprintf(stderr, "expf: verification failed at %a\n", y);
            return 1;
        }
    }
    for (int r = 0; r < 2; ++r) {
        for (uint64_t b = ranges[r][0]; b < ranges[r][1]; b += 997) {
            float y = wh_bits_to_float((uint32_t)b);
            if (wh_float_to_bits(wh_expf_glibc(y, g_tab, flips, (uint32_t)nflips)) != wh_float_to_bits(expf(y))) {
                fprintf(stderr, "expf: verification failed at %a\n", y);
                return 1;
            }
        }
    }

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
    for (int k = -126; k <= 127; ++k) {
        if (wh_float_to_bits(exp2f((float)k)) != wh_float_to_bits(wh_pow2f(k))) {
            fprintf(stderr, "exp2f(%d) is not 2^%d\n", k, k);
            return 1;
        }
    }

    if (check_e4m3_round()) return 1;

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
    fprintf(out, "#define WH_EXP2_TAB_INIT \\\n");
    for (int j = 0; j < 35; ++j) fprintf(out, "  0x%016llxull%s\n", (unsigned long long)g_tab[j], j < 34 ? ", \\" : "");
    fprintf(out, "#define WH_LOG2F_THR_INIT \\\n");
    for (int i = 0; i < 254; ++i) fprintf(out, "  %uu%s\n", thr[i], i < 253 ? ", \\" : "");
    fprintf(out, "#define WH_EXPF_FLIP_COUNT %zuu\n", nflips);
    fprintf(out, "#define WH_EXPF_FLIP_INIT \\\n");
    for (size_t i = 0; i < nflips; ++i) {
        fprintf(out, "0x%08xu%s", flips[i], i + 1 < nflips ? "," : "");
        if (i % 12 == 11 && i + 1 < nflips) fprintf(out, " \\\n");
    }
    fprintf(out, "\n");
    fclose(out);
    fprintf(stderr, "libm tables: %zu expf flips, log2f thresholds written to %s\n", nflips, argv[1]);
    free(flips);
    return 0;
}
