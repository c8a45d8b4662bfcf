/*
 * CPU oracle for the DeepSeek-V4 decode hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C with the same x86 AVX2/FMA intrinsics, the
 * reference engine's CPU kernels for the FP8 block-scaled GEMV, the FP4
 * E2M1 x UE8M0 matvec, the activation quant-dequant (QAT simulation), the
 * SwiGLU expert forward and the routed-expert weighted sum.  Only the test
 * suite, the smoke check and the CPU-baseline leg of the benchmark may load
 * it: it is the checker, never the product.  The product path lives in
 * wohper_amd/csrc and fails loudly without the HIP library.
 *
 * Reference: Twenytwo/wohper, engine/zc_infer_core/src/ (cited as E/...).
 * Arithmetic rules followed exactly:
 *   - scalar Rust `a * b + c` is two roundings (built with -ffp-contract=off);
 *   - AVX2 `_mm256_fmadd_ps` is fused, as in the reference intrinsics;
 *   - libm calls (expf, log2f, exp2f) go to the host glibc, as Rust's f32
 *     methods do on Linux.
 *
 * Pinning (see tests/test_oracle_*.py): codecs against closed forms over all
 * codes and against torch's float8_e4m3fn decode; row kernels against float64
 * dots, against the reference's inline known answers and against each other
 * (AVX2 vs per-element paths); act-quant against brute-force nearest search
 * over the 256-entry E4M3 grid.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* Error codes: same numbering as the product ABI (include/wohper_hip.h),
 * mirroring DeepSeekV4KernelError E/deepseek_v4.rs:398-408. */
enum {
    OR_OK = 0,
    OR_EMPTY_SHAPE = 1,
    OR_INVALID_SHAPE = 2,
    OR_PACKED_WEIGHT_TOO_SMALL = 3,
    OR_SCALE_TOO_SMALL = 4,
    OR_INPUT_TOO_SMALL = 5,
    OR_OUTPUT_TOO_SMALL = 6,
    OR_SCRATCH_TOO_SMALL = 7,
    OR_NON_FINITE_OUTPUT = 8,
};

/* ------------------------------------------------------------------ codecs */

/* E/deepseek_v4.rs:151-164 */
float or_decode_fp8_e4m3(uint8_t byte, float scale) {
    float sign = (byte & 0x80) ? -1.0f : 1.0f;
    int exponent = (byte >> 3) & 0x0f;
    int mantissa = byte & 0x07;
    if (exponent == 0 && mantissa == 0) return 0.0f;
    float value;
    if (exponent == 0) {
        value = ((float)mantissa / 8.0f) * ldexpf(1.0f, -6);
    } else {
        value = (1.0f + (float)mantissa / 8.0f) * ldexpf(1.0f, exponent - 7);
    }
    return sign * value * scale;
}

/* E/deepseek_v4.rs:166-172 */
float or_decode_ue8m0_scale(uint8_t byte) {
    if (byte == 0) return 0.0f;
    return ldexpf(1.0f, (int)byte - 127); /* 2f32.powi: 255 -> +inf */
}

/* E/deepseek_v4.rs:358-372 */
float or_decode_fp4_e2m1(uint8_t nibble, float scale) {
    nibble &= 0x0f;
    float sign = (nibble & 0x08) ? -1.0f : 1.0f;
    int exponent = (nibble >> 1) & 0x03;
    int mantissa = nibble & 0x01;
    if (exponent == 0 && mantissa == 0) return 0.0f;
    float value;
    if (exponent == 0) {
        value = ((float)mantissa / 2.0f) * ldexpf(1.0f, -2);
    } else {
        value = (1.0f + (float)mantissa / 2.0f) * ldexpf(1.0f, exponent - 1);
    }
    return sign * value * scale;
}

static float g_fp8_lut[256];
static float g_ue8m0_lut[256];
static float g_fp4_lut[16];
static float g_fp8_sorted[256];
static pthread_once_t g_lut_once = PTHREAD_ONCE_INIT;

static int cmp_total_f32(const void* a, const void* b) {
    /* f32::total_cmp: order by the sign-magnitude-flipped bit pattern */
    int32_t x, y;
    memcpy(&x, a, 4);
    memcpy(&y, b, 4);
    x ^= (int32_t)(((uint32_t)(x >> 31)) >> 1);
    y ^= (int32_t)(((uint32_t)(y >> 31)) >> 1);
    return (x > y) - (x < y);
}

static void init_luts(void) {
    for (int b = 0; b < 256; ++b) {
        g_fp8_lut[b] = or_decode_fp8_e4m3((uint8_t)b, 1.0f);   /* E/deepseek_v4.rs:195-204 */
        g_ue8m0_lut[b] = or_decode_ue8m0_scale((uint8_t)b);    /* E/deepseek_v4.rs:183-192 */
        g_fp8_sorted[b] = g_fp8_lut[b];
    }
    for (int n = 0; n < 16; ++n) g_fp4_lut[n] = or_decode_fp4_e2m1((uint8_t)n, 1.0f);
    qsort(g_fp8_sorted, 256, sizeof(float), cmp_total_f32);   /* E/compute.rs:2524-2535 */
}

static void ensure_luts(void) { pthread_once(&g_lut_once, init_luts); }

void or_luts(float* fp8_out256, float* ue8m0_out256, float* fp4_out16, float* sorted_out256) {
    ensure_luts();
    if (fp8_out256) memcpy(fp8_out256, g_fp8_lut, sizeof g_fp8_lut);
    if (ue8m0_out256) memcpy(ue8m0_out256, g_ue8m0_lut, sizeof g_ue8m0_lut);
    if (fp4_out16) memcpy(fp4_out16, g_fp4_lut, sizeof g_fp4_lut);
    if (sorted_out256) memcpy(sorted_out256, g_fp8_sorted, sizeof g_fp8_sorted);
}

/* ------------------------------------------------------- row parallelism */

/* E/deepseek_v4.rs:209-221: ZC_COMPUTE_THREADS override, else nproc - 2. */
static int g_threads_override = 0;
void or_set_threads(int n) { g_threads_override = n; }
int or_thread_count(void) {
    if (g_threads_override > 0) return g_threads_override;
    const char* env = getenv("ZC_COMPUTE_THREADS");
    if (env && *env) {
        int v = atoi(env);
        return v < 1 ? 1 : v;
    }
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    n -= 2;
    return n < 1 ? 1 : (int)n;
}

typedef int (*row_work_fn)(void* ctx, size_t row_offset, float* chunk, size_t rows);

typedef struct {
    row_work_fn fn;
    void* ctx;
    size_t offset;
    float* chunk;
    size_t rows;
    int result;
} row_job;

static void* row_job_main(void* p) {
    row_job* j = (row_job*)p;
    j->result = j->fn(j->ctx, j->offset, j->chunk, j->rows);
    return NULL;
}

/* E/deepseek_v4.rs:227-262: per-call thread fan-out over contiguous chunks;
 * the first error (by chunk order here, by completion in the reference)
 * wins. Results are per row, so the split never changes values. */
static int parallel_rows(float* output, size_t n, size_t min_rows, row_work_fn fn, void* ctx) {
    int threads = or_thread_count();
    if (min_rows < 1) min_rows = 1;
    if (threads <= 1 || n < min_rows * 2) return fn(ctx, 0, output, n);
    size_t chunk = (n + (size_t)threads - 1) / (size_t)threads;
    if (chunk < min_rows) chunk = min_rows;
    size_t jobs = (n + chunk - 1) / chunk;
    row_job* js = (row_job*)calloc(jobs, sizeof(row_job));
    pthread_t* ts = (pthread_t*)calloc(jobs, sizeof(pthread_t));
    size_t off = 0;
    for (size_t j = 0; j < jobs; ++j) {
        size_t take = n - off < chunk ? n - off : chunk;
        js[j] = (row_job){fn, ctx, off, output + off, take, 0};
        pthread_create(&ts[j], NULL, row_job_main, &js[j]);
        off += take;
    }
    int err = OR_OK;
    for (size_t j = 0; j < jobs; ++j) {
        pthread_join(ts[j], NULL);
        if (err == OR_OK && js[j].result != OR_OK) err = js[j].result;
    }
    free(js);
    free(ts);
    return err;
}

/* parallel_rows over n rows of `group` floats each (the work function gets
 * its rows' slice of the output) */
static int parallel_rows_grouped(float* output, size_t n, size_t group, size_t min_rows, row_work_fn fn,
                                 void* ctx) {
    int threads = or_thread_count();
    if (min_rows < 1) min_rows = 1;
    if (threads <= 1 || n < min_rows * 2) return fn(ctx, 0, output, n);
    size_t chunk = (n + (size_t)threads - 1) / (size_t)threads;
    if (chunk < min_rows) chunk = min_rows;
    size_t jobs = (n + chunk - 1) / chunk;
    row_job* js = (row_job*)calloc(jobs, sizeof(row_job));
    pthread_t* ts = (pthread_t*)calloc(jobs, sizeof(pthread_t));
    size_t off = 0;
    for (size_t j = 0; j < jobs; ++j) {
        size_t take = n - off < chunk ? n - off : chunk;
        js[j] = (row_job){fn, ctx, off, output + off * group, take, 0};
        pthread_create(&ts[j], NULL, row_job_main, &js[j]);
        off += take;
    }
    int err = OR_OK;
    for (size_t j = 0; j < jobs; ++j) {
        pthread_join(ts[j], NULL);
        if (err == OR_OK && js[j].result != OR_OK) err = js[j].result;
    }
    free(js);
    free(ts);
    return err;
}

/* ------------------------------------------------------------ FP8 rows */

/* E/compute.rs:5967-5973 */
static inline float hsum256(__m256 v) {
    float l[8];
    _mm256_storeu_ps(l, v);
    return ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
}

/* E/compute.rs:5978-6018 (simd_x86::fp8_ue8m0_dot_row_avx2).  `scales` are
 * the already-decoded group scales of this row (scale_lut[byte] in the
 * reference; an fp32 block scale is consumed identically). */
__attribute__((target("avx2,fma")))
float or_fp8_dot_row_avx2(const uint8_t* weight_row, const float* scales, size_t groups,
                          size_t col_group, const float* input) {
    ensure_luts();
    __m256 acc = _mm256_setzero_ps();
    float tail = 0.0f;
    for (size_t g = 0; g < groups; ++g) {
        float scale = scales[g];
        const uint8_t* bytes = weight_row + g * col_group;
        const float* cols = input + g * col_group;
        __m256 g0 = _mm256_setzero_ps();
        __m256 g1 = _mm256_setzero_ps();
        size_t chunks = col_group / 16;
        for (size_t c = 0; c < chunks; ++c) {
            size_t base = c * 16;
            __m256i idx0 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(bytes + base)));
            __m256i idx1 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(bytes + base + 8)));
            __m256 w0 = _mm256_i32gather_ps(g_fp8_lut, idx0, 4);
            __m256 w1 = _mm256_i32gather_ps(g_fp8_lut, idx1, 4);
            g0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(cols + base), g0);
            g1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(cols + base + 8), g1);
        }
        float rem = 0.0f;
        for (size_t i = chunks * 16; i < col_group; ++i) rem += g_fp8_lut[bytes[i]] * cols[i];
        acc = _mm256_fmadd_ps(_mm256_add_ps(g0, g1), _mm256_set1_ps(scale), acc);
        tail += rem * scale;
    }
    return hsum256(acc) + tail;
}

/* E/compute.rs:5937-5960 (non-AVX2 fallback: four unfused accumulators) */
float or_fp8_dot_row_scalar(const uint8_t* weight_row, const float* scales, size_t groups,
                            size_t col_group, const float* input) {
    ensure_luts();
    float acc = 0.0f;
    for (size_t g = 0; g < groups; ++g) {
        float scale = scales[g];
        const uint8_t* bytes = weight_row + g * col_group;
        const float* cols = input + g * col_group;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        size_t quads = col_group / 4;
        for (size_t q = 0; q < quads; ++q) {
            size_t i = q * 4;
            s0 += g_fp8_lut[bytes[i]] * cols[i];
            s1 += g_fp8_lut[bytes[i + 1]] * cols[i + 1];
            s2 += g_fp8_lut[bytes[i + 2]] * cols[i + 2];
            s3 += g_fp8_lut[bytes[i + 3]] * cols[i + 3];
        }
        for (size_t i = quads * 4; i < col_group; ++i) s0 += g_fp8_lut[bytes[i]] * cols[i];
        acc += scale * ((s0 + s1) + (s2 + s3));
    }
    return acc;
}

typedef struct {
    const uint8_t* weight;
    const float* scales; /* decoded, [scale_rows x scale_cols] */
    size_t rows, cols, scale_cols, row_group, col_group, row_start;
    const float* input;
    int use_avx2;
} fp8_gemv_ctx;

static int fp8_gemv_work(void* p, size_t row_offset, float* chunk, size_t n) {
    fp8_gemv_ctx* c = (fp8_gemv_ctx*)p;
    for (size_t i = 0; i < n; ++i) {
        size_t row = c->row_start + row_offset + i;
        const float* srow = c->scales + (row / c->row_group) * c->scale_cols;
        float acc = c->use_avx2
                        ? or_fp8_dot_row_avx2(c->weight + row * c->cols, srow, c->scale_cols,
                                              c->col_group, c->input)
                        : or_fp8_dot_row_scalar(c->weight + row * c->cols, srow, c->scale_cols,
                                                c->col_group, c->input);
        if (!isfinite(acc)) return OR_NON_FINITE_OUTPUT;
        chunk[i] = acc;
    }
    return OR_OK;
}

/* E/compute.rs:6174-6239 (tensorwise) and 6244-6321 (rows).  Scales are
 * given decoded: fp32 per 128x128 block, or UE8M0 bytes decoded by the
 * caller through or_decode_ue8m0_scale.  row_end == 0 means all rows. */
int or_fp8_gemv(const uint8_t* weight, size_t rows, size_t cols, const float* scales,
                size_t scale_rows, size_t scale_cols, size_t row_start, size_t row_end,
                const float* input, float* output, int use_avx2) {
    if (row_end == 0) row_end = rows;
    if (rows == 0 || cols == 0 || scale_rows == 0 || scale_cols == 0 || rows % scale_rows ||
        cols % scale_cols)
        return OR_INVALID_SHAPE;
    if (row_start >= row_end || row_end > rows) return OR_INVALID_SHAPE;
    fp8_gemv_ctx c = {weight, scales, rows, cols, scale_cols, rows / scale_rows,
                      cols / scale_cols, row_start, input, use_avx2};
    return parallel_rows(output, row_end - row_start, 32, fp8_gemv_work, &c);
}

/* E/compute.rs:6384-6577 (gemv_fp8_e4m3_ue8m0_rows_multi): every row's
 * bytes decoded to f32 once (fp8_ue8m0_dot_row_avx2_store_dequant), then each
 * input's dot on the decoded row in the single-input kernel's order
 * (fp8_ue8m0_dot_dequant_row_avx2): the same groups, g0/g1 chains and
 * acc = fma(g0 + g1, scale, acc) as or_fp8_dot_row_avx2 with plain loads
 * in place of the gathers. */
__attribute__((target("avx2,fma")))
static float fp8_dot_dequant_row_avx2(const float* dequant, const float* scales, size_t groups, size_t col_group,
                                      const float* input) {
    __m256 acc = _mm256_setzero_ps();
    float tail = 0.0f;
    for (size_t g = 0; g < groups; ++g) {
        float scale = scales[g];
        const float* w = dequant + g * col_group;
        const float* cols = input + g * col_group;
        __m256 g0 = _mm256_setzero_ps();
        __m256 g1 = _mm256_setzero_ps();
        size_t chunks = col_group / 16;
        for (size_t c = 0; c < chunks; ++c) {
            size_t base = c * 16;
            g0 = _mm256_fmadd_ps(_mm256_loadu_ps(w + base), _mm256_loadu_ps(cols + base), g0);
            g1 = _mm256_fmadd_ps(_mm256_loadu_ps(w + base + 8), _mm256_loadu_ps(cols + base + 8), g1);
        }
        float rem = 0.0f;
        for (size_t i = chunks * 16; i < col_group; ++i) rem += w[i] * cols[i];
        acc = _mm256_fmadd_ps(_mm256_add_ps(g0, g1), _mm256_set1_ps(scale), acc);
        tail += rem * scale;
    }
    return hsum256(acc) + tail;
}

typedef struct {
    const uint8_t* weight;
    const float* scales;
    size_t cols, scale_cols, row_group, col_group, row_start;
    const float* inputs;
    size_t count, in_stride;
} fp8_multi_ctx;

/* rows of the flat [rows][count] result, one decoded row at a time */
static int fp8_multi_work(void* p, size_t row_offset, float* chunk, size_t n) {
    fp8_multi_ctx* c = (fp8_multi_ctx*)p;
    float* dequant = (float*)malloc(c->cols * sizeof(float));
    if (!dequant) return OR_INVALID_SHAPE;
    int err = OR_OK;
    for (size_t i = 0; i < n && err == OR_OK; ++i) {
        size_t row = c->row_start + row_offset + i;
        const uint8_t* bytes = c->weight + row * c->cols;
        for (size_t k = 0; k < c->cols; ++k) dequant[k] = g_fp8_lut[bytes[k]];
        const float* srow = c->scales + (row / c->row_group) * c->scale_cols;
        for (size_t j = 0; j < c->count; ++j) {
            float acc = fp8_dot_dequant_row_avx2(dequant, srow, c->scale_cols, c->col_group,
                                                 c->inputs + j * c->in_stride);
            if (!isfinite(acc)) {
                err = OR_NON_FINITE_OUTPUT;
                break;
            }
            chunk[i * c->count + j] = acc;
        }
    }
    free(dequant);
    return err;
}

/* outputs[j * out_stride + (row - row_start)] for input j at
 * inputs + j * in_stride (scales decoded, as or_fp8_gemv). */
int or_fp8_gemv_rows_multi(const uint8_t* weight, size_t rows, size_t cols, const float* scales,
                           size_t scale_rows, size_t scale_cols, size_t row_start, size_t row_end,
                           const float* inputs, size_t count, size_t in_stride, float* outputs,
                           size_t out_stride) {
    ensure_luts();
    if (rows == 0 || cols == 0 || scale_rows == 0 || scale_cols == 0 || rows % scale_rows ||
        cols % scale_cols || count == 0)
        return OR_INVALID_SHAPE;
    if (row_start >= row_end || row_end > rows) return OR_INVALID_SHAPE;
    size_t n = row_end - row_start;
    /* the flat [rows][count] array parallel_rows fills: count floats per
     * row, so it is run over n * count "rows" of one float grouped by row */
    float* flat = (float*)malloc(n * count * sizeof(float));
    if (!flat) return OR_INVALID_SHAPE;
    fp8_multi_ctx c = {weight, scales, cols, scale_cols, rows / scale_rows, cols / scale_cols, row_start,
                       inputs, count, in_stride};
    int err = parallel_rows_grouped(flat, n, count, 8, fp8_multi_work, &c);
    if (err == OR_OK)
        for (size_t j = 0; j < count; ++j)
            for (size_t r = 0; r < n; ++r) outputs[j * out_stride + r] = flat[r * count + j];
    free(flat);
    return err;
}

/* ------------------------------------------------------------ FP4 rows */

/* E/deepseek_v4.rs:285-287 */
static const int8_t FP4_BASE_X8_I8[16] = {0, 1, 8, 12, 16, 24, 32, 48,
                                          0, -1, -8, -12, -16, -24, -32, -48};

/* E/deepseek_v4.rs:294-347 (fp4_avx2::dot_row) */
__attribute__((target("avx2,fma")))
float or_fp4_dot_row_avx2(const uint8_t* weight_row, const uint8_t* scale_row, size_t scale_cols,
                          size_t group_bytes, size_t group_cols, const float* input) {
    ensure_luts();
    __m128i lut = _mm_loadu_si128((const __m128i*)FP4_BASE_X8_I8);
    __m128i low_mask = _mm_set1_epi8(0x0f);
    __m256 acc = _mm256_setzero_ps();
    float tail = 0.0f;
    for (size_t g = 0; g < scale_cols; ++g) {
        float scale = g_ue8m0_lut[scale_row[g]];
        const uint8_t* bytes = weight_row + g * group_bytes;
        const float* cols = input + g * group_cols;
        size_t chunks = group_bytes / 16;
        __m256 gacc = _mm256_setzero_ps();
        for (size_t c = 0; c < chunks; ++c) {
            __m128i w = _mm_loadu_si128((const __m128i*)(bytes + c * 16));
            __m128i lo = _mm_and_si128(w, low_mask);
            __m128i hi = _mm_and_si128(_mm_srli_epi16(w, 4), low_mask);
            __m128i vlo = _mm_shuffle_epi8(lut, lo);
            __m128i vhi = _mm_shuffle_epi8(lut, hi);
            __m128i il = _mm_unpacklo_epi8(vlo, vhi);
            __m128i ih = _mm_unpackhi_epi8(vlo, vhi);
            const float* base = cols + c * 32;
            __m256 c0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(il));
            __m256 c1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(il, 8)));
            __m256 c2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(ih));
            __m256 c3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(ih, 8)));
            gacc = _mm256_fmadd_ps(c0, _mm256_loadu_ps(base), gacc);
            gacc = _mm256_fmadd_ps(c1, _mm256_loadu_ps(base + 8), gacc);
            gacc = _mm256_fmadd_ps(c2, _mm256_loadu_ps(base + 16), gacc);
            gacc = _mm256_fmadd_ps(c3, _mm256_loadu_ps(base + 24), gacc);
        }
        acc = _mm256_fmadd_ps(gacc, _mm256_set1_ps(scale * 0.125f), acc);
        float rem = 0.0f;
        for (size_t i = chunks * 16; i < group_bytes; ++i) {
            uint8_t b = bytes[i];
            rem += g_fp4_lut[b & 0x0f] * cols[2 * i];
            rem += g_fp4_lut[b >> 4] * cols[2 * i + 1];
        }
        tail += rem * scale;
    }
    return hsum256(acc) + tail;
}

/* E/deepseek_v4.rs:509-530: group-hoisted scalar fallback (no AVX2) */
float or_fp4_dot_row_grouped(const uint8_t* weight_row, const uint8_t* scale_row, size_t scale_cols,
                             size_t group_bytes, size_t group_cols, const float* input) {
    ensure_luts();
    float acc = 0.0f;
    for (size_t g = 0; g < scale_cols; ++g) {
        float scale = g_ue8m0_lut[scale_row[g]];
        const uint8_t* bytes = weight_row + g * group_bytes;
        const float* cols = input + g * group_cols;
        float low = 0.0f, high = 0.0f;
        for (size_t i = 0; i < group_bytes; ++i) {
            low += g_fp4_lut[bytes[i] & 0x0f] * cols[2 * i];
            high += g_fp4_lut[bytes[i] >> 4] * cols[2 * i + 1];
        }
        acc += scale * (low + high);
    }
    return acc;
}

/* E/deepseek_v4.rs:533-547: per-element path (odd shapes) */
float or_fp4_dot_row_elementwise(const uint8_t* weight_row, const uint8_t* scale_row, size_t cols,
                                 size_t group_cols, const float* input) {
    float acc = 0.0f;
    for (size_t col = 0; col < cols; ++col) {
        uint8_t packed = weight_row[col / 2];
        uint8_t nibble = (col & 1) == 0 ? (packed & 0x0f) : (packed >> 4);
        float scale = or_decode_ue8m0_scale(scale_row[col / group_cols]);
        acc += or_decode_fp4_e2m1(nibble, scale) * input[col];
    }
    return acc;
}

typedef struct {
    const uint8_t* packed;
    const uint8_t* scales;
    size_t rows, cols, scale_cols, row_bytes, group_cols;
    const float* input;
    int path; /* 0 avx2, 1 grouped scalar, 2 elementwise */
} fp4_ctx;

static int fp4_work(void* p, size_t row_offset, float* chunk, size_t n) {
    fp4_ctx* c = (fp4_ctx*)p;
    for (size_t i = 0; i < n; ++i) {
        size_t row = row_offset + i;
        const uint8_t* wrow = c->packed + row * c->row_bytes;
        const uint8_t* srow = c->scales + row * c->scale_cols;
        float acc;
        if (c->path == 0)
            acc = or_fp4_dot_row_avx2(wrow, srow, c->scale_cols, c->group_cols / 2, c->group_cols,
                                      c->input);
        else if (c->path == 1)
            acc = or_fp4_dot_row_grouped(wrow, srow, c->scale_cols, c->group_cols / 2,
                                         c->group_cols, c->input);
        else
            acc = or_fp4_dot_row_elementwise(wrow, srow, c->cols, c->group_cols, c->input);
        if (!isfinite(acc)) return OR_NON_FINITE_OUTPUT;
        chunk[i] = acc;
    }
    return OR_OK;
}

/* E/deepseek_v4.rs:434-462 */
int or_fp4_validate(size_t packed_len, size_t scales_len, size_t rows, size_t cols,
                    size_t scale_cols, size_t input_len, size_t output_len) {
    if (rows == 0 || cols == 0 || scale_cols == 0) return OR_EMPTY_SHAPE;
    if (input_len < cols) return OR_INPUT_TOO_SMALL;
    if (output_len < rows) return OR_OUTPUT_TOO_SMALL;
    if (cols % scale_cols != 0) return OR_INVALID_SHAPE;
    if (packed_len < rows * ((cols + 1) / 2)) return OR_PACKED_WEIGHT_TOO_SMALL;
    if (scales_len < rows * scale_cols) return OR_SCALE_TOO_SMALL;
    return OR_OK;
}

/* E/deepseek_v4.rs:464-549 (fp4_e2m1_ue8m0_matvec_scalar).  force_path:
 * -1 = the reference's own dispatch on an AVX2+FMA host, else 0/1/2. */
int or_fp4_matvec(const uint8_t* packed, size_t packed_len, const uint8_t* scales,
                  size_t scales_len, size_t rows, size_t cols, size_t scale_cols,
                  const float* input, size_t input_len, float* output, size_t output_len,
                  int force_path) {
    int err = or_fp4_validate(packed_len, scales_len, rows, cols, scale_cols, input_len, output_len);
    if (err) return err;
    size_t group_cols = cols / scale_cols;
    int path;
    if (cols % 2 == 0 && group_cols % 2 == 0)
        path = force_path < 0 ? 0 : force_path;
    else
        path = 2;
    fp4_ctx c = {packed, scales, rows, cols, scale_cols, (cols + 1) / 2, group_cols, input, path};
    if (path == 0) return parallel_rows(output, rows, 64, fp4_work, &c);
    return fp4_work(&c, 0, output, rows);
}

/* ------------------------------------------------------- act quant-dequant */

/* E/compute.rs:2537-2545: nearest entry of the sorted E4M3 LUT, ties to the
 * lower entry (partition_point + saturating neighbours). */
static float nearest_in_sorted_lut(float target) {
    size_t lo = 0, hi = 256;
    while (lo < hi) { /* partition_point(|v| v < target) */
        size_t mid = (lo + hi) / 2;
        if (g_fp8_sorted[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    size_t idx = lo; /* 0..256 */
    float lower = g_fp8_sorted[idx == 0 ? 0 : idx - 1];
    float upper = g_fp8_sorted[idx > 255 ? 255 : idx];
    if (fabsf(upper - target) < fabsf(lower - target)) return upper;
    return lower;
}

float or_nearest_e4m3(float target) {
    ensure_luts();
    return nearest_in_sorted_lut(target);
}

/* f32::clamp(-448, 448): NaN stays NaN */
static inline float clamp448(float v) {
    if (v < -448.0f) return -448.0f;
    if (v > 448.0f) return 448.0f;
    return v;
}

/* E/compute.rs:2504-2521 */
void or_act_quant_dequant(float* values, size_t n, size_t block_size) {
    if (block_size == 0 || n == 0) return;
    ensure_luts();
    for (size_t start = 0; start < n; start += block_size) {
        size_t end = start + block_size < n ? start + block_size : n;
        float amax = 0.0f;
        for (size_t i = start; i < end; ++i) amax = fmaxf(amax, fabsf(values[i]));
        amax = fmaxf(amax, 1.0e-4f);
        float scale = exp2f(ceilf(log2f(amax / 448.0f)));
        for (size_t i = start; i < end; ++i) {
            float scaled = clamp448(values[i] / scale);
            values[i] = nearest_in_sorted_lut(scaled) * scale;
        }
    }
}

/* The block scale alone, as computed above (exposed for pinning). */
float or_act_quant_scale(float amax) {
    amax = fmaxf(amax, 1.0e-4f);
    return exp2f(ceilf(log2f(amax / 448.0f)));
}

/* ----------------------------------------------------------- expert forward */

/* E/deepseek_v4.rs:551-554 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

#define SWIGLU_LIMIT 10.0f /* E/deepseek_v4.rs:559 */

/* one gate/up pair -> hidden, E/deepseek_v4.rs:590-594 */
float or_swiglu(float g, float u) {
    float gated = fminf(g, SWIGLU_LIMIT);
    float upped = u;
    if (upped < -SWIGLU_LIMIT) upped = -SWIGLU_LIMIT;
    if (upped > SWIGLU_LIMIT) upped = SWIGLU_LIMIT;
    return or_silu(gated) * upped;
}

typedef struct {
    const uint8_t* packed;
    size_t packed_len;
    const uint8_t* scales;
    size_t scales_len;
    size_t rows, cols, scale_cols;
} or_fp4_spec;

/* E/deepseek_v4.rs:561-601 (deepseek_v4_fp4_expert_forward_scalar) */
int or_fp4_expert_forward(const or_fp4_spec* w1, const or_fp4_spec* w3, const or_fp4_spec* w2,
                          const float* input, size_t input_len, float* output, size_t output_len,
                          float* scratch, size_t scratch_len, int force_path) {
    if (w1->cols != input_len || w3->cols != input_len || w1->rows != w3->rows ||
        w2->cols != w1->rows)
        return OR_INVALID_SHAPE;
    if (output_len < w2->rows) return OR_OUTPUT_TOO_SMALL;
    if (scratch_len < w1->rows * 2) return OR_SCRATCH_TOO_SMALL;
    float* gate = scratch;
    float* up = scratch + w1->rows;
    float* input_q = (float*)malloc(sizeof(float) * (w1->cols ? w1->cols : 1));
    memcpy(input_q, input, sizeof(float) * w1->cols);
    or_act_quant_dequant(input_q, w1->cols, 64);
    int err = or_fp4_matvec(w1->packed, w1->packed_len, w1->scales, w1->scales_len, w1->rows,
                            w1->cols, w1->scale_cols, input_q, w1->cols, gate, w1->rows,
                            force_path);
    if (!err)
        err = or_fp4_matvec(w3->packed, w3->packed_len, w3->scales, w3->scales_len, w3->rows,
                            w3->cols, w3->scale_cols, input_q, w3->cols, up, w3->rows, force_path);
    free(input_q);
    if (err) return err;
    for (size_t i = 0; i < w1->rows; ++i) gate[i] = or_swiglu(gate[i], up[i]);
    or_act_quant_dequant(gate, w1->rows, 64);
    err = or_fp4_matvec(w2->packed, w2->packed_len, w2->scales, w2->scales_len, w2->rows, w2->cols,
                        w2->scale_cols, gate, w1->rows, output, output_len, force_path);
    if (err) return err;
    for (size_t i = 0; i < w2->rows; ++i)
        if (!isfinite(output[i])) return OR_NON_FINITE_OUTPUT;
    return OR_OK;
}

/* -------------------------------------------------- routed expert reduction */

/* E/compute.rs:2014-2030 (valid_route_weight_sum): returns 1 and the sum if
 * every weight is finite and >= 0 and the sum exceeds f32::EPSILON. */
int or_route_weight_sum(const float* weights, size_t n, float* sum_out) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float w = weights[i];
        if (!(isfinite(w) && w >= 0.0f)) return 0;
        sum = sum + w;
    }
    if (sum <= 1.1920929e-07f) return 0;
    *sum_out = sum;
    return 1;
}

/* E/compute.rs:1948-2012 (compute_active_experts), with each expert's output
 * already computed in expert order: outs[e*hidden + i].  Single expert: no
 * weight applied.  Otherwise acc[i] += y[i] * (w_e / sum) (two roundings). */
void or_routed_combine(const float* outs, const float* weights, size_t n_experts, size_t hidden,
                       float* out) {
    if (n_experts == 0) return;
    if (n_experts == 1) {
        memcpy(out, outs, hidden * sizeof(float));
        return;
    }
    float sum = 0.0f;
    int valid = or_route_weight_sum(weights, n_experts, &sum);
    float uniform = 1.0f / (float)n_experts;
    for (size_t i = 0; i < hidden; ++i) out[i] = 0.0f;
    for (size_t e = 0; e < n_experts; ++e) {
        float w = valid ? weights[e] / sum : uniform;
        const float* y = outs + e * hidden;
        for (size_t i = 0; i < hidden; ++i) {
            float prod = y[i] * w;
            out[i] = out[i] + prod;
        }
    }
}

/* E/compute.rs:1779-1810 (accumulate_expert_for_positions), one expert:
 * acc[p] += y[p] * weight for each (position, weight) target, in order. */
void or_accumulate_expert(const float* y_per_target, const size_t* positions, const float* weights,
                          size_t n_targets, size_t hidden, float* routed_acc) {
    for (size_t t = 0; t < n_targets; ++t) {
        float* acc = routed_acc + positions[t] * hidden;
        const float* y = y_per_target + t * hidden;
        for (size_t i = 0; i < hidden; ++i) {
            float prod = y[i] * weights[t];
            acc[i] = acc[i] + prod;
        }
    }
}

/* E/server/generation.rs:2491-2503 (the batch union's per-position weights):
 * sum = sequential f32 sum of the scores; when the sum is finite and > 0
 * and every score is finite, w_k = score_k / sum, else 1 / topk.  Unlike
 * valid_route_weight_sum, negative scores and sums below f32::EPSILON pass. */
void or_batch_route_weights(const float* scores, size_t npos, size_t topk, float* weights) {
    for (size_t p = 0; p < npos; ++p) {
        const float* s = scores + p * topk;
        float sum = 0.0f;
        int finite = 1;
        for (size_t k = 0; k < topk; ++k) {
            sum = sum + s[k];
            finite = finite && isfinite(s[k]);
        }
        finite = finite && isfinite(sum) && sum > 0.0f;
        float uniform = 1.0f / (float)topk;
        for (size_t k = 0; k < topk; ++k) weights[p * topk + k] = finite ? s[k] / sum : uniform;
    }
}

/* ----------------------------------------------------------- FP8 shared FFN */

/* E/compute.rs:5545-5614 (compute_deepseek_fp8_shared_expert_into_hidden):
 * act-quant(x,64); g = W1 x; u = W3 x; h = swiglu; act-quant(h,64); y = W2 h.
 * Scales decoded by the caller (UE8M0 bytes or fp32 block scales). */
int or_fp8_shared_expert(const uint8_t* w1, const float* s1, const uint8_t* w3, const float* s3,
                         const uint8_t* w2, const float* s2, size_t hidden, size_t inter,
                         size_t s1_rows, size_t s1_cols, size_t s2_rows, size_t s2_cols,
                         const float* input, float* output) {
    float* xq = (float*)malloc(sizeof(float) * hidden);
    float* gate = (float*)malloc(sizeof(float) * inter);
    float* up = (float*)malloc(sizeof(float) * inter);
    memcpy(xq, input, sizeof(float) * hidden);
    or_act_quant_dequant(xq, hidden, 64);
    int err = or_fp8_gemv(w1, inter, hidden, s1, s1_rows, s1_cols, 0, 0, xq, gate, 1);
    if (!err) err = or_fp8_gemv(w3, inter, hidden, s3, s1_rows, s1_cols, 0, 0, xq, up, 1);
    if (!err) {
        for (size_t i = 0; i < inter; ++i) gate[i] = or_swiglu(gate[i], up[i]);
        or_act_quant_dequant(gate, inter, 64);
        err = or_fp8_gemv(w2, hidden, inter, s2, s2_rows, s2_cols, 0, 0, gate, output, 1);
    }
    free(xq);
    free(gate);
    free(up);
    return err;
}

/* ------------------------------------------------------- array helpers */

/* Element-wise glibc silu / expf, for exhaustive-style device checks. */
void or_swiglu_array(const float* g, const float* u, float* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = or_swiglu(g[i], u[i]);
}

void or_silu_array(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = or_silu(x[i]);
}

void or_expf_array(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

void or_act_quant_scale_array(const float* amax, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_act_quant_scale(amax[i]);
}

/* ------------------------------------------------------------------ router */

enum { OR_ROUTER_RAW_LOGITS = 0, OR_ROUTER_SQRT_SOFTPLUS = 1 };

static inline float bf16_value(uint16_t raw) {
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)raw << 16;
    return v.f;
}

/* dot_bf16_row on x86 = dot_bf16_row_avx2 (E/compute.rs:2910-2919,
 * 6116-6136): two 8-lane fused accumulators over 16-column chunks, hsum256
 * of their sum, then an unfused sequential tail. */
float or_bf16_dot_row_avx2(const uint16_t* row, const float* x, size_t cols) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    const size_t chunks = cols / 16;
    for (size_t c = 0; c < chunks; ++c) {
        const __m128i r0 = _mm_loadu_si128((const __m128i*)(row + 16 * c));
        const __m128i r1 = _mm_loadu_si128((const __m128i*)(row + 16 * c + 8));
        const __m256 w0 = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(r0), 16));
        const __m256 w1 = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(r1), 16));
        acc0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x + 16 * c), acc0);
        acc1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x + 16 * c + 8), acc1);
    }
    float tail = 0.0f;
    for (size_t i = chunks * 16; i < cols; ++i) tail += bf16_value(row[i]) * x[i];
    return hsum256(_mm256_add_ps(acc0, acc1)) + tail;
}

/* gemv_bf16_tensorwise (E/compute.rs:6139-6172): one dot per row. */
void or_bf16_gemv(const uint16_t* w, size_t rows, size_t cols, const float* x, float* y) {
    for (size_t r = 0; r < rows; ++r) y[r] = or_bf16_dot_row_avx2(w + r * cols, x, cols);
}

/* sqrt_softplus, E/compute.rs:2239-2249 (Rust f32::exp / ln_1p are libm
 * expf / log1pf; max(NaN, 0) is 0; sqrt is the IEEE square root). */
float or_sqrt_softplus(float v) {
    float sp;
    if (v > 20.0f) sp = v;
    else if (v < -20.0f) sp = expf(v);
    else sp = log1pf(expf(v));
    return sqrtf(fmaxf(sp, 0.0f));
}

void or_sqrt_softplus_array(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = or_sqrt_softplus(x[i]);
}

void or_log1pf_array(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = log1pf(x[i]);
}

/* f32::total_cmp as a signed integer key. */
static inline int32_t total_key(float f) {
    union { uint32_t u; float f; } v;
    v.f = f;
    int32_t k = (int32_t)v.u;
    return k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1);
}

/* finalize_route_weights, E/compute.rs:2254-2268. */
static void finalize_routes(float* scores, size_t n, int math, float route_scale) {
    if (math != OR_ROUTER_SQRT_SOFTPLUS || n == 0) return;
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) sum += scores[i];
    if (sum > 0.0f && isfinite(sum)) {
        for (size_t i = 0; i < n; ++i) scores[i] = scores[i] / sum * route_scale;
    } else {
        const float uniform = route_scale / (float)n;
        for (size_t i = 0; i < n; ++i) scores[i] = uniform;
    }
}

/* route_experts_from_dense_block after its gate GEMV (E/compute.rs:2129-2237):
 * `logits` are the gate rows' outputs.  sqrt-softplus for the DeepSeek math;
 * with `hash_ids` (the token's tid2eid row) the experts are those ids that
 * are available, in table order; otherwise the available experts sorted
 * (stable) by score + bias, descending in total_cmp order.  Truncated to
 * `active`, then finalized.  Available ids at or past `rows` have no score
 * and are dropped. */
int or_route_select(const float* logits, size_t rows, const float* bias, const uint32_t* available, size_t n_avail,
                    size_t active, int math, float route_scale, const uint32_t* hash_ids, size_t n_hash,
                    uint32_t* out_ids, float* out_scores, size_t* n_out) {
    *n_out = 0;
    if (active == 0 || n_avail == 0) return OR_OK;
    float* scores = (float*)malloc((rows ? rows : 1) * sizeof(float));
    for (size_t i = 0; i < rows; ++i)
        scores[i] = math == OR_ROUTER_SQRT_SOFTPLUS ? or_sqrt_softplus(logits[i]) : logits[i];
    size_t n = 0;
    if (hash_ids) {
        for (size_t h = 0; h < n_hash && n < active; ++h) {
            const uint32_t id = hash_ids[h];
            int avail = 0;
            for (size_t a = 0; a < n_avail; ++a) avail |= available[a] == id;
            if (!avail || id >= rows) continue;
            out_ids[n] = id;
            out_scores[n] = scores[id];
            ++n;
        }
    } else {
        /* stable insertion sort of (key, id, score) by key, descending */
        int32_t* keys = (int32_t*)malloc(n_avail * sizeof(int32_t));
        uint32_t* ids = (uint32_t*)malloc(n_avail * sizeof(uint32_t));
        size_t m = 0;
        for (size_t a = 0; a < n_avail; ++a) {
            const uint32_t id = available[a];
            if (id >= rows) continue;
            const float sel = (math == OR_ROUTER_SQRT_SOFTPLUS && bias) ? scores[id] + bias[id] : scores[id];
            const int32_t k = total_key(sel);
            size_t j = m;
            while (j > 0 && keys[j - 1] < k) {
                keys[j] = keys[j - 1];
                ids[j] = ids[j - 1];
                --j;
            }
            keys[j] = k;
            ids[j] = id;
            ++m;
        }
        for (n = 0; n < m && n < active; ++n) {
            out_ids[n] = ids[n];
            out_scores[n] = scores[ids[n]];
        }
        free(keys);
        free(ids);
    }
    free(scores);
    finalize_routes(out_scores, n, math, route_scale);
    *n_out = n;
    return OR_OK;
}

/* ---------------------------------------------------------------- MLA glue */

/* rms_norm_in_place (E/compute.rs:7110-7122) when w is NULL, else
 * apply_weighted_rms_norm (E/compute.rs:3077-3107) with bf16 weights:
 * the squares summed in order (Iterator::sum), mean_square = s / n,
 * inv_rms = 1 / sqrt(mean_square + 1e-6), out = x * inv_rms (* w). */
void or_rms_norm(const float* x, size_t n, const uint16_t* w, float* out) {
    if (n == 0) return;
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
    const float ms = s / (float)n;
    const float inv = 1.0f / sqrtf(ms + 1.0e-6f);
    for (size_t i = 0; i < n; ++i) out[i] = w ? x[i] * inv * bf16_value(w[i]) : x[i] * inv;
}

/* rope_inv_freqs (E/compute.rs:2591-2620): theta^(-(2i)/dim) per pair, then
 * with YaRN the linear ramp between the beta_fast / beta_slow correction
 * dims blends freq / factor and freq. */
void or_rope_inv_freqs(size_t rope_dim, float theta, int yarn, float factor, float beta_fast, float beta_slow,
                       size_t original_seq_len, float* out) {
    const size_t pairs = rope_dim / 2;
    for (size_t p = 0; p < pairs; ++p) out[p] = powf(theta, -(float)(2 * p) / (float)rope_dim);
    if (!yarn || original_seq_len == 0) return;
    const float dim = (float)rope_dim;
    const float base_ln = logf(theta);
    const float pi = 3.14159265358979323846f;
    const float cf = dim * logf((float)original_seq_len / (beta_fast * 2.0f * pi)) / (2.0f * base_ln);
    const float cs = dim * logf((float)original_seq_len / (beta_slow * 2.0f * pi)) / (2.0f * base_ln);
    const float low = fmaxf(floorf(cf), 0.0f);
    float high = fminf(ceilf(cs), dim - 1.0f);
    if (fabsf(low - high) < 1.1920929e-7f) high = low + 0.001f;
    for (size_t p = 0; p < pairs; ++p) {
        float ramp = ((float)p - low) / (high - low);
        if (ramp < 0.0f) ramp = 0.0f;
        else if (ramp > 1.0f) ramp = 1.0f;
        const float smooth = 1.0f - ramp;
        out[p] = out[p] / factor * (1.0f - smooth) + out[p] * smooth;
    }
}

/* apply_rope_interleaved_with_freqs (E/compute.rs:2623-2649): pair i of
 * values rotated by position * inv[i] (f32 sin / cos of the host libm). */
void or_rope_apply(float* v, size_t position, const float* inv, size_t pairs, int inverse) {
    const float pos = (float)position;
    for (size_t p = 0; p < pairs; ++p) {
        const float ang = pos * inv[p];
        float s = sinf(ang);
        const float c = cosf(ang);
        if (inverse) s = -s;
        const float e = v[2 * p], o = v[2 * p + 1];
        v[2 * p] = e * c - o * s;
        v[2 * p + 1] = e * s + o * c;
    }
}

/* The window loop of compute_deepseek_v4_mla_attention (E/compute.rs:
 * 4106-4197) for every head: keys = the n_win window rows (stride win_ld)
 * then the n_comp compressed rows (head_dim apart). */
void or_window_attention(const float* q, size_t heads, size_t head_dim, size_t nope_dim, const float* win,
                         size_t n_win, size_t win_ld, const float* comp, size_t n_comp, const float* sink,
                         const float* inv, size_t pairs, size_t token_pos, float* out) {
    const size_t nk = n_win + n_comp;
    const float scale = powf((float)head_dim, -0.5f);  /* (head_dim as f32).powf(-0.5), E/compute.rs:4083 */
    for (size_t h = 0; h < heads; ++h) {
        const float* qh = q + h * head_dim;
        float mx = -INFINITY;
        for (size_t j = 0; j < nk; ++j) {
            const float* key = j < n_win ? win + j * win_ld : comp + (j - n_win) * head_dim;
            float s = 0.0f;
            for (size_t d = 0; d < head_dim; ++d) s += qh[d] * key[d];
            s *= scale;
            if (s > mx) mx = s;
        }
        float denom = 0.0f;
        if (sink) denom += expf(sink[h] - mx);
        float* oh = out + h * head_dim;
        for (size_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
        float wsum = 0.0f;
        for (size_t j = 0; j < nk; ++j) {
            const float* key = j < n_win ? win + j * win_ld : comp + (j - n_win) * head_dim;
            float s = 0.0f;
            for (size_t d = 0; d < head_dim; ++d) s += qh[d] * key[d];
            const float w = expf((s * scale) - mx);
            wsum += w;
            for (size_t d = 0; d < head_dim; ++d) oh[d] += w * key[d];
        }
        denom += wsum;
        if (denom > 0.0f)
            for (size_t d = 0; d < head_dim; ++d) oh[d] /= denom;
        or_rope_apply(oh + nope_dim, token_pos, inv, pairs, 1);
    }
}

/* ------------------------------------------------------ mHC (hyper-connections) */

static float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

static void or_comb_rows(float* comb, size_t hc, float eps) {
    for (size_t j = 0; j < hc; ++j) {
        float s = 0.0f;
        for (size_t k = 0; k < hc; ++k) s += comb[j * hc + k];
        for (size_t k = 0; k < hc; ++k) comb[j * hc + k] /= s + eps;
    }
}

static void or_comb_cols(float* comb, size_t hc, float eps) {
    for (size_t k = 0; k < hc; ++k) {
        float s = 0.0f;
        for (size_t j = 0; j < hc; ++j) s += comb[j * hc + k];
        for (size_t j = 0; j < hc; ++j) comb[j * hc + k] /= s + eps;
    }
}

/* hc_split_sinkhorn_scalar (E/compute.rs:4945-5000) with normalize_comb_rows
 * / normalize_comb_cols (E/compute.rs:4992-5014): pre = sigmoid(m*s0 + b) +
 * eps, post = 2 sigmoid(m*s1 + b), comb = row softmax(m*s2 + b) + eps, one
 * column normalisation, then iters - 1 rounds of rows then columns. */
int or_hc_split_sinkhorn(const float* mixes, const float* scale, const float* base, size_t hc, size_t iters,
                         float eps, float* pre, float* post, float* comb) {
    for (size_t j = 0; j < hc; ++j) {
        pre[j] = or_sigmoid(mixes[j] * scale[0] + base[j]) + eps;
        post[j] = 2.0f * or_sigmoid(mixes[j + hc] * scale[1] + base[j + hc]);
    }
    for (size_t j = 0; j < hc; ++j)
        for (size_t k = 0; k < hc; ++k)
            comb[j * hc + k] = mixes[2 * hc + j * hc + k] * scale[2] + base[2 * hc + j * hc + k];
    for (size_t j = 0; j < hc; ++j) {
        float* row = comb + j * hc;
        float mx = -INFINITY;
        for (size_t k = 0; k < hc; ++k) mx = fmaxf(mx, row[k]);
        float s = 0.0f;
        for (size_t k = 0; k < hc; ++k) {
            row[k] = expf(row[k] - mx);
            s += row[k];
        }
        for (size_t k = 0; k < hc; ++k) row[k] = row[k] / s + eps;
    }
    or_comb_cols(comb, hc, eps);
    for (size_t it = 1; it < iters; ++it) {
        or_comb_rows(comb, hc, eps);
        or_comb_cols(comb, hc, eps);
    }
    return OR_OK;
}

/* hc_pre_into (E/compute.rs:5016-5050): fn [mix_hc][hc * hidden] f32;
 * mixes_out (optional) receives the pre-sinkhorn mixes. */
int or_hc_pre(const float* fn, const float* scale, const float* base, size_t hc, size_t hidden, size_t iters,
              float eps, const float* x, float* y, float* pre, float* post, float* comb, float* mixes_out) {
    const size_t hc_dim = hc * hidden, mix_hc = (2 + hc) * hc;
    float s = 0.0f;
    for (size_t i = 0; i < hc_dim; ++i) s += x[i] * x[i];
    const float ms = s / (float)hc_dim;
    const float inv = 1.0f / sqrtf(ms + eps);
    float* mixes = (float*)malloc(mix_hc * sizeof(float));
    if (!mixes) return OR_SCRATCH_TOO_SMALL;
    for (size_t j = 0; j < mix_hc; ++j) {
        float acc = 0.0f;
        for (size_t i = 0; i < hc_dim; ++i) acc += fn[j * hc_dim + i] * x[i];
        mixes[j] = acc * inv;
    }
    if (mixes_out) memcpy(mixes_out, mixes, mix_hc * sizeof(float));
    or_hc_split_sinkhorn(mixes, scale, base, hc, iters, eps, pre, post, comb);
    free(mixes);
    for (size_t d = 0; d < hidden; ++d) {
        float acc = 0.0f;
        for (size_t i = 0; i < hc; ++i) acc += pre[i] * x[i * hidden + d];
        y[d] = acc;
    }
    return OR_OK;
}

/* hc_post_into (E/compute.rs:5055-5092): out[k] = post[k] * y + sum over i
 * of comb[k][i] * residual[i], the sum from the post term in order of i. */
void or_hc_post(const float* y, const float* residual, const float* post, const float* comb, float* out, size_t hc,
                size_t hidden) {
    for (size_t k = 0; k < hc; ++k)
        for (size_t d = 0; d < hidden; ++d) {
            float acc = post[k] * y[d];
            for (size_t i = 0; i < hc; ++i) acc += comb[k * hc + i] * residual[i * hidden + d];
            out[k * hidden + d] = acc;
        }
}
