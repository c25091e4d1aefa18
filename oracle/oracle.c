/*
 * oracle.c — CPU restatement of mini-rust-inference's quantized-matmul hot
 * path.  TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the
 * timed CPU baseline; never part of the product library.
 *
 * Build: oracle/Makefile (gcc, -O2 -ffp-contract=off, baseline x86-64 with the
 * AVX2 dot compiled under target("avx2") only, mirroring the reference's
 * `#[target_feature(enable = "avx2")]`, no FMA, no VNNI).
 *
 * Citations are src/<file>:<line> of the reference crate.
 *
 * Parity status of each function (how it is pinned; see tests/):
 *   orc_f16_to_f32            KATs quantization.rs:529-545 + exhaustive check
 *                             against numpy float16 for all 65536 bit patterns
 *   orc_f32_to_f16            KATs quantization.rs:516-527 + truncation
 *                             invariant (bits>>13) over the normal range
 *   orc_quantize_symmetric    KATs symmetric.rs:33-40,171-242 + closed form
 *                             with explicit half-away-from-zero rounding
 *   orc_quantize_per_channel  KATs per_channel.rs:84-96,243-289 + closed form
 *   orc_dot_i8_*              KATs int8_avx2.rs:219-297 + int64 brute force
 *   orc_matmul_int8*          int64 matmul + float32 epilogue (numpy), KATs
 *                             int8.rs:171-353, parallel.rs:369-468
 *   orc_create/dequantize_q8_0  KATs dequant.rs:944-983 + doctest :88-101
 *   orc_matmul_q8_0_direct    int64 block dots + sequential float32 sum
 *                             (numpy) + KATs q8_direct.rs:355-509
 *   orc_create/dequantize_q4_0  KATs quantization.rs:589-611, dequant.rs
 *                             doctest :453-470, :1246-1290
 *   orc_matmul_q4_0_dequant   sequential float32 restatement (numpy) + KATs
 *                             q4_0.rs:214-390
 *   orc_matmul_q4_0_w4a8      (extension, no reference counterpart) equals
 *                             orc_matmul_q8_0_direct on the same blocks
 *                             expanded to Q8_0 (bit for bit); GGML order
 *                             equals the interleaved order on byte-permuted
 *                             blocks; int64 block dots (numpy)
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <immintrin.h>

/* ---------------------------------------------------------------------- */
/* error reporting (TensorError's `reason` string)                         */
/* ---------------------------------------------------------------------- */

static __thread char g_err[512];

const char *orc_last_error(void) { return g_err; }

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

/* ---------------------------------------------------------------------- */
/* f16 codec                                                               */
/* ---------------------------------------------------------------------- */

/* f16_to_f32, gguf/quantization.rs:416-459.  Every branch is exact in f32:
 * (1 + m/1024) has 11 significant bits and the power of two scales it
 * exactly; subnormals are m * 2^-10 * 2^-14. */
float orc_f16_to_f32(uint16_t h) {
    unsigned sign = (h >> 15) & 1u;
    unsigned exp = (h >> 10) & 0x1Fu;
    unsigned mant = h & 0x3FFu;
    float val;
    if (exp == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        val = (float)mant * (1.0f / 1024.0f) * (1.0f / 16384.0f);
    } else if (exp == 31) {
        if (mant == 0) return sign ? -INFINITY : INFINITY;
        return NAN; /* f32::NAN, sign dropped (quantization.rs:448) */
    } else {
        val = (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, (int)exp - 15);
    }
    return sign ? -val : val;
}

/* f32_to_f16, gguf/quantization.rs:464-497: truncating encoder.  The
 * subnormal branch shifts by (126-exp)+13, which exceeds 31 for exp <= 106;
 * Rust release builds mask the shift amount to 5 bits, restated here. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 255) {
        if (mant == 0) return (uint16_t)((sign << 15) | 0x7C00u);
        uint16_t m = (uint16_t)(mant >> 13);
        if (m < 1) m = 1;
        return (uint16_t)((sign << 15) | 0x7C00u | m);
    } else if (exp > 142) {
        return (uint16_t)((sign << 15) | 0x7C00u);
    } else if (exp < 103) {
        return (uint16_t)(sign << 15);
    } else if (exp < 113) {
        uint32_t mant_with_implicit = mant | 0x800000u;
        uint32_t shift = (uint32_t)(126 - exp);
        uint16_t mant16 = (uint16_t)(mant_with_implicit >> ((shift + 13u) & 31u));
        return (uint16_t)((sign << 15) | mant16);
    } else {
        uint16_t exp16 = (uint16_t)((exp - 112) & 0x1F);
        uint16_t mant16 = (uint16_t)(mant >> 13);
        return (uint16_t)((sign << 15) | (exp16 << 10) | mant16);
    }
}

/* ---------------------------------------------------------------------- */
/* quantizers                                                              */
/* ---------------------------------------------------------------------- */

/* `(v * inv).round().clamp(lo, hi) as i8` with Rust semantics: round half
 * away from zero (roundf), clamp leaves NaN as NaN, and the saturating `as`
 * cast maps NaN to 0. */
static inline int8_t round_clamp_i8(float y, float lo, float hi) {
    float r = roundf(y);
    if (isnan(r)) return 0;
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int8_t)r;
}

/* fold(0.0, f32::max) over |v|: f32::max returns the non-NaN operand, like
 * C fmaxf. */
static inline float max_abs_of(const float *v, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) m = fmaxf(m, fabsf(v[i]));
    return m;
}

/* quantize_symmetric, quant/int8/symmetric.rs:42-57 */
float orc_quantize_symmetric(const float *values, size_t n, int8_t *q_out) {
    float max_abs = max_abs_of(values, n);
    float scale = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
    float inv_scale = 1.0f / scale;
    for (size_t i = 0; i < n; i++)
        q_out[i] = round_clamp_i8(values[i] * inv_scale, -127.0f, 127.0f);
    return scale;
}

/* quantize_per_channel, quant/int8/per_channel.rs:98-128 */
int orc_quantize_per_channel(const float *w, size_t len, size_t n_out,
                             size_t k_in, int8_t *data, float *scales) {
    if (len != n_out * k_in)
        return fail(ORC_INVALID_SHAPE, "weights.len()=%zu != n_out*k_in=%zu",
                    len, n_out * k_in);
    for (size_t n = 0; n < n_out; n++) {
        const float *row = w + n * k_in;
        float max_abs = max_abs_of(row, k_in);
        float scale = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
        float inv = 1.0f / scale;
        scales[n] = scale;
        for (size_t k = 0; k < k_in; k++)
            data[n * k_in + k] = round_clamp_i8(row[k] * inv, -127.0f, 127.0f);
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* int8 dots                                                               */
/* ---------------------------------------------------------------------- */

/* dot_i8_scalar, ops/matmul/int8_avx2.rs:117-122 */
int32_t orc_dot_i8_scalar(const int8_t *a, const int8_t *b, size_t n) {
    int32_t s = 0;
    for (size_t i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

/* hsum_epi32, ops/matmul/int8_avx2.rs:49-60 */
__attribute__((target("avx2"))) static inline int32_t hsum_epi32(__m256i v) {
    __m128i lo128 = _mm256_castsi256_si128(v);
    __m128i hi128 = _mm256_extracti128_si256(v, 1);
    __m128i sum4 = _mm_add_epi32(lo128, hi128);
    __m128i shuf = _mm_shuffle_epi32(sum4, 0xB1); /* 0b10_11_00_01 */
    __m128i sum2 = _mm_add_epi32(sum4, shuf);
    __m128i shuf2 = _mm_shuffle_epi32(sum2, 0x4E); /* 0b01_00_11_10 */
    __m128i sum1 = _mm_add_epi32(sum2, shuf2);
    return _mm_cvtsi128_si32(sum1);
}

/* avx2_impl::dot_i8, ops/matmul/int8_avx2.rs:69-111.  Exact for a in
 * [-127,127]; like the reference it is wrong for a < 0 with b == -128
 * (sign() wraps), which per-channel weights never contain. */
__attribute__((target("avx2"))) static int32_t dot_i8_avx2_impl(
    const int8_t *a, const int8_t *b, size_t n) {
    size_t chunks = n / 32;
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i acc = _mm256_setzero_si256();
    for (size_t i = 0; i < chunks; i++) {
        __m256i va = _mm256_loadu_si256((const __m256i *)(a + i * 32));
        __m256i vb = _mm256_loadu_si256((const __m256i *)(b + i * 32));
        __m256i va_abs = _mm256_abs_epi8(va);
        __m256i vb_sign = _mm256_sign_epi8(vb, va);
        __m256i prod16 = _mm256_maddubs_epi16(va_abs, vb_sign);
        __m256i prod32 = _mm256_madd_epi16(prod16, ones);
        acc = _mm256_add_epi32(acc, prod32);
    }
    int32_t result = hsum_epi32(acc);
    for (size_t i = chunks * 32; i < n; i++)
        result += (int32_t)a[i] * (int32_t)b[i];
    return result;
}

int orc_have_avx2(void) { return __builtin_cpu_supports("avx2") ? 1 : 0; }

/* dot_i8_avx2, ops/matmul/int8_avx2.rs:136-148 (runtime feature check). */
int32_t orc_dot_i8_avx2(const int8_t *a, const int8_t *b, size_t n) {
    static int have = -1;
    if (have < 0) have = orc_have_avx2();
    if (have) return dot_i8_avx2_impl(a, b, n);
    return orc_dot_i8_scalar(a, b, n);
}

/* ---------------------------------------------------------------------- */
/* per-channel INT8 GEMMs                                                  */
/* ---------------------------------------------------------------------- */

static int check_act_len(const char *fn, size_t len, size_t m, size_t k) {
    if (len != m * k)
        return fail(ORC_INVALID_SHAPE, "%s: act_q.len()=%zu != m*k=%zu*%zu=%zu",
                    fn, len, m, k, m * k);
    return ORC_OK;
}

/* The epilogue `acc as f32 * act_scale * scales[n]` (int8.rs:93): i32 -> f32
 * round-to-nearest-even, then two f32 multiplies left to right. */
static inline float epilogue(int32_t acc, float s_a, float s_w) {
    float t = (float)acc * s_a;
    return t * s_w;
}

/* matmul_int8, ops/matmul/int8.rs:61-98 */
int orc_matmul_int8(const int8_t *act_q, size_t act_q_len, float act_scale,
                    const int8_t *w, const float *scales, size_t n_out,
                    size_t k_in, size_t m, float *out, int32_t *acc_out) {
    int rc = check_act_len("matmul_int8", act_q_len, m, k_in);
    if (rc) return rc;
    for (size_t mi = 0; mi < m; mi++) {
        const int8_t *a_row = act_q + mi * k_in;
        for (size_t ni = 0; ni < n_out; ni++) {
            const int8_t *w_row = w + ni * k_in;
            int32_t acc = 0;
            for (size_t ki = 0; ki < k_in; ki++)
                acc += (int32_t)a_row[ki] * (int32_t)w_row[ki];
            if (acc_out) acc_out[mi * n_out + ni] = acc;
            out[mi * n_out + ni] = epilogue(acc, act_scale, scales[ni]);
        }
    }
    return ORC_OK;
}

/* matmul_int8_avx2, ops/matmul/int8_avx2.rs:174-207 */
int orc_matmul_int8_avx2(const int8_t *act_q, size_t act_q_len,
                         float act_scale, const int8_t *w,
                         const float *scales, size_t n_out, size_t k_in,
                         size_t m, float *out) {
    int rc = check_act_len("matmul_int8_avx2", act_q_len, m, k_in);
    if (rc) return rc;
    for (size_t mi = 0; mi < m; mi++)
        for (size_t ni = 0; ni < n_out; ni++)
            out[mi * n_out + ni] =
                epilogue(orc_dot_i8_avx2(act_q + mi * k_in, w + ni * k_in, k_in),
                         act_scale, scales[ni]);
    return ORC_OK;
}

/* Per-row activation scale variant (no reference counterpart). */
int orc_matmul_int8_rows(const int8_t *act_q, size_t act_q_len,
                         const float *act_scales, const int8_t *w,
                         const float *scales, size_t n_out, size_t k_in,
                         size_t m, float *out, int32_t *acc_out) {
    int rc = check_act_len("matmul_int8_rows", act_q_len, m, k_in);
    if (rc) return rc;
    for (size_t mi = 0; mi < m; mi++)
        for (size_t ni = 0; ni < n_out; ni++) {
            int32_t acc = orc_dot_i8_scalar(act_q + mi * k_in, w + ni * k_in, k_in);
            if (acc_out) acc_out[mi * n_out + ni] = acc;
            out[mi * n_out + ni] = epilogue(acc, act_scales[mi], scales[ni]);
        }
    return ORC_OK;
}

/* ---- worker pool standing in for rayon's global pool ------------------ */

typedef struct {
    const int8_t *act_q;
    float act_scale;
    const int8_t *w;
    const float *scales;
    size_t n_out, k_in, m;
    float *out;
} par_job;

#define POOL_MAX 256
static struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_work, cv_done;
    pthread_t th[POOL_MAX];
    int n;               /* workers in the pool */
    int active;          /* workers allowed on the current job */
    unsigned long gen;   /* job generation */
    par_job job;
    size_t next_row;     /* row counter (guarded by mu) */
    int busy;            /* workers still inside the current job */
    int used[POOL_MAX];  /* worker i took >= 1 row of the current job */
} pool = {.mu = PTHREAD_MUTEX_INITIALIZER,
          .cv_work = PTHREAD_COND_INITIALIZER,
          .cv_done = PTHREAD_COND_INITIALIZER};
static pthread_once_t pool_once = PTHREAD_ONCE_INIT;

/* One output row, parallel.rs:336-343. */
static void par_row(const par_job *j, size_t mi) {
    const int8_t *a_row = j->act_q + mi * j->k_in;
    float *out_row = j->out + mi * j->n_out;
    for (size_t ni = 0; ni < j->n_out; ni++) {
        int32_t acc = orc_dot_i8_avx2(a_row, j->w + ni * j->k_in, j->k_in);
        out_row[ni] = epilogue(acc, j->act_scale, j->scales[ni]);
    }
}

static void *pool_main(void *arg) {
    int id = (int)(intptr_t)arg;
    unsigned long seen = 0;
    pthread_mutex_lock(&pool.mu);
    for (;;) {
        while (pool.gen == seen) pthread_cond_wait(&pool.cv_work, &pool.mu);
        seen = pool.gen;
        if (id >= pool.active) continue;
        for (;;) {
            if (pool.next_row >= pool.job.m) break;
            size_t mi = pool.next_row++;
            pool.used[id] = 1;
            par_job j = pool.job;
            pthread_mutex_unlock(&pool.mu);
            par_row(&j, mi);
            pthread_mutex_lock(&pool.mu);
        }
        if (--pool.busy == 0) pthread_cond_signal(&pool.cv_done);
    }
    return NULL;
}

static void pool_init(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > POOL_MAX) n = POOL_MAX;
    pool.n = (int)n;
    for (int i = 0; i < pool.n; i++)
        pthread_create(&pool.th[i], NULL, pool_main, (void *)(intptr_t)i);
}

/* matmul_int8_parallel, ops/matmul/parallel.rs:308-346 */
int orc_matmul_int8_parallel(const int8_t *act_q, size_t act_q_len,
                             float act_scale, const int8_t *w,
                             const float *scales, size_t n_out, size_t k_in,
                             size_t m, float *out, int n_threads,
                             int *cores_used) {
    int rc = check_act_len("matmul_int8_parallel", act_q_len, m, k_in);
    if (rc) return rc;
    pthread_once(&pool_once, pool_init);
    int active = (n_threads <= 0 || n_threads > pool.n) ? pool.n : n_threads;
    pthread_mutex_lock(&pool.mu);
    pool.job = (par_job){act_q, act_scale, w, scales, n_out, k_in, m, out};
    pool.next_row = 0;
    pool.active = active;
    pool.busy = active;
    memset(pool.used, 0, sizeof pool.used);
    pool.gen++;
    pthread_cond_broadcast(&pool.cv_work);
    while (pool.busy > 0) pthread_cond_wait(&pool.cv_done, &pool.mu);
    int used = 0;
    for (int i = 0; i < active; i++) used += pool.used[i];
    pthread_mutex_unlock(&pool.mu);
    if (cores_used) *cores_used = used;
    return ORC_OK;
}

/* matmul_int8_from_f32, ops/matmul/int8.rs:113-143 */
int orc_matmul_int8_from_f32(const float *input, const size_t *dims,
                             size_t ndim, const int8_t *w,
                             const float *scales, size_t n_out, size_t k_in,
                             float *out, int8_t *act_q_out,
                             float *act_scale_out, int32_t *acc_out) {
    if (ndim != 2)
        return fail(ORC_INVALID_SHAPE,
                    "matmul_int8_from_f32: input must be 2-D, got %zuD", ndim);
    size_t m = dims[0], k = dims[1];
    if (k != k_in)
        return fail(ORC_SHAPE_MISMATCH, "expected [%zu, %zu], got [%zu, %zu]",
                    m, k_in, m, k);
    int8_t *q = act_q_out ? act_q_out : (int8_t *)malloc(m * k + 1);
    float s = orc_quantize_symmetric(input, m * k, q);
    if (act_scale_out) *act_scale_out = s;
    int rc = orc_matmul_int8(q, m * k, s, w, scales, n_out, k_in, m, out, acc_out);
    if (!act_q_out) free(q);
    return rc;
}

/* ---------------------------------------------------------------------- */
/* Q8_0                                                                    */
/* ---------------------------------------------------------------------- */

/* create_q8_0_block, gguf/dequant.rs:389-421 */
void orc_create_q8_0_block(const float *values32, uint8_t *block34) {
    float max_abs = max_abs_of(values32, ORC_QK);
    float scale = (max_abs == 0.0f) ? 0.0f : max_abs / 127.0f;
    uint16_t d = orc_f32_to_f16(scale);
    memset(block34, 0, ORC_Q8_0_BLOCK_BYTES);
    block34[0] = (uint8_t)(d & 0xFF);
    block34[1] = (uint8_t)(d >> 8);
    if (scale > 0.0f) {
        float inv = 1.0f / scale;
        for (int i = 0; i < ORC_QK; i++)
            block34[2 + i] =
                (uint8_t)round_clamp_i8(values32[i] * inv, -128.0f, 127.0f);
    }
}

/* dequantize_q8_0, gguf/dequant.rs:103-134 (scale * q, f32 multiply) */
int orc_dequantize_q8_0(const uint8_t *data, size_t n_bytes, float *out) {
    if (n_bytes % ORC_Q8_0_BLOCK_BYTES)
        return fail(ORC_INVALID_SHAPE, "Q8_0 data length %zu not a multiple of 34",
                    n_bytes);
    size_t nb = n_bytes / ORC_Q8_0_BLOCK_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * ORC_Q8_0_BLOCK_BYTES;
        float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < ORC_QK; i++)
            out[b * ORC_QK + i] = d * (float)(int8_t)blk[2 + i];
    }
    return ORC_OK;
}

/* Q8_0WeightMatrix::from_raw_bytes, ops/matmul/q8_direct.rs:80-107 */
int orc_q8_0_check_raw(size_t n_bytes, size_t n_out, size_t k_in) {
    if (k_in % ORC_QK)
        return fail(ORC_INVALID_SHAPE,
                    "Q8_0WeightMatrix: k_in=%zu is not a multiple of 32", k_in);
    size_t expected = n_out * (k_in / ORC_QK) * ORC_Q8_0_BLOCK_BYTES;
    if (n_bytes != expected)
        return fail(ORC_INVALID_SHAPE,
                    "Q8_0WeightMatrix: data.len()=%zu != expected %zu", n_bytes,
                    expected);
    return ORC_OK;
}

/* matmul_q8_0_direct, ops/matmul/q8_direct.rs:229-289 */
int orc_matmul_q8_0_direct(const float *input, const size_t *dims,
                           size_t ndim, const uint8_t *w_raw, size_t n_bytes,
                           size_t n_out, size_t k_in, float *out,
                           int32_t *block_dots_out, float *act_scales_out) {
    int rc = orc_q8_0_check_raw(n_bytes, n_out, k_in);
    if (rc) return rc;
    if (ndim != 2)
        return fail(ORC_INVALID_SHAPE,
                    "matmul_q8_0_direct: input must be 2-D, got %zuD", ndim);
    size_t m = dims[0], k = dims[1];
    if (k != k_in)
        return fail(ORC_SHAPE_MISMATCH, "expected [%zu, %zu], got [%zu, %zu]",
                    m, k_in, m, k);
    size_t nb = k_in / ORC_QK;
    int8_t *aq = (int8_t *)malloc(k + 1);
    for (size_t mi = 0; mi < m; mi++) {
        float s_a = orc_quantize_symmetric(input + mi * k, k, aq); /* :264 */
        if (act_scales_out) act_scales_out[mi] = s_a;
        for (size_t ni = 0; ni < n_out; ni++) {
            float acc = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                const uint8_t *blk = w_raw + (ni * nb + b) * ORC_Q8_0_BLOCK_BYTES;
                float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                const int8_t *wq = (const int8_t *)(blk + 2);
                int32_t dot = 0;
                for (int i = 0; i < ORC_QK; i++)
                    dot += (int32_t)aq[b * ORC_QK + i] * (int32_t)wq[i];
                if (block_dots_out) block_dots_out[(mi * n_out + ni) * nb + b] = dot;
                float t = (float)dot * s_a; /* :281, left to right */
                t = t * d;
                acc = acc + t;
            }
            out[mi * n_out + ni] = acc;
        }
    }
    free(aq);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Q4_0                                                                    */
/* ---------------------------------------------------------------------- */

/* create_q4_0_block, gguf/dequant.rs:706-749 */
void orc_create_q4_0_block(const float *values32, uint8_t *block18) {
    float max_abs = max_abs_of(values32, ORC_QK);
    float scale = (max_abs == 0.0f) ? 0.0f : max_abs / 7.0f;
    uint16_t d = orc_f32_to_f16(scale);
    block18[0] = (uint8_t)(d & 0xFF);
    block18[1] = (uint8_t)(d >> 8);
    if (scale > 0.0f) {
        float inv = 1.0f / scale;
        for (int i = 0; i < 16; i++) {
            /* `(v*inv).round() as i32 + 8` then clamp(0,15): the f32 -> i32
             * `as` cast saturates and maps NaN to 0. */
            int q[2];
            for (int h = 0; h < 2; h++) {
                float r = roundf(values32[2 * i + h] * inv);
                int32_t qi;
                if (isnan(r)) qi = 0;
                else if (r >= 2147483647.0f) qi = 2147483647;
                else if (r <= -2147483648.0f) qi = (int32_t)0x80000000u;
                else qi = (int32_t)r;
                int64_t v = (int64_t)qi + 8;
                q[h] = v < 0 ? 0 : (v > 15 ? 15 : (int)v);
            }
            block18[2 + i] = (uint8_t)(q[0] | (q[1] << 4));
        }
    } else {
        for (int i = 0; i < 16; i++) block18[2 + i] = 0x88;
    }
}

/* dequantize_q4_0, gguf/dequant.rs:471-506: element 2i = low nibble - 8,
 * element 2i+1 = high nibble - 8, value = scale * q. */
int orc_dequantize_q4_0(const uint8_t *data, size_t n_bytes, float *out) {
    if (n_bytes % ORC_Q4_0_BLOCK_BYTES)
        return fail(ORC_INVALID_SHAPE, "Q4_0 data length %zu not a multiple of 18",
                    n_bytes);
    size_t nb = n_bytes / ORC_Q4_0_BLOCK_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * ORC_Q4_0_BLOCK_BYTES;
        float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 16; i++) {
            out[b * ORC_QK + 2 * i] = d * (float)((int)(blk[2 + i] & 0x0F) - 8);
            out[b * ORC_QK + 2 * i + 1] = d * (float)((int)(blk[2 + i] >> 4) - 8);
        }
    }
    return ORC_OK;
}

/* matmul_q4_0_dequant, ops/matmul/q4_0.rs:94-181 */
int orc_matmul_q4_0_dequant(const float *input, const size_t *dims,
                            size_t ndim, const uint8_t *w_q4, size_t n_bytes,
                            size_t n_out, size_t k, float *out) {
    if (ndim != 2)
        return fail(ORC_INVALID_SHAPE,
                    "matmul_q4_0_dequant: `input` must be 2-D, got %zuD", ndim);
    size_t m = dims[0], k_in = dims[1];
    if (k_in != k)
        return fail(ORC_SHAPE_MISMATCH, "expected [%zu, %zu], got [%zu, %zu]",
                    m, k, m, k_in);
    if (k % ORC_QK)
        return fail(ORC_INVALID_SHAPE,
                    "matmul_q4_0_dequant: k=%zu must be a multiple of 32", k);
    size_t bpr = k / ORC_QK;
    size_t expected = n_out * bpr * ORC_Q4_0_BLOCK_BYTES;
    if (n_bytes != expected)
        return fail(ORC_INVALID_SHAPE,
                    "matmul_q4_0_dequant: weight_q4 has %zu bytes, expected %zu",
                    n_bytes, expected);
    float buf[ORC_QK];
    for (size_t n = 0; n < n_out; n++) {
        for (size_t mi = 0; mi < m; mi++) {
            float acc = 0.0f;
            const float *x = input + mi * k;
            for (size_t b = 0; b < bpr; b++) {
                const uint8_t *blk = w_q4 + (n * bpr + b) * ORC_Q4_0_BLOCK_BYTES;
                /* dequant_block_into, q4_0.rs:59-68 */
                float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                for (int i = 0; i < 16; i++) {
                    buf[2 * i] = d * (float)((int)(blk[2 + i] & 0x0F) - 8);
                    buf[2 * i + 1] = d * (float)((int)((blk[2 + i] >> 4) & 0x0F) - 8);
                }
                for (int i = 0; i < ORC_QK; i++) {
                    float t = x[b * ORC_QK + i] * buf[i];
                    acc = acc + t;
                }
            }
            out[mi * n_out + n] = acc;
        }
    }
    return ORC_OK;
}

/* Quant e (0..31) of a Q4_0 block as a signed value nibble - 8, in either
 * nibble order: ORC_Q4_INTERLEAVED (the reference's create_q4_0_block,
 * gguf/dequant.rs:706-749 and q4_0.rs:59-68: element 2i = low nibble of byte
 * i, 2i+1 = high nibble) or ORC_Q4_GGML (upstream GGML: element i < 16 = low
 * nibble of byte i, element i + 16 = high nibble of byte i). */
static int q4_quant(const uint8_t *blk, int e, int order) {
    int byte, hi;
    if (order == ORC_Q4_GGML) {
        byte = e & 15;
        hi = e >> 4;
    } else {
        byte = e >> 1;
        hi = e & 1;
    }
    const int nib = hi ? (blk[2 + byte] >> 4) & 0x0F : blk[2 + byte] & 0x0F;
    return nib - 8;
}

/* Q4_0 weights with int8 activations (W4A8).  An extension with no
 * counterpart in the reference: matmul_q8_0_direct (q8_direct.rs:229-289)
 * applied to Q4_0 blocks.  Per row, quantize_symmetric of the row
 * (symmetric.rs:42-57); per output and block, the exact int32 dot of the
 * int8 activations with the quants (nibble - 8), then
 * acc += ((f32)dot * s_a) * d in block order.  Error order as
 * matmul_q4_0_dequant: non-2-D, K mismatch, K%32, byte length. */
int orc_matmul_q4_0_w4a8(const float *input, const size_t *dims, size_t ndim,
                         const uint8_t *w_q4, size_t n_bytes, size_t n_out, size_t k,
                         int order, float *out, int32_t *block_dots_out,
                         float *act_scales_out) {
    if (ndim != 2)
        return fail(ORC_INVALID_SHAPE, "matmul_q4_0_w4a8: input must be 2-D, got %zuD", ndim);
    size_t m = dims[0], k_in = dims[1];
    if (k_in != k)
        return fail(ORC_SHAPE_MISMATCH, "expected [%zu, %zu], got [%zu, %zu]", m, k, m, k_in);
    if (k % ORC_QK)
        return fail(ORC_INVALID_SHAPE, "matmul_q4_0_w4a8: k=%zu is not a multiple of 32", k);
    size_t nb = k / ORC_QK, expected = n_out * nb * ORC_Q4_0_BLOCK_BYTES;
    if (n_bytes != expected)
        return fail(ORC_INVALID_SHAPE, "matmul_q4_0_w4a8: weight_q4 has %zu bytes, expected %zu",
                    n_bytes, expected);
    int8_t *aq = (int8_t *)malloc(k + 1);
    for (size_t mi = 0; mi < m; mi++) {
        float s_a = orc_quantize_symmetric(input + mi * k, k, aq);
        if (act_scales_out) act_scales_out[mi] = s_a;
        for (size_t ni = 0; ni < n_out; ni++) {
            float acc = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                const uint8_t *blk = w_q4 + (ni * nb + b) * ORC_Q4_0_BLOCK_BYTES;
                float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                int32_t dot = 0;
                for (int e = 0; e < ORC_QK; e++)
                    dot += (int32_t)aq[b * ORC_QK + e] * q4_quant(blk, e, order);
                if (block_dots_out) block_dots_out[(mi * n_out + ni) * nb + b] = dot;
                float t = (float)dot * s_a;
                t = t * d;
                acc = acc + t;
            }
            out[mi * n_out + ni] = acc;
        }
    }
    free(aq);
    return ORC_OK;
}
