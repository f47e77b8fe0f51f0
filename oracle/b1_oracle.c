/*
 * CPU oracle for the B1_0 1-bit linear — TEST INFRASTRUCTURE ONLY.
 * See b1_oracle.h for what each function restates and how it is pinned.
 *
 * Build flags matter for the AVX2 restatement: it is compiled with
 * -ffp-contract=off so that the multiply and add of src/b1_0_kernel.h:134
 * stay two roundings, as the reference source writes them
 * (_mm256_mul_ps then _mm256_add_ps).  The reference's CMakeLists.txt:7-21
 * sets -mavx2 -mfma and no optimisation level.
 */
#define _GNU_SOURCE
#include "b1_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__AVX2__)
#include <immintrin.h>
#endif

/* ---------------------------------------------------------------- fp16 -- */

float b1o_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (e == 0x1f) {
        /* Inf keeps a zero mantissa; NaN keeps its payload, made quiet. */
        bits = sign | 0x7f800000u | (m << 13) | (m ? 0x00400000u : 0u);
    } else if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        f = (float)m * 5.9604644775390625e-08f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

void b1o_fp16_to_fp32_n(const uint16_t *h, float *f, size_t n) {
    for (size_t i = 0; i < n; i++) f[i] = b1o_fp16_to_fp32(h[i]);
}

uint16_t b1o_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* Inf / NaN */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (ax < 0x38800000u) {                                     /* < 2^-14 */
        uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign; /* < 2^-25 rounds to zero */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* ------------------------------------------------------- pack / unpack -- */

/* Sum of 32 fp32 values in the order numpy's add.reduce uses for a
 * contiguous length-32 row (first element as the start value, then its
 * 8-accumulator pairwise kernel over the remaining 31).  This makes the C
 * packer produce the same fp32 mean that convert_to_b1_0_packed.py:34
 * (np.mean(np.abs(...), axis=-1)) produces; tests check the two agree. */
static float np_sum32(const float *a) {
    const float *p = a + 1;
    const int n = 31;
    float r[8];
    for (int j = 0; j < 8; j++) r[j] = p[j];
    int i;
    for (i = 8; i < n - (n % 8); i += 8)
        for (int j = 0; j < 8; j++) r[j] += p[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; i++) res += p[i];
    return a[0] + res;
}

/* convert_to_b1_0_packed.py:21-43: scale = fp16(mean|w|), bit = (w >= 0),
 * bytes [scale_lo, scale_hi, bits0..bits3] per 32-weight block. */
void b1o_pack(const float *W, int N, int K, uint8_t *P) {
    const int nb = K / B1O_BLOCK_SIZE;
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < nb; b++) {
            const float *blk = W + (size_t)n * K + (size_t)b * B1O_BLOCK_SIZE;
            float ab[B1O_BLOCK_SIZE];
            uint32_t bits = 0;
            for (int i = 0; i < B1O_BLOCK_SIZE; i++) {
                ab[i] = fabsf(blk[i]);
                if (blk[i] >= 0.0f) bits |= 1u << i;
            }
            uint16_t s = b1o_fp32_to_fp16(np_sum32(ab) / 32.0f);
            uint8_t *o = P + ((size_t)n * nb + b) * B1O_BLOCK_BYTES;
            o[0] = (uint8_t)(s & 0xff);
            o[1] = (uint8_t)(s >> 8);
            o[2] = (uint8_t)(bits & 0xff);
            o[3] = (uint8_t)((bits >> 8) & 0xff);
            o[4] = (uint8_t)((bits >> 16) & 0xff);
            o[5] = (uint8_t)(bits >> 24);
        }
    }
}

/* tests/c_ops/test_b1_linear.cpp:129-163, the reference's C++ writer: the
 * same layout, with the block sum taken left to right (it can differ from
 * the numpy order by one fp16 ulp at a rounding tie). */
void b1o_pack_seq(const float *W, int N, int K, uint8_t *P) {
    const int nb = K / B1O_BLOCK_SIZE;
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < nb; b++) {
            const float *blk = W + (size_t)n * K + (size_t)b * B1O_BLOCK_SIZE;
            float sum = 0.0f;
            uint32_t bits = 0;
            for (int i = 0; i < B1O_BLOCK_SIZE; i++) {
                sum += fabsf(blk[i]);
                if (blk[i] >= 0.0f) bits |= 1u << i;
            }
            uint16_t s = b1o_fp32_to_fp16(sum / 32.0f);
            uint8_t *o = P + ((size_t)n * nb + b) * B1O_BLOCK_BYTES;
            o[0] = (uint8_t)(s & 0xff);
            o[1] = (uint8_t)(s >> 8);
            o[2] = (uint8_t)(bits & 0xff);
            o[3] = (uint8_t)((bits >> 8) & 0xff);
            o[4] = (uint8_t)((bits >> 16) & 0xff);
            o[5] = (uint8_t)(bits >> 24);
        }
    }
}

static inline uint16_t rd_scale(const uint8_t *b) {
    return (uint16_t)(b[0] | ((uint16_t)b[1] << 8));
}
static inline uint32_t rd_bits(const uint8_t *b) {
    return (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
           ((uint32_t)b[5] << 24);
}

/* tests/test_weight_parity.py:13-23: W = (2*bit-1) * fp32(scale) */
void b1o_unpack(const uint8_t *P, int N, int K, float *W) {
    const int nb = K / B1O_BLOCK_SIZE;
    for (int n = 0; n < N; n++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = P + ((size_t)n * nb + b) * B1O_BLOCK_BYTES;
            float s = b1o_fp16_to_fp32(rd_scale(blk));
            uint32_t bits = rd_bits(blk);
            for (int i = 0; i < B1O_BLOCK_SIZE; i++)
                W[(size_t)n * K + (size_t)b * B1O_BLOCK_SIZE + i] =
                    ((bits >> i) & 1u) ? s : -s;
        }
}

/* ------------------------------------------------------- scalar path -- */

/* ggml's split of out_dim over nth tasks, src/b1_0_kernel.h:75-77 */
static void row_range(int N, int ith, int nth, int *r0, int *r1) {
    int per = (N + nth - 1) / nth;
    int s = ith * per;
    int e = s + per > N ? N : s + per;
    *r0 = s;
    *r1 = e < s ? s : e;
}

/* One output element in the canonical order of src/b1_0_kernel.h:253-277:
 * block_sum accumulates +-a sequentially, sum += scale * block_sum. */
static inline float dot_scalar(const float *a, const uint8_t *wrow, int nb) {
    float sum = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = wrow + (size_t)b * B1O_BLOCK_BYTES;
        float scale = b1o_fp16_to_fp32(rd_scale(blk));
        uint32_t bits = rd_bits(blk);
        float bs = 0.0f;
        for (int i = 0; i < B1O_BLOCK_SIZE; i++) {
            float x = a[b * B1O_BLOCK_SIZE + i];
            if ((bits >> i) & 1u)
                bs += x;
            else
                bs -= x;
        }
        sum += scale * bs;
    }
    return sum;
}

int64_t b1o_linear_scalar_task(const float *act, const uint8_t *w, float *out,
                               int M, int K, int N, int ith, int nth) {
    const int nb = K / B1O_BLOCK_SIZE;
    const size_t rs = (size_t)nb * B1O_BLOCK_BYTES;
    int r0, r1;
    row_range(N, ith, nth, &r0, &r1);
    int64_t bad = 0;
    for (int b0 = 0; b0 < M; b0 += 4) {
        int bc = b0 + 4 <= M ? 4 : M - b0;
        for (int r = r0; r < r1; r++)
            for (int b = b0; b < b0 + bc; b++) {
                float s = dot_scalar(act + (size_t)b * K, w + (size_t)r * rs, nb);
                if (!isfinite(s)) bad++;
                out[(size_t)b * N + r] = s;
            }
    }
    return bad;
}

/* --------------------------------------------------------- AVX2 path -- */

#if defined(__AVX2__)
/* Per-lane sign masks for one 32-bit word: lane l of mask j carries the
 * fp32 sign bit when bit (8j + l) is CLEAR (bit = 0 -> -a), as in
 * src/b1_0_kernel.h:87-91,127-131. */
static inline void sign_masks(uint32_t bits, __m256 m[4]) {
    const __m256i lane = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
    const __m256i one = _mm256_set1_epi32(1);
    const __m256i sgn = _mm256_set1_epi32((int)0x80000000u);
    __m256i w = _mm256_set1_epi32((int)bits);
    for (int j = 0; j < 4; j++) {
        __m256i sh = _mm256_add_epi32(lane, _mm256_set1_epi32(8 * j));
        __m256i bit = _mm256_and_si256(_mm256_srlv_epi32(w, sh), one);
        /* bit == 0 -> all ones & sign -> sign; bit == 1 -> 0 */
        __m256i neg = _mm256_cmpeq_epi32(bit, _mm256_setzero_si256());
        m[j] = _mm256_castsi256_ps(_mm256_and_si256(neg, sgn));
    }
}

/* 8-lane horizontal sum in the reference's order (src/b1_0_kernel.h:180-187):
 * v_i = s_i + s_{i+4}; then ((v0 + v1) + (v2 + v3)). */
static inline float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}
#endif

int b1o_has_avx2(void) {
#if defined(__AVX2__)
    return 1;
#else
    return 0;
#endif
}

int64_t b1o_linear_avx2_task(const float *act, const uint8_t *w, float *out,
                             int M, int K, int N, int ith, int nth) {
#if defined(__AVX2__)
    const int nb = K / B1O_BLOCK_SIZE;
    const size_t rs = (size_t)nb * B1O_BLOCK_BYTES;
    int r0, r1;
    row_range(N, ith, nth, &r0, &r1);
    int64_t bad = 0;
    for (int b0 = 0; b0 < M; b0 += 4) {
        int bc = b0 + 4 <= M ? 4 : M - b0;
        for (int rt = r0; rt < r1; rt += 4) {
            int rc = rt + 4 <= r1 ? 4 : r1 - rt;
            for (int b = b0; b < b0 + bc; b++) {
                const float *a = act + (size_t)b * K;
                if (rc == 4) {
                    __m256 acc[4];
                    for (int q = 0; q < 4; q++) acc[q] = _mm256_setzero_ps();
                    for (int blk = 0; blk < nb; blk++) {
                        __m256 x[4];
                        for (int j = 0; j < 4; j++)
                            x[j] = _mm256_loadu_ps(a + blk * 32 + 8 * j);
                        for (int q = 0; q < 4; q++) {
                            const uint8_t *wb =
                                w + (size_t)(rt + q) * rs + (size_t)blk * B1O_BLOCK_BYTES;
                            __m256 sc = _mm256_set1_ps(b1o_fp16_to_fp32(rd_scale(wb)));
                            __m256 m[4];
                            sign_masks(rd_bits(wb), m);
                            __m256 t01 = _mm256_add_ps(_mm256_xor_ps(x[0], m[0]),
                                                       _mm256_xor_ps(x[1], m[1]));
                            __m256 t23 = _mm256_add_ps(_mm256_xor_ps(x[2], m[2]),
                                                       _mm256_xor_ps(x[3], m[3]));
                            acc[q] = _mm256_add_ps(acc[q],
                                                   _mm256_mul_ps(_mm256_add_ps(t01, t23), sc));
                        }
                    }
                    for (int q = 0; q < 4; q++) {
                        float s = hsum8(acc[q]);
                        if (!isfinite(s)) bad++;
                        out[(size_t)b * N + rt + q] = s;
                    }
                } else {
                    /* remainder rows: scalar arithmetic, :204-236 */
                    for (int q = 0; q < rc; q++) {
                        float s = dot_scalar(a, w + (size_t)(rt + q) * rs, nb);
                        if (!isfinite(s)) bad++;
                        out[(size_t)b * N + rt + q] = s;
                    }
                }
            }
        }
    }
    return bad;
#else
    (void)act; (void)w; (void)out; (void)M; (void)K; (void)N; (void)ith; (void)nth;
    return -1;
#endif
}

/* ---------------------------------------------------- threaded driver -- */

typedef struct {
    const float *act;
    const uint8_t *w;
    float *out;
    int M, K, N, nth, nthreads, tid, variant;
    int64_t bad;
} job_t;

static void *run_job(void *p) {
    job_t *j = (job_t *)p;
    j->bad = 0;
    for (int ith = j->tid; ith < j->nth; ith += j->nthreads) {
        int64_t r = j->variant == 1
                        ? b1o_linear_avx2_task(j->act, j->w, j->out, j->M, j->K, j->N, ith, j->nth)
                        : b1o_linear_scalar_task(j->act, j->w, j->out, j->M, j->K, j->N, ith, j->nth);
        if (r < 0) {
            j->bad = -1;
            return NULL;
        }
        j->bad += r;
    }
    return NULL;
}

int64_t b1o_linear(const float *act, const uint8_t *w, float *out, int M,
                   int K, int N, int nth, int nthreads, int variant) {
    if (variant == 1 && !b1o_has_avx2()) return -1;
    if (nth < 1) nth = 1;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > nth) nthreads = nth;
    job_t *jobs = (job_t *)calloc((size_t)nthreads, sizeof(job_t));
    pthread_t *th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    for (int t = 0; t < nthreads; t++) {
        job_t j = {act, w, out, M, K, N, nth, nthreads, t, variant, 0};
        jobs[t] = j;
    }
    for (int t = 1; t < nthreads; t++) pthread_create(&th[t], NULL, run_job, &jobs[t]);
    run_job(&jobs[0]);
    int64_t bad = 0;
    for (int t = 0; t < nthreads; t++) {
        if (t > 0) pthread_join(th[t], NULL);
        if (jobs[t].bad < 0) bad = -1;
        if (bad >= 0) bad += jobs[t].bad;
    }
    free(jobs);
    free(th);
    return bad;
}

/* -------------------------------------------------------- fp64 brute -- */

void b1o_linear_f64(const float *act, const uint8_t *w, double *out, int M,
                    int K, int N) {
    const int nb = K / B1O_BLOCK_SIZE;
    const size_t rs = (size_t)nb * B1O_BLOCK_BYTES;
    for (int n = 0; n < N; n++) {
        const uint8_t *wr = w + (size_t)n * rs;
        for (int m = 0; m < M; m++) {
            const float *a = act + (size_t)m * K;
            double s = 0.0;
            for (int b = 0; b < nb; b++) {
                double sc = (double)b1o_fp16_to_fp32(rd_scale(wr + (size_t)b * 6));
                uint32_t bits = rd_bits(wr + (size_t)b * 6);
                for (int i = 0; i < 32; i++) {
                    double x = (double)a[b * 32 + i];
                    s += ((bits >> i) & 1u) ? sc * x : -sc * x;
                }
            }
            out[(size_t)m * N + n] = s;
        }
    }
}
