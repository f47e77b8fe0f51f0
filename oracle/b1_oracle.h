/*
 * CPU oracle for the B1_0 1-bit linear — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline).
 * The product path (bonsai.cpp_amd/) never calls it.
 *
 * It restates, in repo-owned C, the arithmetic of the reference kernel
 * src/b1_0_kernel.h of Juste-Leo2/bonsai.cpp:
 *   - scalar spec path        src/b1_0_kernel.h:240-287 (and the AVX2
 *                             remainder :204-236, same arithmetic)
 *   - AVX2 path               src/b1_0_kernel.h:79-203 (B_TILE=4 tokens x
 *                             R_TILE=4 rows, per-lane sums, 8-lane hsum)
 *   - ggml row split          src/b1_0_kernel.h:75-77
 *   - fp16 -> fp32            src/b1_0_kernel.h:17-19 (ggml_fp16_to_fp32,
 *                             an exact IEEE conversion)
 *   - packed layout writer    convert_to_b1_0_packed.py:21-43 (numpy sum
 *                             order) and tests/c_ops/test_b1_linear.cpp:129-163
 *                             (sequential sum order)
 *   - packed layout reader    tests/test_weight_parity.py:13-23
 * The reference's abort() on a non-finite output (src/b1_0_kernel.h:194-198,
 * 230-233, 279-282) is reported here as a returned count instead.
 *
 * Pinning (each function's check lives in tests/test_oracle.py):
 *   b1o_fp16_to_fp32      exhaustive over all 65536 patterns vs numpy/F16C
 *   b1o_fp32_to_fp16      random + edge values vs numpy astype(float16)
 *   b1o_pack / b1o_unpack round trip bit-exact; pack == numpy quantize_b1_0
 *   b1o_pack_seq          scale == fp16(np.cumsum(|w|)[-1] / 32) (numpy's
 *                         cumulative sum is sequential in float32)
 *   b1o_linear_scalar     fp64 brute force, closed forms (ones -> 16.0,
 *                         complement -> negation, one-hot -> +-scale),
 *                         reference cosine gates on the reference's own
 *                         seeded inputs
 *   b1o_linear_avx2       vs an independent lane-by-lane numpy restatement
 *                         (bit-exact), vs scalar and fp64 (ulp bounds)
 */
#ifndef B1_ORACLE_H
#define B1_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define B1O_BLOCK_SIZE 32
#define B1O_BLOCK_BYTES 6

/* IEEE binary16 <-> binary32 */
float b1o_fp16_to_fp32(uint16_t h);
uint16_t b1o_fp32_to_fp16(float f); /* round to nearest even */
void b1o_fp16_to_fp32_n(const uint16_t *h, float *f, size_t n);

/* Packed layout: W[N][K] fp32 -> P[N][K/32*6] */
void b1o_pack(const float *W, int N, int K, uint8_t *P);
void b1o_pack_seq(const float *W, int N, int K, uint8_t *P);
void b1o_unpack(const uint8_t *P, int N, int K, float *W);

/* One ggml task (ith of nth) of the reference kernel.  act [M][K] fp32
 * contiguous, w packed [N][K/32*6], out [M][N].  Returns the number of
 * non-finite outputs this task produced (the reference aborts instead). */
int64_t b1o_linear_scalar_task(const float *act, const uint8_t *w, float *out,
                               int M, int K, int N, int ith, int nth);
int64_t b1o_linear_avx2_task(const float *act, const uint8_t *w, float *out,
                             int M, int K, int N, int ith, int nth);

/* Runs all nth tasks on nthreads pthreads (nthreads <= nth; task i runs on
 * thread i % nthreads).  variant: 0 = scalar, 1 = AVX2.  Returns the number
 * of non-finite outputs, or -1 if the variant is unavailable. */
int64_t b1o_linear(const float *act, const uint8_t *w, float *out, int M,
                   int K, int N, int nth, int nthreads, int variant);

/* fp64 brute force: out64[m][n] = sum_k a[m][k] * dequant(w)[n][k] */
void b1o_linear_f64(const float *act, const uint8_t *w, double *out, int M,
                    int K, int N);

int b1o_has_avx2(void);

#ifdef __cplusplus
}
#endif
#endif
