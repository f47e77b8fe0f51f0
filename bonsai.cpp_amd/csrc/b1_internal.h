// Internal launcher interface between the C ABI (b1_capi.hip) and the
// gfx950 kernels (b1_kernels.hip).  Not installed; no HIP types beyond the
// stream.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace b1 {

// What the packed GEMM's epilogue writes besides the plain product y
// (kind 1: out = res + gate[n] * y; kind 2: SwiGLU over 2 glu_h weight
// rows, out[m][j] = silu(y[m][j]) * y[m][glu_h + j]; kind 3: columns
// [0, split) of y to out as fp32, columns split + j as act(y) into packed
// fp16 activations, column j of pk's rows of ldpw dwords, act 1 = GELU-tanh).
struct GemmEpi {
    const float *gate = nullptr; // [N]
    const float *res = nullptr;  // [M][ldr]
    int64_t ldr = 0;
    int glu_h = 0;
    uint32_t *pk = nullptr; // kind 3: packed fp16 pairs, 16-byte aligned
    int64_t ldpw = 0;       // its row stride in dwords (a multiple of 4)
    int split = 0;          // a multiple of 32
    int act = 0;            // 0 none, 1 GELU-tanh
    // per-row output scales of range-safe packing ([M], powers of two; 1
    // for rows packed unscaled), or nullptr: y[m][n] *= rsc[m] before the
    // epilogue
    const float *rsc = nullptr;
};

struct LinearArgs {
    const float *act;   // [M][lda] fp32
    int64_t lda;        // elements
    const uint8_t *w;   // packed [N][K/32*6]
    int K, N, M;
    float *out;         // [M][ldo] fp32
    int64_t ldo;        // elements
    int32_t *nonfinite; // optional device counter
    const float *rsc = nullptr; // packed inputs only: row scales (see GemmEpi)
};

// fp32 VALU kernel in the reference scalar order; any K % 32 == 0.
hipError_t launch_exact(const LinearArgs &a, int num_cus, hipStream_t s);

// fp16 MFMA GEMM; requires K % 64 == 0, lda % 4 == 0, act 16-byte aligned.
// With a workspace of gemm_workspace_bytes(a) bytes (> 0 when K % 384 == 0)
// the activations are packed to fp16 once (range-safe, launch_pack_rows)
// and streamed into LDS directly; otherwise the kernel converts them while
// staging each tile, and launch_fixup_rows follows.
bool gemm_supported(const LinearArgs &a);
size_t gemm_workspace_bytes(const LinearArgs &a);
// With room for the split-K partials after the packing (256-byte aligned),
// launch_gemm splits K when gemm_splits says so.
size_t gemm_workspace_bytes_total(const LinearArgs &a, int num_cus);
hipError_t launch_gemm(const LinearArgs &a, int num_cus, void *workspace, size_t ws_bytes, hipStream_t s);

// Split-K for plain GEMMs whose tiles would leave most CUs idle: the number
// of K ranges (1 = none; a function of the shape and CU count only, so
// every caller splits a given shape the same way) and the fp32 partial
// area it needs (splits x M x N rounded up to 4 columns).
int gemm_splits(int M, int K, int N, int num_cus);
size_t gemm_split_bytes(int M, int N, int splits);
// The tile kernel of the packed GEMM with the plain, gate-residual or
// packed-output (GELU or none) epilogue: 0 b1_gemm_kernel, 128 x 512 tiles
// (any shape; 64-row tiles for a short last round, split-K for few tiles);
// 1 b1_gemm16_kernel 144 x 384 and 2 b1_gemm16_kernel 128 x 384 (16x16x32
// MFMAs; full tiles, K % 384 == 0, no split), whichever needs the fewest
// rounds on num_cus CUs, counting a BM x BN tile as BM BN / 65536 of a
// 128 x 512 round; ties stay on 0.  A function of the shape and CU count
// only, so every entry point picks alike, for every epilogue (the packed
// output's SwiGLU columns need split % 384 == 0 for the 16x16 kernels;
// otherwise kernel 0).  The kernels sum K in different orders (the same to
// ~1e-6 relative).
int gemm_tiles(int M, int K, int N, int num_cus);

// The two halves of the workspace path.  Packed activations: u32 word
// (row m, 16 j + d) = fp16(a[m][32 j + d]) | fp16(a[m][32 j + d + 16]) << 16,
// row stride ldp/2 words (ldp >= K fp16 elements, ldp % 8 == 0; the GEMM
// reads ldp == K).  pack: K % 32 == 0, lda % 4 == 0, act 16-byte aligned.
// gemm_packed: gemm_packed_ok(M, K, N), packed 16-byte aligned, w 4-byte
// aligned.
bool pack_supported(const float *act, int64_t lda, int M, int K);
hipError_t launch_pack(const float *act, int64_t lda, int M, int K, void *packed, int64_t ldp, hipStream_t s);
bool gemm_packed_ok(int M, int K, int N);
hipError_t launch_gemm_packed(const void *packed, const uint8_t *w, int K, int N, int M, float *out, int64_t ldo,
                              int32_t *nonfinite, int num_cus, hipStream_t s);
// The same split into `splits` K ranges (a divisor of K / 384) with the
// partials in `partials` (gemm_split_bytes, 16-byte aligned), summed in
// order by a second kernel.
hipError_t launch_gemm_packed_split(const void *packed, const uint8_t *w, int K, int N, int M, float *out,
                                    int64_t ldo, int32_t *nonfinite, int num_cus, int splits, void *partials,
                                    hipStream_t s, const float *rsc = nullptr);

// Range-safe packing of the fp32 entry points' activations into a packing
// area of pack_area_bytes(M, K) bytes (16-byte aligned): the packed fp16
// rows (row stride K) and, 256-byte aligned after them, M row scales
// (pack_area_rsc): a row whose largest |a| would overflow fp16 is packed
// times 2^-e and gets scale 2^e (every other row 1 and the plain packing's
// bits), for the GEMM's epilogue to undo.
size_t pack_area_bytes(int M, int K);
float *pack_area_rsc(void *area, int M, int K);
hipError_t launch_pack_rows(const float *act, int64_t lda, int M, int K, void *area, hipStream_t s);
// The same into a packing (row stride K, 16-byte aligned) and M row scales
// at places of the caller's choosing.
hipError_t launch_pack_rows_to(const float *act, int64_t lda, int M, int K, void *packed, float *rsc,
                               hipStream_t s);

// Rows of a linear holding activations beyond the fp16 range (|a| >=
// 65520), recomputed exactly (EXACT mode's bits) over what a kernel that
// converts fp32 activations itself wrote; other rows are only read.  Needs
// 16-byte aligned activation rows.
hipError_t launch_fixup_rows(const LinearArgs &a, hipStream_t s);
// The same GEMM with a fused epilogue (kind 0 plain, 1 gate-residual,
// 2 SwiGLU with N = 2 glu_h, glu_h % 32 == 0, out [M][ldo >= glu_h],
// 3 fp32 / packed fp16 columns with N % 32 == 0; with split > 0, out 16-byte
// aligned and ldo % 4 == 0).
hipError_t launch_gemm_packed_epi(const void *packed, const uint8_t *w, int K, int N, int M, float *out,
                                  int64_t ldo, int32_t *nonfinite, int num_cus, int kind, const GemmEpi &epi,
                                  hipStream_t s);

// The epilogue (kind 1 or 2) as a separate pass over y [M][ldy] (N columns
// of y; kind 2 writes glu_h of them).
hipError_t launch_epi(const float *y, int64_t ldy, int M, int N, int kind, const GemmEpi &epi, float *out,
                      int64_t ldo, hipStream_t s);
// Kind 3 as separate passes over y [M][ldy] (16-byte aligned, ldy % 4 ==
// 0): columns [0, split) copied to out, the rest through the producer of
// epi.act into epi.pk -- the values the fused epilogue writes.
hipError_t launch_epi_packed(const float *y, int64_t ldy, int M, int N, const GemmEpi &epi, float *out,
                             int64_t ldo, hipStream_t s);

// LayerNorm (no affine, eps inside the square root) + modulation
// x_n * (scale + 1) + shift over rows of H (H % 32 == 0, 16-byte aligned
// rows and vectors); writes fp32 y [rows][ldy] or, with packed != nullptr,
// the packed fp16 activations.
hipError_t launch_norm_mod(const float *x, int64_t ldx, int H, int rows, const float *scale, const float *shift,
                           float eps, float *y, int64_t ldy, void *packed, hipStream_t s);

// Small-M (M <= 16) bandwidth-bound kernel; requires K % 64 == 0,
// lda % 4 == 0, act 16-byte aligned.  Range-safe: rows of tokens with an
// activation beyond the fp16 range come out in EXACT mode's arithmetic
// (inside the kernel when K % 256 == 0, else by launch_fixup_rows after it).
bool gemv_supported(const LinearArgs &a);
hipError_t launch_gemv(const LinearArgs &a, int num_cus, hipStream_t s);

constexpr int kGemvMaxM = 16;

// The small-M kernel over packed fp16 activations (the layout launch_pack
// writes, row stride K): M <= 16, K % 256 == 0, weights and packing under
// 2^31 bytes (gemv_packed_ok adds the packed entry's gemm_packed_ok); rsc:
// row scales of launch_pack_rows, or nullptr.
bool gemv_packed_ok(int M, int K, int N);
hipError_t launch_gemv_packed(const void *packed, const uint8_t *w, int K, int N, int M, float *out, int64_t ldo,
                              int32_t *nonfinite, int num_cus, hipStream_t s, const float *rsc = nullptr);

// Up to kGemvGroupMax small-M linears over one packed activation matrix in
// one launch (M <= 16, K % 256 == 0, K <= 3072, each op's weights under
// 2^31 bytes); the outputs must not overlap one another.
constexpr int kGemvGroupMax = 8;
struct GemvGroupOp {
    const uint8_t *w;
    int N;
    float *out;
    int64_t ldo;
};
bool gemv_group_ok(int M, int K, const GemvGroupOp *ops, int nops);
hipError_t launch_gemv_group(const void *packed, const float *rsc, int K, int M, const GemvGroupOp *ops, int nops,
                             int32_t *nonfinite, int num_cus, hipStream_t s);
// The same straight from fp32 activations, at most kGemvGroupF32MaxM tokens
// (rows 16-byte aligned, lda % 4 == 0, under 2^31 bytes): no packing pass,
// each op's outputs bit for bit those of its own small-M call, rows of
// tokens beyond the fp16 range included (EXACT rows, as the single call).
// launch_gemv runs a single op of at most 4 tokens this way.
constexpr int kGemvGroupF32MaxM = 8;
bool gemv_group_f32_ok(const float *act, int64_t lda, int M, int K);
hipError_t launch_gemv_group_f32(const float *act, int64_t lda, int K, int M, const GemvGroupOp *ops, int nops,
                                 int32_t *nonfinite, int num_cus, hipStream_t s);

// GELU-tanh over [rows][cols] fp32 (cols % 4 == 0, rows 16-byte aligned via
// ld % 4 == 0); the fused form writes packed fp16 activations (pack rules).
hipError_t launch_gelu(const float *x, int64_t ldx, float *y, int64_t ldy, int cols, int rows, hipStream_t s);
hipError_t launch_gelu_pack(const float *act, int64_t lda, int M, int K, void *packed, int64_t ldp,
                            hipStream_t s);
// SwiGLU over act [M][2H] (gate half first) into packed fp16 [M][H] at row
// stride ldp (pack rules with K = 2H for the input).
hipError_t launch_swiglu_pack(const float *act, int64_t lda, int M, int H, void *packed, int64_t ldp,
                              hipStream_t s);

// Packed B1_0 writer over device fp32 weights [N][ldw]; order 0 = numpy's
// np.mean summation, 1 = left to right.
hipError_t launch_quantize(const float *w, int64_t ldw, int K, int N, void *packed, int order, hipStream_t s);

} // namespace b1
