/*
 * bonsai_b1.h — C ABI of the MI355X (gfx950) B1_0 1-bit linear.
 *
 * Drop-in for the B1_0 weight matmul of Juste-Leo2/bonsai.cpp:
 *   out[m][n] = sum_blk fp32(scale[n][blk]) *
 *               sum_{i<32} (bit_i ? +act[m][32*blk+i] : -act[m][32*blk+i])
 * with the packed layout written by convert_to_b1_0_packed.py:21-43:
 * rows are N-major, row n starts at byte n*(K/32)*6, and each 32-weight block
 * is 6 bytes: fp16 scale (little-endian) then the u32 sign word (bit i set ->
 * +scale for element i, clear -> -scale).
 *
 * Everything here is plain C: pointers, sizes and a HIP stream.  Device
 * pointers are HIP device (or managed) addresses on the current device.
 * All compute entry points are stream-ordered and never synchronise the host.
 */
#ifndef BONSAI_B1_H
#define BONSAI_B1_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/diffuser_types.h:10-11 */
#define BONSAI_B1_BLOCK_SIZE 32
#define BONSAI_B1_BLOCK_BYTES 6
/* src/b1_0_kernel.h:32 — "1B1B", how GPU backends recognise the op */
#define BONSAI_B1_MAGIC 0x31423142

/* Op descriptor; replaces bonsai::B1LinearUserData (src/b1_0_kernel.h:31-35).
 * Same field order and sizes: {int magic; int in_dim; int out_dim;}. */
typedef struct B1LinearUserData {
    int magic;
    int in_dim;
    int out_dim;
} B1LinearUserData;

/* Device-resident packed weights; replaces bonsai::B1Weights
 * (src/diffuser_types.h:32-36), whose `data` was a GGML_TYPE_I8 [nbytes,1]
 * tensor.  Here `data` is a hipMalloc'd buffer of out_dim*(in_dim/32)*6
 * bytes, 256-byte aligned. */
typedef struct B1Weights {
    void *data;
    int in_dim;
    int out_dim;
    size_t nbytes;
    int device;
} B1Weights;

/* Status codes.  The reference has none: it abort()s on a non-finite output
 * (src/b1_0_kernel.h:194-198,230-233,279-282) and leaves its preconditions
 * unchecked (K % 32 == 0, act->ne[0] == in_dim). */
enum {
    BONSAI_B1_OK = 0,
    BONSAI_B1_ERR_ARG = 1,       /* bad shape, stride, pointer or mode */
    BONSAI_B1_ERR_HIP = 2,       /* a HIP runtime call failed */
    BONSAI_B1_ERR_NONFINITE = 3, /* output held NaN/Inf (reference: abort) */
    BONSAI_B1_ERR_DEVICE = 4,    /* no usable gfx950 device */
    BONSAI_B1_ERR_NOT_FOUND = 5, /* no tensor of that name in the file */
    BONSAI_B1_ERR_FORMAT = 6,    /* malformed file or not a B1_0 tensor */
    BONSAI_B1_ERR_IO = 7,        /* file could not be opened or mapped */
    BONSAI_B1_ERR_SCRATCH = 8    /* call needs more than the static scratch */
};

/* Arithmetic modes.
 *  AUTO  : FAST numerics; small batches (M <= 16) take the bandwidth-bound
 *          kernel, larger ones the MFMA GEMM.
 *  FAST  : activations rounded to fp16 (RNE), weights expanded to exactly
 *          +-scale in fp16, fp32 MFMA accumulation.  Per-element error vs
 *          the reference <= 1e-2 of max(|y|, rms(y)).  Any finite fp32
 *          activation is accepted by the fp32 entry points: a row whose
 *          largest |act| would overflow fp16 (>= 65520) is packed times a
 *          power of two 2^-e, and its outputs are multiplied by 2^e, which
 *          keeps fp16 relative precision; where the kernel converts
 *          activations itself (no workspace, see below) such a row is
 *          computed again in EXACT arithmetic instead.  Entry points that
 *          take packed fp16 activations get whatever their producer wrote
 *          (its inputs beyond 65504 are +-inf there).
 *  EXACT : fp32 VALU in the reference's scalar summation order
 *          (src/b1_0_kernel.h:253-277); bit-identical to that path.
 *  GEMM / GEMV : FAST numerics with the kernel forced (for benchmarks). */
enum {
    BONSAI_B1_MODE_AUTO = 0,
    BONSAI_B1_MODE_FAST = 1,
    BONSAI_B1_MODE_EXACT = 2,
    BONSAI_B1_MODE_GEMM = 3,
    BONSAI_B1_MODE_GEMV = 4
};

/*
 * The B1_0 linear on device buffers; the compute of the reference CPU custom
 * op b1_linear_f32_f32(dst, ith, nth, userdata) (src/b1_0_kernel.h:37-288),
 * done for all rows by one stream-ordered launch.
 *   act      [batch][lda] fp32, rows of in_dim used (reference: src[0], rows
 *            contiguous with stride in_dim, src/b1_0_kernel.h:103)
 *   w        packed B1_0 [out_dim][in_dim/32*6] bytes (reference: src[1])
 *   out      [batch][ldo] fp32, columns [0,out_dim) written
 *            (reference: out[b*out_dim + r], src/b1_0_kernel.h:200-203)
 *   nonfinite  optional device int32 counter; every non-finite output adds 1
 *            (NULL: not counted).  Replaces the reference's abort().
 * Preconditions checked on the host: in_dim % 32 == 0, in_dim, out_dim > 0,
 * batch >= 0, lda >= in_dim, ldo >= out_dim, non-NULL pointers.  Not
 * checked (as in the reference, whose graph never aliases them): out must
 * not overlap act or w; the small-M and EXACT kernels read act while other
 * work-groups write out.
 * Returns BONSAI_B1_OK or an error code; never blocks the host.
 */
int bonsai_b1_linear_f32(const float *act, int64_t lda, const void *w,
                         int in_dim, int out_dim, int batch, float *out,
                         int64_t ldo, int mode, int32_t *nonfinite,
                         hipStream_t stream);

/*
 * The GEMM kernels pack the activations to fp16 once (with the row scales
 * of the range-safe packing, and, for shapes that split along K, the split
 * partials after them) into a device workspace of
 * bonsai_b1_workspace_bytes(batch, in_dim, out_dim, mode) bytes (0 when the
 * call needs none: EXACT, and small batches, whose kernel converts the
 * activations itself).  bonsai_b1_linear_f32 keeps library-owned workspaces
 * per (device, stream) -- per calling thread for hipStreamPerThread, whose
 * one handle value names each thread's own stream -- grown on demand with
 * hipMalloc; while a stream is
 * being captured it never allocates and, lacking a large enough buffer,
 * runs the kernel variant that converts activations tile by tile.  A buffer
 * handed out during a capture is pinned, since the graph holds its address:
 * the library never frees or replaces it (growth allocates another one) and
 * later calls on the capture stream may share it, so replay such a graph on
 * that stream (or ordered with it).  bonsai_b1_linear_f32_ws takes the
 * caller's workspace instead (NULL or too small selects that same variant)
 * and never allocates.  The variants agree bit for bit, except (a) for a
 * shape split along K, which the variant without room for the partials sums
 * unsplit (the same values up to the order of the K summation), and (b) for
 * rows beyond the fp16 range, which the converting variant computes in
 * EXACT arithmetic.  Concurrent calls on one stream are ordered; calls on
 * different streams use different workspaces.  A workspace is found by the
 * stream's handle, so synchronize a stream before destroying it while calls
 * on it may still run: a stream created later can get the same handle.
 */
size_t bonsai_b1_workspace_bytes(int batch, int in_dim, int out_dim, int mode);

int bonsai_b1_linear_f32_ws(const float *act, int64_t lda, const void *w,
                            int in_dim, int out_dim, int batch, float *out,
                            int64_t ldo, int mode, int32_t *nonfinite,
                            void *workspace, size_t workspace_bytes,
                            hipStream_t stream);

/* Frees every library-owned workspace (all devices), pinned ones included:
 * destroy graphs captured with the library's workspace first.  Waits for
 * the device. */
void bonsai_b1_release_workspaces(void);

/*
 * bonsai_b1_linear_f32 for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  No counterpart in the reference (its CPU op needs no
 * workspace).  Same arguments, kernels and results, bit for bit, as
 * bonsai_b1_linear_f32; the workspace those kernels use (the fp16 packing
 * of the activations and the split-K partials) is a static device array of
 * BONSAI_B1_NOALLOC_SCRATCH_BYTES that the library holds on each device it
 * runs on until the process ends.  Never calls hipMalloc or hipFree.
 * Returns BONSAI_B1_ERR_SCRATCH, launching nothing, when the kernel the
 * call runs needs more than that (for aligned activations,
 * bonsai_b1_workspace_bytes(batch, in_dim, out_dim, mode) >
 * BONSAI_B1_NOALLOC_SCRATCH_BYTES; activations that are not 16-byte
 * aligned, or lda % 4 != 0, run EXACT mode, which needs none, at any
 * size).  Every call on a device shares that
 * device's array and leaves its contents behind: calls that overlap in time
 * on one device (other streams, other threads) race and must be serialised
 * by the caller; calls on one stream are ordered.
 */
#define BONSAI_B1_NOALLOC_SCRATCH_BYTES (32u << 20)
int bonsai_b1_linear_f32_noalloc(const float *act, int64_t lda, const void *w,
                                 int in_dim, int out_dim, int batch,
                                 float *out, int64_t ldo, int mode,
                                 int32_t *nonfinite, hipStream_t stream);

/*
 * The FAST GEMM in two halves, for a producer of activations that can emit
 * them in fp16 once (the LayerNorm + modulation feeding each linear,
 * src/diffuser_graph.cpp:347-352,444-448,479-480) and for linears that
 * share one input (q/k/v of a block, src/diffuser_graph.cpp:354-361).
 * Together they compute what bonsai_b1_linear_f32 computes in FAST mode for
 * in_dim % 384 == 0; the reference's single op b1_linear_f32_f32
 * (src/b1_0_kernel.h:37) has no such split.
 *
 * Packed activations: row m is in_dim/2 little-endian u32 words; word
 * 16*j + d of the row holds fp16(act[m][32j+d]) in its low half and
 * fp16(act[m][32j+d+16]) in its high half (round to nearest even), for
 * block j < in_dim/32 and d < 16.  Total bonsai_b1_packed_act_bytes() bytes.
 */
size_t bonsai_b1_packed_act_bytes(int batch, int in_dim);

/* act [batch][lda] fp32 (lda % 4 == 0, 16-byte aligned; in_dim % 32 == 0)
 * -> packed (16-byte aligned, bonsai_b1_packed_act_bytes bytes).
 * |act| must stay below 65504 (fp16 range). */
int bonsai_b1_pack_act_f16(const float *act, int64_t lda, int in_dim,
                           int batch, void *packed, hipStream_t stream);

/* The same into a column range of wider packed activations: packed rows of
 * ldp fp16 elements (ldp >= in_dim, ldp % 8 == 0), `packed` pointing at
 * the range's first column (a multiple of 32, so 64-byte aligned within
 * the row).  Producers of adjacent ranges build the packed input of a GEMM
 * over concatenated activations, such as the single-stream block's
 * linear2 over [attention output | GELU(MLP)] (src/diffuser_graph.cpp:
 * 533-536), without an fp32 concatenation.  No reference counterpart
 * (ggml_concat there). */
int bonsai_b1_pack_act_f16_ld(const float *act, int64_t lda, int in_dim,
                              int batch, void *packed, int64_t ldp,
                              hipStream_t stream);

/* out[m][n] for packed activations (in_dim % 384 == 0, packed 16-byte
 * aligned, w 4-byte aligned); same outputs as bonsai_b1_linear_f32 in
 * FAST/GEMM mode on the activations that were packed, or, for batch <= 16
 * with in_dim % 256 == 0, as its small-M (GEMV) mode, bit for bit (for
 * activations within the fp16 range).  A shape that bonsai_b1_linear_f32
 * splits along K is split the same way, with the partials in the library's
 * per-stream workspace (allocated on demand like bonsai_b1_linear_f32's;
 * under capture without one it runs unsplit).  The _ws form takes the
 * caller's workspace of bonsai_b1_linear_packed_workspace_bytes bytes
 * (0: none needed; NULL or smaller: unsplit) and never allocates. */
int bonsai_b1_linear_packed_f16(const void *packed_act, const void *w,
                                int in_dim, int out_dim, int batch,
                                float *out, int64_t ldo, int32_t *nonfinite,
                                hipStream_t stream);
size_t bonsai_b1_linear_packed_workspace_bytes(int batch, int in_dim,
                                               int out_dim);
int bonsai_b1_linear_packed_f16_ws(const void *packed_act, const void *w,
                                   int in_dim, int out_dim, int batch,
                                   float *out, int64_t ldo,
                                   int32_t *nonfinite, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/*
 * The two halves of bonsai_b1_linear_f32's range-safe FAST path, for callers
 * that pack an input once for several linears (q/k/v of a block,
 * src/diffuser_graph.cpp:354-361) and still take any finite activation.
 * _pack_act_f16_scaled writes the packing of bonsai_b1_pack_act_f16
 * (row stride in_dim, same requirements) of act[m][:] * 2^-e[m] and
 * row_scale[m] = 2^e[m] (batch floats, 4-byte aligned): e[m] = 0 for a row
 * within the fp16 range (the same bits as bonsai_b1_pack_act_f16), else the
 * smallest shift that brings its largest |act| below 2^15.
 * _linear_packed_f16_scaled is bonsai_b1_linear_packed_f16 with row m's
 * outputs multiplied by row_scale[m] (exact: powers of two); together they
 * give bonsai_b1_linear_f32's FAST results bit for bit (for batch <= 16 on
 * rows within the fp16 range: bonsai_b1_linear_f32 computes the others in
 * EXACT arithmetic there).  No reference
 * counterpart (the reference's single op has no such split).
 */
int bonsai_b1_pack_act_f16_scaled(const float *act, int64_t lda, int in_dim,
                                  int batch, void *packed, float *row_scale,
                                  hipStream_t stream);
int bonsai_b1_linear_packed_f16_scaled(const void *packed_act,
                                       const float *row_scale, const void *w,
                                       int in_dim, int out_dim, int batch,
                                       float *out, int64_t ldo,
                                       int32_t *nonfinite, hipStream_t stream);

/*
 * A sequence of B1_0 linears on one stream: the linear dispatch of a
 * diffusion step (the b1 lambda at src/diffuser_graph.cpp:277-281 and its
 * call sites, :354-361,434-457,482,536), run in the order given.  Each op is
 * what bonsai_b1_linear would run for it.  Consecutive ops that read the
 * same activations (same act, lda, batch and in_dim -- q/k/v of a block,
 * :354-361) share one fp16 packing of them, so only the first pays the pack
 * pass; when their weights are also adjacent row ranges of one buffer
 * (bonsai_b1_weights_concat) and their outputs adjacent column ranges with
 * one row stride, they run as a single GEMM over the concatenated rows.
 * Up to 8 consecutive small-batch ops (batch <= 16, in_dim % 256 == 0,
 * in_dim <= 3072, no epilogue) on the same activations -- the modulation
 * projections of a step, all over vec_silu at one token (:308-311,
 * 470-471,548) -- run as one launch when their outputs lie apart from
 * those activations and from one another: from the fp32 rows at batch <= 8
 * (no workspace), over one packing above; each op's outputs are those of
 * its own small-batch call, bit for bit (above batch 8 for activations
 * within the fp16 range).  workspace: device buffer of
 * bonsai_b1_linear_batch_workspace_bytes bytes, or NULL for the library's
 * per-stream workspace.  On an invalid op
 * nothing is launched and *bad_op (if given) receives its index.
 * No reference counterpart: the reference builds one ggml node per linear.
 */
typedef struct bonsai_b1_linear_op {
    const float *act;    /* fp32 [batch][lda] */
    int64_t lda;
    const B1Weights *w;  /* device-resident weights (in_dim, out_dim) */
    float *out;          /* fp32 [batch][ldo] */
    int64_t ldo;
    int batch;
} bonsai_b1_linear_op;

size_t bonsai_b1_linear_batch_workspace_bytes(const bonsai_b1_linear_op *ops,
                                              int n_ops, int mode);

int bonsai_b1_linear_batch(const bonsai_b1_linear_op *ops, int n_ops,
                           int mode, int32_t *nonfinite, void *workspace,
                           size_t workspace_bytes, int *bad_op,
                           hipStream_t stream);

/*
 * bonsai_b1_linear_batch with an epilogue per op (bonsai_b1_epilogue,
 * declared below): a step's linears and the element-wise ops the graph puts
 * right after them (SwiGLU after FF-in, the gated residual add after
 * out-projections and FF-out) in one call.  Ops with an epilogue are not
 * merged into N-concatenated GEMMs; an epilogue that cannot be fused (EXACT
 * mode, small batch, K % 384 != 0) runs as a separate pass over the
 * linear's output in the workspace.
 */
struct bonsai_b1_epilogue;
typedef struct bonsai_b1_linear_op_epi bonsai_b1_linear_op_epi;
size_t bonsai_b1_linear_batch_epi_workspace_bytes(const bonsai_b1_linear_op_epi *ops, int n_ops, int mode);
int bonsai_b1_linear_batch_epi(const bonsai_b1_linear_op_epi *ops, int n_ops,
                               int mode, int32_t *nonfinite, void *workspace,
                               size_t workspace_bytes, int *bad_op,
                               hipStream_t stream);

/*
 * Builder-style call; replaces bonsai::b1_linear(ctx, act, w, n_threads, ud)
 * (src/b1_0_kernel.h:290-300): fills ud from w (magic, in_dim, out_dim) and
 * runs the op for `batch` rows of act (the reference's act->ne[1]).
 * ud may be NULL.
 */
int bonsai_b1_linear(const float *act, const B1Weights *w, int batch,
                     float *out, B1LinearUserData *ud, int mode,
                     int32_t *nonfinite, hipStream_t stream);

/*
 * ggml custom-op callback over a device-side stand-in tensor; same signature
 * and meaning as the reference's b1_linear_f32_f32 (src/b1_0_kernel.h:37):
 * dst->src[0] = act, dst->src[1] = packed weights, the userdata holds
 * {magic, in_dim, out_dim}.  Task ith == 0 runs the whole op on the calling
 * thread's current stream (hipStreamPerThread) and synchronises it; other
 * tasks return at once.  When AUTO mode's outputs hold a non-finite value
 * the op runs again in EXACT mode (the reference's scalar arithmetic); like
 * the reference, a non-finite output of that prints "B1_FATAL_OUT" to
 * stderr and abort()s.  Returns nothing.
 */
typedef struct bonsai_b1_tensor {
    int64_t ne[4];                    /* ne[0] = in_dim/out_dim, ne[1] = rows */
    size_t nb[4];                     /* byte strides; nb[1] = row stride */
    struct bonsai_b1_tensor *src[2];  /* act, packed weights */
    void *data;                       /* device pointer */
} bonsai_b1_tensor;

void bonsai_b1_linear_f32_f32(bonsai_b1_tensor *dst, int ith, int nth,
                              void *userdata);

/*
 * Deferred checking for bonsai_b1_linear_f32_f32 on the calling thread (no
 * counterpart in the reference, whose CPU op finishes before the callback
 * returns; for graph runners that do not want a host synchronisation per
 * op).  After bonsai_b1_callback_defer(1) the callback runs each op in AUTO
 * mode on hipStreamPerThread and returns without synchronising: no EXACT
 * rerun, no abort; the op's non-finite outputs are added to a counter of
 * this thread and device (the first deferred op on a device allocates it,
 * so run one before capturing a graph).  bonsai_b1_callback_finish
 * synchronises the thread's stream once, stores that count in *count
 * (count may be NULL), resets it, and returns BONSAI_B1_ERR_NONFINITE when
 * it was non-zero -- the caller then aborts as the reference would have
 * after the op -- else BONSAI_B1_OK.  bonsai_b1_callback_defer(0) restores
 * the per-op behaviour.  AUTO mode is range-safe: a finite activation never
 * makes an output non-finite that the reference's fp32 sums keep finite,
 * short of sums near FLT_MAX, so skipping the EXACT rerun changes no
 * finite result.
 */
int bonsai_b1_callback_defer(int on);
int bonsai_b1_callback_finish(int32_t *count);

/*
 * Weight residency; replaces load_b1 (src/diffuser.cpp:39-50, memcpy of the
 * safetensors U8 [out_dim, in_dim/32*6] tensor into a ggml I8 tensor) and the
 * deferred upload of the WebGPU driver (src/diffuser_webgpu.cpp:49-64,
 * 246-250).  Allocates device memory on the current device and enqueues the
 * host->device copy of nbytes on `stream`.  The host buffer must stay valid
 * until the stream has passed the copy.  nbytes must equal
 * out_dim*(in_dim/32)*6.
 */
int bonsai_b1_weights_upload(const void *host_packed, size_t nbytes,
                             int in_dim, int out_dim, hipStream_t stream,
                             B1Weights *out);
int bonsai_b1_weights_free(B1Weights *w);

/*
 * One device copy of several weight tensors of the same in_dim, rows back
 * to back (out_dim = sum of the parts'): the N-concatenated weights of
 * q, k and v (src/diffuser_graph.cpp:354-361) for one GEMM.  A part's rows
 * stay a contiguous range, so a B1Weights {data + offset, in_dim, rows}
 * names it; bonsai_b1_linear_batch runs consecutive ops over such adjacent
 * ranges, with adjacent output columns, as one GEMM.  Free only the
 * returned whole.  No reference counterpart (the reference keeps q, k, v
 * separate).
 */
int bonsai_b1_weights_concat(const B1Weights *parts, int n_parts,
                             hipStream_t stream, B1Weights *out);

/*
 * Fused epilogues of the graph around a linear (src/diffuser_graph.cpp):
 *  - BONSAI_B1_EPI_GATE_RESIDUAL: out = residual + gate[n] * y, the
 *    modulation-gated residual add after out-projections and FF-out
 *    (:441-442,459-460,538): h = h + gate * y, an fp32 multiply then an fp32
 *    add.  residual [batch][ldr] may be out itself (same rows, ldr == ldo).
 *  - BONSAI_B1_EPI_SWIGLU: the linear's out_dim = 2H outputs are [gate |
 *    value] (weights rows [0, H) then [H, 2H)); out[m][j] = silu(y[m][j]) *
 *    y[m][H + j], H columns (ggml_swiglu on FF-in, :453-456, 228).
 *    H % 32 == 0; silu(x) = x / (1 + exp(-x)) in fp32.
 *  - BONSAI_B1_EPI_PACKED: the output of bonsai_b1_linear_packed_f16_to_packed
 *    (declared below): columns [0, split) of y as fp32 in out (ldo >= split;
 *    out may be NULL when split == 0), columns [split, out_dim) through
 *    `act` into the packed fp16 activations `packed` (row stride ldp), with
 *    that entry's requirements.
 * The non-finite counter counts the linear's own outputs y, as the
 * reference's abort checks them (src/b1_0_kernel.h:194-198).
 * No reference counterpart: the reference runs these as separate ggml ops.
 */
enum {
    BONSAI_B1_EPI_NONE = 0,
    BONSAI_B1_EPI_GATE_RESIDUAL = 1,
    BONSAI_B1_EPI_SWIGLU = 2,
    BONSAI_B1_EPI_PACKED = 3
};
typedef struct bonsai_b1_epilogue {
    int kind;
    const float *gate;     /* GATE_RESIDUAL: [out_dim], device */
    const float *residual; /* GATE_RESIDUAL: [batch][ldr], device */
    int64_t ldr;
    int split;             /* PACKED: fp32 columns, a multiple of 32 */
    int act;               /* PACKED: BONSAI_B1_ACT_* */
    void *packed;          /* PACKED: packed fp16 output, device */
    int64_t ldp;           /* PACKED: its row stride in fp16 elements */
} bonsai_b1_epilogue;

/* An op of bonsai_b1_linear_batch_epi: the linear and its epilogue. */
struct bonsai_b1_linear_op_epi {
    bonsai_b1_linear_op op;
    bonsai_b1_epilogue epi;
};

/* bonsai_b1_linear_packed_f16 with the epilogue fused into the GEMM. */
int bonsai_b1_linear_packed_f16_epi(const void *packed_act, const void *w,
                                    int in_dim, int out_dim, int batch,
                                    float *out, int64_t ldo,
                                    const bonsai_b1_epilogue *epi,
                                    int32_t *nonfinite, hipStream_t stream);

/*
 * bonsai_b1_linear_packed_f16 whose output feeds the next B1_0 linear
 * directly: columns [0, split) of y are stored as fp32 in out (row stride
 * ldo), and columns [split, out_dim) pass through `act` and are stored as
 * packed fp16 activations in packed_out (row stride ldp fp16 elements, the
 * layout of bonsai_b1_pack_act_f16_ld):
 *  - BONSAI_B1_ACT_NONE / _GELU_TANH: column split + j -> packed column j;
 *  - BONSAI_B1_ACT_SWIGLU: columns [split, out_dim) are [gate | value] of
 *    H = (out_dim - split) / 2 each (weight rows split.. then split + H..),
 *    packed column j = silu(y[split + j]) * y[split + H + j].
 * The results equal bonsai_b1_linear_packed_f16 followed by
 * bonsai_b1_pack_act_f16_ld, bonsai_b1_gelu_tanh_pack_f16_ld or
 * bonsai_b1_swiglu_pack_f16_ld over those columns, bit for bit, without
 * the fp32 round trip.  It fuses the reference single block's linear1
 * (src/diffuser_graph.cpp:482-488: q/k/v columns to attention, MLP columns
 * through mlp_act = ggml_swiglu, :227-229, into the second half of
 * ggml_concat's input to to_out, :531-534) and the double block's FF-in
 * (:450-456).  The non-finite counter counts y.
 * split and out_dim multiples of 32 (64 for SwiGLU, both split and
 * out_dim - split); in_dim % 384 == 0; split > 0: out 16-byte aligned,
 * ldo >= split, ldo % 4 == 0; packed columns: packed_out 16-byte aligned,
 * ldp >= their count, ldp % 8 == 0; the outputs apart from packed_act and
 * from each other.  Always the 128-row GEMM tile, also for a few rows.
 * No reference counterpart as one op (the reference runs separate ggml ops).
 */
enum {
    BONSAI_B1_ACT_NONE = 0,
    BONSAI_B1_ACT_GELU_TANH = 1,
    BONSAI_B1_ACT_SWIGLU = 2
};
int bonsai_b1_linear_packed_f16_to_packed(const void *packed_act, const void *w,
                                          int in_dim, int out_dim, int batch,
                                          float *out, int64_t ldo, int split,
                                          int act, void *packed_out,
                                          int64_t ldp, int32_t *nonfinite,
                                          hipStream_t stream);

/* fp32 activations, any mode.  Where the packed FAST GEMM runs, the
 * epilogue is fused into it; elsewhere (EXACT, small batch, K % 384 != 0)
 * the linear writes y into the workspace and a separate pass applies the
 * same fp32 arithmetic.  workspace: bonsai_b1_linear_epi_workspace_bytes
 * bytes, or NULL for the library's per-stream workspace (which is never
 * allocated while the stream is being captured: a capture needs a large
 * enough library workspace from an earlier call, or the caller's, or the
 * call returns BONSAI_B1_ERR_ARG). */
size_t bonsai_b1_linear_epi_workspace_bytes(int batch, int in_dim,
                                            int out_dim, int kind, int mode);
int bonsai_b1_linear_epi_f32(const float *act, int64_t lda, const void *w,
                             int in_dim, int out_dim, int batch, float *out,
                             int64_t ldo, const bonsai_b1_epilogue *epi,
                             int mode, int32_t *nonfinite, void *workspace,
                             size_t workspace_bytes, hipStream_t stream);

/*
 * The producer of the linears' activations: LayerNorm without affine
 * (ggml_norm, eps inside the square root) and the modulation
 * x_n * (scale + 1) + shift, as the reference graph computes before each
 * block's first linears (src/diffuser_graph.cpp:347-352, 444-448,
 * 479-480).  Per row of H: mean and variance accumulated in double (the
 * ggml CPU norm's accumulators), every other step an fp32 op.  The _pack
 * form writes the packed fp16 activations bonsai_b1_linear_packed_f16
 * reads, so the linear that follows runs without its own pack pass.
 * H % 32 == 0; x, scale, shift, y 16-byte aligned; ldx, ldy % 4 == 0.
 * No reference counterpart as one op (three ggml ops and a conversion).
 */
int bonsai_b1_norm_mod_f32(const float *x, int64_t ldx, int H, int rows,
                           const float *scale, const float *shift, float eps,
                           float *y, int64_t ldy, hipStream_t stream);
int bonsai_b1_norm_mod_pack_f16(const float *x, int64_t ldx, int H, int rows,
                                const float *scale, const float *shift,
                                float eps, void *packed, hipStream_t stream);

/*
 * GELU with the tanh approximation, 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715
 * x^3))), between the up- and down-projections of the Flux MLP workload.
 * Not a reference op: the reference MLP uses SwiGLU
 * (src/diffuser_graph.cpp:453,456).  fp32 [rows][ldx] -> fp32 [rows][ldy]
 * (x == y allowed); cols % 4 == 0, ldx and ldy multiples of 4, 16-byte
 * aligned pointers.
 */
int bonsai_b1_gelu_tanh_f32(const float *x, int64_t ldx, float *y,
                            int64_t ldy, int cols, int rows,
                            hipStream_t stream);

/* GELU-tanh fused with bonsai_b1_pack_act_f16: packed fp16 activations of
 * gelu(act), ready for bonsai_b1_linear_packed_f16.  Same requirements as
 * bonsai_b1_pack_act_f16. */
int bonsai_b1_gelu_tanh_pack_f16(const float *act, int64_t lda, int in_dim,
                                 int batch, void *packed, hipStream_t stream);
/* ... into a column range of wider packed activations, as
 * bonsai_b1_pack_act_f16_ld. */
int bonsai_b1_gelu_tanh_pack_f16_ld(const float *act, int64_t lda,
                                    int in_dim, int batch, void *packed,
                                    int64_t ldp, hipStream_t stream);

/* SwiGLU fused with the packing: replaces ggml_swiglu (mlp_act,
 * src/diffuser_graph.cpp:227-229) feeding a B1_0 linear.  act [batch][lda]
 * holds 2*hidden columns per row, gates first; the packed output holds
 * hidden columns, silu(a[m][j]) * a[m][hidden + j] in fp32 (no
 * contraction) rounded to fp16, the same values as the SwiGLU epilogue of
 * bonsai_b1_linear_packed_f16_epi.  hidden % 32 == 0; the input as for
 * bonsai_b1_pack_act_f16 over 2*hidden columns; ldp and `packed` as for
 * bonsai_b1_pack_act_f16_ld (the plain form writes rows of hidden). */
int bonsai_b1_swiglu_pack_f16(const float *act, int64_t lda, int hidden,
                              int batch, void *packed, hipStream_t stream);
int bonsai_b1_swiglu_pack_f16_ld(const float *act, int64_t lda, int hidden,
                                 int batch, void *packed, int64_t ldp,
                                 hipStream_t stream);

/*
 * The B1_0 writer on the device; replaces quantize_b1_0 of
 * convert_to_b1_0_packed.py:21-43 and of tests/c_ops/test_b1_linear.cpp:
 * 129-163.  w: fp32 [out_dim][ldw] device weights (ldw >= in_dim,
 * in_dim % 32 == 0); packed: device buffer of out_dim*(in_dim/32)*6 bytes,
 * 2-byte aligned.  Per 32-weight block: scale = fp16(mean |w|) (round to
 * nearest even), bit i set when w_i >= 0.  order selects which reference
 * writer's float32 summation is reproduced bit for bit (they differ by one
 * fp16 ulp on rare ties).
 */
enum {
    BONSAI_B1_SUM_NUMPY = 0,      /* np.mean, convert_to_b1_0_packed.py */
    BONSAI_B1_SUM_SEQUENTIAL = 1  /* left to right, the C++ test writer */
};
int bonsai_b1_quantize_f32(const float *w, int64_t ldw, int in_dim,
                           int out_dim, void *packed, int order,
                           hipStream_t stream);

/*
 * Weight residency from a .safetensors file; replaces load_b1
 * (src/diffuser.cpp:39-50) over the reader of src/safetensors.h:39-76.
 * The tensor `name` must be U8 (or I8) [out_dim, in_dim/32*6], as
 * convert_to_b1_0_packed.py writes it.  One tensor through
 * bonsai_b1_safetensors_open / _load / _close: the file is mapped
 * read-only and the call returns once the copy has completed.  Errors:
 * ERR_IO (open/map), ERR_NOT_FOUND, ERR_FORMAT (header, dtype, shape or
 * offsets inconsistent).  For many tensors of one file, open it once.
 */
int bonsai_b1_weights_load_safetensors(const char *path, const char *name,
                                       hipStream_t stream, B1Weights *out);

/* The same lookup without a device: dimensions of tensor `name` and where
 * its bytes lie in the file.  Any output pointer may be NULL. */
int bonsai_b1_safetensors_info(const char *path, const char *name,
                               int *in_dim, int *out_dim,
                               uint64_t *data_offset, uint64_t *nbytes);

/*
 * An open .safetensors file, for loading a whole model: the file is mapped
 * once and its header parsed once, as bonsai::SafetensorsFile
 * (src/safetensors.h:27-90: open, find, tensors()) holds it, instead of
 * once per tensor.  open: ERR_IO (open/map), ERR_FORMAT (header).  count
 * and name enumerate every tensor of the header (B1_0 or not) in header
 * order; name returns NULL past the end, and the string lives as long as
 * the handle.  find is bonsai_b1_safetensors_info on the open file.  A
 * handle may be used from one thread at a time.
 */
typedef struct bonsai_b1_safetensors bonsai_b1_safetensors;
int bonsai_b1_safetensors_open(const char *path, bonsai_b1_safetensors **out);
void bonsai_b1_safetensors_close(bonsai_b1_safetensors *f);
int bonsai_b1_safetensors_count(const bonsai_b1_safetensors *f);
const char *bonsai_b1_safetensors_name(const bonsai_b1_safetensors *f, int i);
int bonsai_b1_safetensors_find(const bonsai_b1_safetensors *f,
                               const char *name, int *in_dim, int *out_dim,
                               uint64_t *data_offset, uint64_t *nbytes);

/*
 * Weight residency for n B1_0 tensors of an open file, on the current
 * device; replaces load_b1 (src/diffuser.cpp:39-50) applied tensor by
 * tensor.  Every name is checked before anything is allocated (errors as
 * bonsai_b1_safetensors_find).  Each tensor gets its own device allocation
 * (free with bonsai_b1_weights_free).  The bytes pass through pinned host
 * buffers held by the handle (up to 3 x 16 MB, allocated on first use):
 * host threads copy a piece out of the mapping while the DMA engine moves
 * the previous pieces on `stream`.  Returns once every copy has completed;
 * on any error nothing stays allocated and out[] is zeroed.
 */
int bonsai_b1_safetensors_load(bonsai_b1_safetensors *f,
                               const char *const *names, int n,
                               hipStream_t stream, B1Weights *out);

/* Human-readable text for a status code (static storage). */
const char *bonsai_b1_status_string(int status);

/* Library version, major*10000 + minor*100 + patch. */
int bonsai_b1_version(void);

#ifdef __cplusplus
}
#endif
#endif /* BONSAI_B1_H */
