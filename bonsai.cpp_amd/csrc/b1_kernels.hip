// B1_0 1-bit linear kernels for MI355X (gfx950, CDNA4, wave64).
//
// Arithmetic being reproduced (src/b1_0_kernel.h:37-288 of the reference):
//   out[m][n] = sum_blk fp32(scale[n][blk]) *
//               sum_{i<32} (bit_i ? +a[m][32 blk + i] : -a[m][32 blk + i])
// Packed block (convert_to_b1_0_packed.py:21-43): bytes 0-1 fp16 scale,
// bytes 2-5 little-endian u32 sign word; row n starts at byte n*(K/32)*6.
//
// Three kernels:
//  * b1_exact_kernel — fp32 VALU, the reference's scalar summation order
//    (src/b1_0_kernel.h:253-277) with contraction off: bit-identical output.
//  * b1_gemm_kernel  — wide-tile MFMA GEMM for large M over activations
//    packed to fp16 once (b1_pack_act_kernel) and streamed global -> LDS
//    directly; each weight block is expanded in registers to fp16 +-scale
//    (exact: a sign flip of an fp16 value), so the per-block scale rides
//    inside the MFMA operand and no per-block rescale of fp32 partial sums
//    is needed.  b1_gemm_fused_kernel is the same GEMM converting fp32
//    activations while staging each tile (used when no workspace is given).
//  * b1_gemv_kernel  — small M (<= 16): persistent work-groups, split-K over
//    the waves of a work-group, activations held in registers, packed
//    weights streamed once from HBM; MFMA 16x16x32 with M padded to 16.
//
// K-slot pairing shared by both MFMA kernels.  Inside a 32-element block,
// fp16 dword d (d = 0..15) holds elements (d, d+16).  On the weight side the
// two sign bits for dword d are then bits d and d+16 of the sign word, which
// one left shift by (15 - d) lands on bits 15 and 31 — the two fp16 sign bits
// — so a single three-input bit op against the replicated scale builds the
// pair: sign = scale sign XOR (NOT bit), i.e. bit 1 -> +scale and bit 0 ->
// -scale exactly as in the reference, for negative scales too.  The
// activation side is written in the same pairing when it is packed to fp16.
// Any consistent permutation of K inside the MFMA leaves the dot product
// unchanged.
#include <hip/hip_runtime.h>

#include <mutex>

#include "b1_internal.h"

namespace b1 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kSignPair = 0x80008000u;

// Bits of m: ~(x ^ y); other bits: y.  One v_bitop3_b32, whose 8-bit table
// is indexed by (x_bit << 2) | (m_bit << 1) | y_bit: 0xa6 = {0,1,1,0,0,1,0,1}
// for indices 0..7.  Through the compiler builtin, not inline asm: the
// compiler must see the VALU write, or it cannot insert the wait states an
// MFMA reading the result as a source operand needs (an MFMA issued too
// soon after an asm-hidden write read stale operands here).
__device__ __forceinline__ uint32_t xnor_sel(uint32_t m, uint32_t x, uint32_t y) {
    return __builtin_amdgcn_bitop3_b32(x, m, y, 0xa6);
}

// (lo, hi) -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    float2v v = {lo, hi};
    half2v h = __builtin_convertvector(v, half2v);
    return __builtin_bit_cast(uint32_t, h);
}

// fp32 -> fp16 bits of one value, rounded once from the fp32 value: the
// empty asm keeps the compiler from folding the multiply that produced x
// into the conversion (v_fma_mixlo_f16 rounds the exact product to fp16
// once, which differs from the producer passes' fp32-then-fp16 rounding in
// the rare products an fp32 rounding puts on an fp16 midpoint).
__device__ __forceinline__ uint16_t half_bits(float x) {
    asm("" : "+v"(x));
    return (uint16_t)pack_f16(x, 0.0f);
}

// (lo, hi) -> packed fp16 pair, each rounded once from its fp32 value (the
// fold half_bits keeps out, for two values).
__device__ __forceinline__ uint32_t pack_f16_rounded(float lo, float hi) {
    asm("" : "+v"(lo), "+v"(hi));
    return pack_f16(lo, hi);
}

// max(m, |a|, |b|) in one v_max3_f32: the running largest magnitude of the
// activations a lane converts, against fp16's range (a quiet NaN operand is
// passed over, as IEEE maxNum does: a NaN does not count as out of range).
__device__ __forceinline__ float absmax3(float m, float a, float b) {
    float r;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}
// fp32 magnitudes from this on round to fp16 infinity
constexpr float kF16Overflow = 65520.0f;

// s_waitcnt vmcnt(N) leaving expcnt and lgkmcnt alone (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Waits for this wave's LDS operations only (vmcnt and expcnt left open).
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}

// Work-group barrier that does not drain outstanding global->LDS loads
// (__syncthreads() would add s_waitcnt vmcnt(0) while LDS-DMA is pending).
// Each wave waits for its own loads with wait_vmcnt<> before arriving.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Global -> LDS copies without VGPR staging.  `lds` must be wave-uniform
// (it goes through M0).  Lane i's 16 bytes land at lds + 16 i; 12-byte
// loads also land at lds + 16 i (a 16-byte lane stride, measured on gfx950
// for the global and the buffer forms), leaving 4 bytes untouched per lane.
// Kept as plain device functions: a kernel template that calls these
// builtins directly loses its host-side launch stub.
// global_load_lds_dword: lane i's 4 bytes land at lds + 4 i.  The compiler
// treats this global form as a FLAT access that may touch LDS, and with one
// in a kernel it makes every LDS wait of that kernel a full lgkmcnt(0).  In
// the GEMM (its row-scale copy) the buffer form instead gives waits that
// count only the reads a step needs, and it measured no faster (252.9-253.4
// vs 253.1 us at M=4096 K=3072 N=12288, 0.3-0.6 % slower on four other
// shapes, bit-identical): the fragment reads' latency is already covered.
__device__ __forceinline__ void dma_lds4(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds, 4, 0, 0);
}

// Raw buffer loads with range checking (offsets at or past num_records read
// zeros); word 3 of the resource for gfx9-family raw buffers.
constexpr int kBufferFlags = 0x00020000;
// Cache policy of the GEMM's full-tile output stores: the default.  Each
// 16-byte store covers 32 rows x 32 bytes, a quarter of each 128-byte line,
// and L2 merges the four quarters before the line goes to memory; the
// non-temporal policy sends each quarter on its own (355 vs ~267 us at
// M=4096 K=3072 N=12288).
#ifndef B1_STORE_AUX
#define B1_STORE_AUX 0
#endif
constexpr int kStoreNT = B1_STORE_AUX;
// A 16-byte buffer store followed by 5 wait states before any instruction
// may rewrite its data registers.  A store of more than 8 bytes reads its
// data in the cycles after it issues; the compiler inserts that gap only
// for stores whose soffset is not a register, and the epilogue stores carry
// their row offset in an SGPR.  Without it, a VALU write issued right after
// such a store changed the stored values of some lanes (the SwiGLU
// epilogue: 2272 of 786,432 outputs, different on every launch).  The asm
// takes the data as an input, so its registers stay live until the nops
// have issued, and its memory clobber keeps it after the store.
template <int AUX>
__device__ __forceinline__ void store16_guarded(u32x4 v, __amdgpu_buffer_rsrc_t rsrc, int voff, int soff) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, soff, AUX);
    asm volatile("s_nop 4" ::"v"(v) : "memory");
}

// 16 bytes per lane from the buffer at byte offset voff, landing at
// lds + 16 * lane (wave-uniform lds, through M0).
__device__ __forceinline__ void dma_buf_lds16(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)lds, 16, voff, 0, 0, 0);
}
// The same, 16 or 12 bytes per lane (12-byte lanes also land 16 bytes
// apart), with a wave-uniform byte offset soff (an SGPR) added to voff.  A
// constant offset goes into soff, not the instruction's offset field: for
// these loads the instruction offset moves the LDS destination as well.
__device__ __forceinline__ void dma_buf_lds16s(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma_buf_lds12s(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)lds, 12, voff, soff, 0, 0);
}
// 4 bytes per lane, landing at lds + 4 * lane.
__device__ __forceinline__ void dma_buf_lds4(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)lds, 4, voff, 0, 0, 0);
}

__device__ __forceinline__ uint32_t dup_lo16(uint32_t d) {
    return __builtin_amdgcn_perm(d, d, 0x01000100u);
}
__device__ __forceinline__ uint32_t dup_hi16(uint32_t d) {
    return __builtin_amdgcn_perm(d, d, 0x03020302u);
}

// Weight dword for fp16 pair slot (bits p and p+16 of `w`, p = 15 - sh):
// each half is the fp16 scale with its sign flipped where the bit is 0.
__device__ __forceinline__ uint32_t wpair(uint32_t w, int sh, uint32_t scale2) {
    return xnor_sel(kSignPair, w << sh, scale2);
}

// One v_lshlrev_b64 of the pair (w, w >> 8): its low dword is w << SH and
// its high dword carries bits d + 8 and d + 24 of w at 15 and 31 (d = 15 -
// SH < 8), so that one shift serves the weight dwords of pairs d and d + 8.
// A 64-bit shift costs what a 32-bit one does on gfx950 (measured: both
// about 2 ns per wave instruction per SIMD with the SIMDs saturated, a
// v_bitop3 1.2 ns); the compiler splits a constant 64-bit shift into two
// 32-bit ops, hence the asm.  Its result only feeds VALU bit ops (no MFMA
// operand hazard).
template <int SH>
__device__ __forceinline__ uint64_t shl64(uint64_t v) {
    static_assert(SH >= 8 && SH <= 15, "pairs d < 8");
    uint64_t r;
    asm("v_lshlrev_b64 %0, %1, %2" : "=v"(r) : "I"(SH), "v"(v));
    return r;
}
// The weight dwords of pairs 4T + j (lo) and 4T + j + 8 (hi), j = 0..3,
// T = 0 or 1, from the sign word w and w8 = w >> 8: the same values as
// wpair(w, 15 - 4T - j, scale2) and wpair(w, 7 - 4T - j, scale2).
template <int T>
__device__ __forceinline__ void wpair_quads(uint32_t w, uint32_t w8, uint32_t scale2, u32x4 &lo, u32x4 &hi) {
    const uint64_t v = (uint64_t)w8 << 32 | w;
    const uint64_t v0 = shl64<15 - 4 * T>(v), v1 = shl64<14 - 4 * T>(v), v2 = shl64<13 - 4 * T>(v),
                   v3 = shl64<12 - 4 * T>(v);
    lo[0] = xnor_sel(kSignPair, (uint32_t)v0, scale2);
    lo[1] = xnor_sel(kSignPair, (uint32_t)v1, scale2);
    lo[2] = xnor_sel(kSignPair, (uint32_t)v2, scale2);
    lo[3] = xnor_sel(kSignPair, (uint32_t)v3, scale2);
    hi[0] = xnor_sel(kSignPair, (uint32_t)(v0 >> 32), scale2);
    hi[1] = xnor_sel(kSignPair, (uint32_t)(v1 >> 32), scale2);
    hi[2] = xnor_sel(kSignPair, (uint32_t)(v2 >> 32), scale2);
    hi[3] = xnor_sel(kSignPair, (uint32_t)(v3 >> 32), scale2);
}

__device__ __forceinline__ void count_nonfinite(int32_t *ctr, int bad) {
    if (bad && ctr) atomicAdd(ctr, bad);
}

// ---------------------------------------------------------------- exact --

constexpr int kExTN = 256; // output columns per work-group (one per thread)
constexpr int kExKC = 256; // K staged in LDS per pass

// EXACT mode: every output in the reference's scalar order
// (src/b1_0_kernel.h:253-277): block_sum takes +-a over the block's 32
// elements in order, then sum += scale * block_sum (an fp32 multiply and
// an fp32 add, no contraction).  Each +-a step is fma(a, s, block_sum) with
// s = +-1.0: the product is exact, so the fma rounds once, exactly as the
// add or the subtract does, to the same value (signed zeros included; a
// NaN may carry another payload).  The 32 signs of a block are formed once
// (a shift and a bit op each) for the work-group's TM rows, which share
// them: about 1 + 2 / TM VALU operations per multiply-accumulate, where a
// select between a and -a and an add made 2 + 2 / TM.
template <int TM>
__global__ __launch_bounds__(kExTN) void b1_exact_kernel(LinearArgs p) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float As[TM][kExKC];
    const int n = blockIdx.x * kExTN + threadIdx.x;
    const int m0 = blockIdx.y * TM;
    const int nb = p.K / 32;
    const int nrow = n < p.N ? n : p.N - 1;
    const uint16_t *wr = reinterpret_cast<const uint16_t *>(p.w + (size_t)nrow * nb * 6);
    float sum[TM];
#pragma unroll
    for (int r = 0; r < TM; ++r) sum[r] = 0.0f;

    for (int kc = 0; kc < p.K; kc += kExKC) {
        const int klen = min(kExKC, p.K - kc);
        __syncthreads();
        for (int i = threadIdx.x; i < TM * kExKC; i += kExTN) {
            const int r = i / kExKC, c = i - r * kExKC;
            As[r][c] = (m0 + r < p.M && c < klen)
                           ? p.act[(size_t)(m0 + r) * p.lda + kc + c]
                           : 0.0f;
        }
        __syncthreads();
        const int nbk = klen / 32;
        for (int b = 0; b < nbk; ++b) {
            const uint16_t *blk = wr + (size_t)(kc / 32 + b) * 3;
            const float scale = (float)__builtin_bit_cast(_Float16, blk[0]);
            const uint32_t bits = (uint32_t)blk[1] | ((uint32_t)blk[2] << 16);
            float bs[TM];
#pragma unroll
            for (int r = 0; r < TM; ++r) bs[r] = 0.0f;
#pragma unroll
            for (int i4 = 0; i4 < 8; ++i4) {
                // +1.0 for a set bit, -1.0 for a clear one
                float sg[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 4 * i4 + j;
                    sg[j] = __builtin_bit_cast(float, ((bits << (31 - i)) & 0x80000000u) ^ 0xBF800000u);
                }
#pragma unroll
                for (int r = 0; r < TM; ++r) {
                    const floatx4 a = *reinterpret_cast<const floatx4 *>(&As[r][b * 32 + 4 * i4]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) bs[r] = __builtin_fmaf(a[j], sg[j], bs[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < TM; ++r) sum[r] = sum[r] + scale * bs[r];
        }
    }
    if (n >= p.N) return;
    int bad = 0;
#pragma unroll
    for (int r = 0; r < TM; ++r) {
        if (m0 + r < p.M) {
            bad += !__builtin_isfinite(sum[r]);
            p.out[(size_t)(m0 + r) * p.ldo + n] = sum[r];
        }
    }
    count_nonfinite(p.nonfinite, bad);
}

// ----------------------------------------------------------------- gemm --

template <int BM, int BN, int WM, int WN>
struct GemmCfg {
    static constexpr int NWM = BM / WM, NWN = BN / WN, NW = NWM * NWN;
    static constexpr int NT = NW * 64;
    static constexpr int MT = WM / 32, NTL = WN / 32; // 32x32 sub-tiles/wave
    static constexpr int KC = 64;                     // K per stage (2 blocks)
    static constexpr int ROW = KC * 2 + 16;           // LDS bytes per A row
    static constexpr int STAGE = BM * ROW;
    static constexpr int UNITS = BM * 8; // (row, block, quad) staging units
    static constexpr int UPT = UNITS / NT;
    static_assert(UNITS % NT == 0, "staging units must divide evenly");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "32x32 sub-tiles");
};

// Work-groups are dispatched round-robin over the 8 XCDs (bid % 8).  Give
// each XCD a contiguous run of tiles (N-fastest) so the work-groups resident
// on one XCD share activation rows in that XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int nblk) {
    const int xcd = bid & 7, loc = bid >> 3;
    const int q = nblk >> 3, r = nblk & 7;
    return xcd * q + min(xcd, r) + loc;
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void b1_gemm_fused_kernel(LinearArgs p, int tiles_n) {
    using C = GemmCfg<BM, BN, WM, WN>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * C::STAGE];

    const int t = xcd_tile(blockIdx.x, gridDim.x);
    const int tm = t / tiles_n, tn = t - tm * tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::NWN, wn = wave - wm * C::NWN;
    const int li = lane & 31, g = lane >> 5;
    const size_t rs = (size_t)(p.K / 32) * 6;
    const int nstage = p.K / C::KC;

    // ---- activation staging: unit id -> (row, block, quad c) -------------
    floatx4 ar[C::UPT][2];
    auto load_a = [&](int ks) {
#pragma unroll
        for (int u = 0; u < C::UPT; ++u) {
            const int id = tid + u * C::NT;
            const int c = id & 3, blk = (id >> 2) & 1, row = id >> 3;
            const int gm = m0 + row;
            if (gm < p.M) {
                const float *src = p.act + (size_t)gm * p.lda + ks * C::KC + blk * 32 + c * 4;
                ar[u][0] = *reinterpret_cast<const floatx4 *>(src);
                ar[u][1] = *reinterpret_cast<const floatx4 *>(src + 16);
            } else {
                ar[u][0] = floatx4{0.f, 0.f, 0.f, 0.f};
                ar[u][1] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int u = 0; u < C::UPT; ++u) {
            const int id = tid + u * C::NT;
            const int c = id & 3, blk = (id >> 2) & 1, row = id >> 3;
            u32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = pack_f16(ar[u][0][j], ar[u][1][j]);
            *reinterpret_cast<u32x4 *>(lds + buf * C::STAGE + row * C::ROW + blk * 64 + c * 16) = v;
        }
    };

    // ---- packed weights: lane column n, 12 bytes (2 blocks) per stage ----
    uint32_t br[C::NTL][3];
    const int ncol = n0 + wn * WN + li;
    auto load_b = [&](int ks) {
#pragma unroll
        for (int nt = 0; nt < C::NTL; ++nt) {
            const int n = ncol + nt * 32;
            if (n < p.N) {
                const uint32_t *src = reinterpret_cast<const uint32_t *>(p.w + (size_t)n * rs + (size_t)ks * 12);
                br[nt][0] = src[0];
                br[nt][1] = src[1];
                br[nt][2] = src[2];
            } else {
                br[nt][0] = br[nt][1] = br[nt][2] = 0u;
            }
        }
    };

    floatx16 acc[C::MT][C::NTL];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NTL; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    auto compute = [&](int buf, const uint32_t (&bq)[C::NTL][3]) {
        const uint8_t *base = lds + buf * C::STAGE + (wm * WM + li) * C::ROW + g * 16;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            uint32_t s2[C::NTL], wg[C::NTL];
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt) {
                uint32_t wd;
                if (b == 0) {
                    s2[nt] = dup_lo16(bq[nt][0]);
                    wd = __builtin_amdgcn_alignbit(bq[nt][1], bq[nt][0], 16);
                } else {
                    s2[nt] = dup_hi16(bq[nt][1]);
                    wd = bq[nt][2];
                }
                wg[nt] = wd >> (4 * g);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                half8 af[C::MT];
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
                    af[mt] = *reinterpret_cast<const half8 *>(base + mt * 32 * C::ROW + b * 64 + h * 32);
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
                    u32x4 bd;
#pragma unroll
                    for (int j = 0; j < 4; ++j) bd[j] = wpair(wg[nt], 15 - 8 * h - j, s2[nt]);
                    const half8 bf = __builtin_bit_cast(half8, bd);
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mt], bf, acc[mt][nt], 0, 0, 0);
                }
            }
        }
    };

    load_a(0);
    load_b(0);
    store_a(0);
    __syncthreads();
    for (int s = 0; s < nstage; ++s) {
        uint32_t bc[C::NTL][3];
#pragma unroll
        for (int nt = 0; nt < C::NTL; ++nt) {
            bc[nt][0] = br[nt][0];
            bc[nt][1] = br[nt][1];
            bc[nt][2] = br[nt][2];
        }
        const bool more = s + 1 < nstage;
        if (more) {
            load_a(s + 1);
            load_b(s + 1);
        }
        compute(s & 1, bc);
        if (more) store_a((s + 1) & 1);
        __syncthreads();
    }

    // ---- epilogue: 32x32 accumulator layout: lane column li, rows
    // 8*(v/4) + 4*g + v%4 of each sub-tile ------------------------------
    int bad = 0;
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) {
#pragma unroll
        for (int nt = 0; nt < C::NTL; ++nt) {
            const int n = ncol + nt * 32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * WM + mt * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
                if (m < p.M && n < p.N) {
                    const float y = acc[mt][nt][v];
                    bad += !__builtin_isfinite(y);
                    p.out[(size_t)m * p.ldo + n] = y;
                }
            }
        }
    }
    count_nonfinite(p.nonfinite, bad);
}

// A 16-byte fp32 load; NT: non-temporal, for producer inputs larger than
// the Infinity Cache that are read exactly once (see b1_pack_act_kernel).
template <bool NT>
__device__ __forceinline__ floatx4 load_f4(const float *p) {
    if constexpr (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(p));
    else
        return *reinterpret_cast<const floatx4 *>(p);
}

// Producer inputs from this size on are streamed with non-temporal loads.
constexpr uint64_t kNtInputBytes = 128ull << 20;

template <bool NT>
__device__ __forceinline__ void store_f4(float *p, const floatx4 &v) {
    if constexpr (NT)
        __builtin_nontemporal_store(v, reinterpret_cast<floatx4 *>(p));
    else
        *reinterpret_cast<floatx4 *>(p) = v;
}

// ------------------------------------------------------------- GELU-tanh --
//
// 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), elementwise in
// fp32.  The plain form writes fp32; the fused forms write the fp16
// K-slot-paired activations that the packed GEMM reads, so a GELU between
// two B1_0 linears costs one read and one half-size write (or, in the
// GEMM's epilogue, nothing beyond the GEMM's own half-size output).
//
// Evaluated as x / (1 + e^(-2u)), the same function (1 + tanh(u) =
// 2 / (1 + e^(-2u))), with e^(-2u) = 2^(x (c1 + c2 x^2)), c1 = -2
// sqrt(2/pi) / ln 2 and c2 = 0.044715 c1: one hardware exp2 and one
// reciprocal instead of a library tanh, which matters in the GEMM epilogue
// where no MFMA work overlaps it.  Within 3e-7 max(1, |x|) of the float64
// function (1-ulp exp2 and reciprocal included).  Large negative x: the
// exponential overflows to inf and the result is -0; NaN stays NaN.
__device__ __forceinline__ float gelu_tanh(float x) {
    const float c1 = -2.30220819f;  // -2 sqrt(2/pi) log2(e)
    const float c2 = -0.102943242f; // 0.044715 c1
    const float t = x * __builtin_fmaf(c2, x * x, c1);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// Four float4 units in flight per thread (loads first), non-temporal past
// 128 MB: a grid of at most 8192 blocks walking one unit at a time ran
// 81.2 us at 4608 x 12288 (2.8 TB/s read), this form 72.0 us.  In place
// (x == y) too: a thread writes only the units it has read.
template <bool NT>
__global__ __launch_bounds__(256) void b1_gelu_kernel(const float *x, int64_t ldx, float *y, int64_t ldy, int cols,
                                                      int rows) {
    const int q = cols / 4; // float4 units per row (cols % 4 == 0)
    const int64_t units = (int64_t)rows * q;
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; u + 3 * stride < units; u += 4 * stride) {
        int64_t r[4];
        int c[4];
        floatx4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t uk = u + k * stride;
            r[k] = uk / q;
            c[k] = (int)(uk - r[k] * q) * 4;
            v[k] = load_f4<NT>(x + r[k] * ldx + c[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            floatx4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = gelu_tanh(v[k][j]);
            store_f4<NT>(y + r[k] * ldy + c[k], o);
        }
    }
    for (; u < units; u += stride) {
        const int64_t r = u / q;
        const int c = (int)(u - r * q) * 4;
        const floatx4 v = load_f4<NT>(x + r * ldx + c);
        floatx4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = gelu_tanh(v[j]);
        store_f4<NT>(y + r * ldy + c, o);
    }
}

template <bool NT>
__global__ __launch_bounds__(256) void b1_gelu_pack_kernel(const float *__restrict__ act, int64_t lda,
                                                           uint32_t *__restrict__ ah, int64_t ldw, int M, int K) {
    const int nb = K / 32;
    const int units = M * nb * 4; // (row, block, quad)
    for (int u = blockIdx.x * 256 + threadIdx.x; u < units; u += gridDim.x * 256) {
        const int c = u & 3, rb = u >> 2;
        const int row = rb / nb, blk = rb - row * nb;
        const float *src = act + (size_t)row * lda + blk * 32 + c * 4;
        const floatx4 lo = load_f4<NT>(src);
        const floatx4 hi = load_f4<NT>(src + 16);
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = pack_f16(gelu_tanh(lo[j]), gelu_tanh(hi[j]));
        *reinterpret_cast<u32x4 *>(ah + (size_t)row * ldw + blk * 16 + c * 4) = v;
    }
}

// silu(x) = x / (1 + e^-x), in fp32 with the device library's expf.
__device__ __forceinline__ float silu_f32(float x) {
#pragma clang fp contract(off)
    return x / (1.0f + expf(-x));
}

// r + g y as the reference's two ggml ops (a multiply, then an add), each
// rounded to fp32: never contracted into one FMA.
__device__ __forceinline__ float gate_residual(float r, float g, float y) {
#pragma clang fp contract(off)
    const float t = g * y;
    return r + t;
}

__device__ __forceinline__ float mul_f32(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}

// SwiGLU (ggml_swiglu: silu of the first half of a row times its second
// half) fused with the fp16 packing, written at a packed row stride of ldw
// words: act [M][lda] holds 2H columns, the packed output H.
template <bool NT>
__global__ __launch_bounds__(256) void b1_swiglu_pack_kernel(const float *__restrict__ act, int64_t lda,
                                                             uint32_t *__restrict__ ah, int64_t ldw, int M, int H) {
    const int nb = H / 32;
    const int units = M * nb * 4; // (row, block, quad)
    for (int u = blockIdx.x * 256 + threadIdx.x; u < units; u += gridDim.x * 256) {
        const int c = u & 3, rb = u >> 2;
        const int row = rb / nb, blk = rb - row * nb;
        const float *g = act + (size_t)row * lda + blk * 32 + c * 4;
        const float *v = g + H;
        const floatx4 glo = load_f4<NT>(g);
        const floatx4 ghi = load_f4<NT>(g + 16);
        const floatx4 vlo = load_f4<NT>(v);
        const floatx4 vhi = load_f4<NT>(v + 16);
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            o[j] = pack_f16(mul_f32(silu_f32(glo[j]), vlo[j]), mul_f32(silu_f32(ghi[j]), vhi[j]));
        *reinterpret_cast<u32x4 *>(ah + (size_t)row * ldw + blk * 16 + c * 4) = o;
    }
}

// ------------------------------------------- LayerNorm + modulation (A) --
//
// The producer of the linears' activations in the reference graph
// (src/diffuser_graph.cpp:347-352, 444-448, 479-480):
//   x_n = ggml_norm(x, eps):  (x - mean) / sqrt(var + eps) over a row,
//   out = x_n * (scale[j] + 1) + shift[j],
// each step an fp32 op (no FMA).  mean and var are accumulated in double
// (the ggml CPU norm's ggml_float sums), mean = sum / H rounded to fp32,
// var = sum((x - mean)^2) / H with each square an fp32 product.  One wave
// per row; the row is read three times (sum, squares, output), from L2 after
// the first.  The output is fp32 [rows][ldy], or fp16 in the K-slot pairing
// the packed GEMM reads (word 16 blk + d = out[32 blk + d] | out[32 blk + d
// + 16] << 16).

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float norm_mod(float x, float mean, float rstd, float sc, float sh) {
#pragma clang fp contract(off)
    const float n = (x - mean) * rstd;
    return n * (sc + 1.0f) + sh;
}

// Output of one (block, quad) unit: the 4 + 4 values of elements c..c+3
// and c+16..c+19, as fp32 or as 4 packed fp16 words.
__device__ __forceinline__ void norm_mod_store(const floatx4 &lo, const floatx4 &hi, int c, int u, int row, int H,
                                               float mean, float rstd, const float *__restrict__ scale,
                                               const float *__restrict__ shift, float *__restrict__ y, int64_t ldy,
                                               uint32_t *__restrict__ packed) {
    const floatx4 sl = *reinterpret_cast<const floatx4 *>(scale + c);
    const floatx4 sh = *reinterpret_cast<const floatx4 *>(scale + c + 16);
    const floatx4 tl = *reinterpret_cast<const floatx4 *>(shift + c);
    const floatx4 th = *reinterpret_cast<const floatx4 *>(shift + c + 16);
    floatx4 ol, oh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ol[j] = norm_mod(lo[j], mean, rstd, sl[j], tl[j]);
        oh[j] = norm_mod(hi[j], mean, rstd, sh[j], th[j]);
    }
    if (packed) {
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = pack_f16(ol[j], oh[j]);
        *reinterpret_cast<u32x4 *>(packed + (size_t)row * (H / 2) + (u >> 2) * 16 + (u & 3) * 4) = v;
    } else {
        *reinterpret_cast<floatx4 *>(y + (size_t)row * ldy + c) = ol;
        *reinterpret_cast<floatx4 *>(y + (size_t)row * ldy + c + 16) = oh;
    }
}

// U > 0: the row is held in registers (H <= 512 U), read once with all its
// loads in flight.  U == 0: any H, the row read three times.  U == 6 is held to 96
// VGPRs, 5 waves a SIMD: 1280 work-groups of 4 rows resident at once, so
// 4608 rows (the Flux token count) run in one round (17.6 -> 15.9 us).
template <int U>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(U == 6 ? 5 : 1, 8))) void b1_norm_mod_kernel(const float *__restrict__ x, int64_t ldx, int H, int rows,
                                                          const float *__restrict__ scale,
                                                          const float *__restrict__ shift, float eps,
                                                          float *__restrict__ y, int64_t ldy,
                                                          uint32_t *__restrict__ packed) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return; // whole wave
    const float *xr = x + (size_t)row * ldx;
    const int units = H / 32 * 4; // (block, quad): elements 32 blk + 4 t .. +3 and 16 later
    auto col = [](int u) { return (u >> 2) * 32 + (u & 3) * 4; };
    if constexpr (U > 0) {
        floatx4 lo[U], hi[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int u = lane + 64 * i;
            if (u < units) {
                lo[i] = *reinterpret_cast<const floatx4 *>(xr + col(u));
                hi[i] = *reinterpret_cast<const floatx4 *>(xr + col(u) + 16);
            } else {
                lo[i] = hi[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < U; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) s += (double)lo[i][j] + (double)hi[i][j];
        const float mean = (float)(wave_sum_f64(s) / H);
        double s2 = 0.0;
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (lane + 64 * i < units) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float a = lo[i][j] - mean, b = hi[i][j] - mean;
                    s2 += (double)(a * a);
                    s2 += (double)(b * b);
                }
            }
        }
        const float var = (float)(wave_sum_f64(s2) / H);
        const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int u = lane + 64 * i;
            if (u < units) norm_mod_store(lo[i], hi[i], col(u), u, row, H, mean, rstd, scale, shift, y, ldy, packed);
        }
    } else {
        double s = 0.0;
        for (int u = lane; u < units; u += 64) {
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(xr + col(u));
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(xr + col(u) + 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) s += (double)lo[j] + (double)hi[j];
        }
        const float mean = (float)(wave_sum_f64(s) / H);
        double s2 = 0.0;
        for (int u = lane; u < units; u += 64) {
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(xr + col(u));
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(xr + col(u) + 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = lo[j] - mean, b = hi[j] - mean;
                s2 += (double)(a * a);
                s2 += (double)(b * b);
            }
        }
        const float var = (float)(wave_sum_f64(s2) / H);
        const float rstd = 1.0f / sqrtf(var + eps);
        for (int u = lane; u < units; u += 64) {
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(xr + col(u));
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(xr + col(u) + 16);
            norm_mod_store(lo, hi, col(u), u, row, H, mean, rstd, scale, shift, y, ldy, packed);
        }
    }
}

// ------------------------------------------------------ unfused epilogue --
//
// The GEMM epilogues as a separate pass over a linear's output y [M][ldy],
// for the paths that do not run the packed GEMM; the same fp32 arithmetic
// as the fused epilogue.  kind 1: out[m][c] = res[m][c] + gate[c] y[m][c];
// kind 2: out[m][c] = silu(y[m][c]) y[m][H + c]; c < cols.

__global__ __launch_bounds__(256) void b1_epi_kernel(const float *__restrict__ y, int64_t ldy, int M, int cols,
                                                     int kind, const float *gate, const float *res, int64_t ldr,
                                                     int H, float *out, int64_t ldo) {
    const int64_t units = (int64_t)M * cols;
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
        const int64_t m = u / cols;
        const int c = (int)(u - m * cols);
        const float v = y[m * ldy + c];
        out[m * ldo + c] = kind == 1 ? gate_residual(res[m * ldr + c], gate[c], v)
                                     : mul_f32(silu_f32(v), y[m * ldy + H + c]);
    }
}

// --------------------------------------------------------- weight writer --
//
// fp32 weights [N][ldw] -> packed B1_0, one thread per 32-weight block:
// scale = fp16(mean |w|) rounded to nearest even, bit i = (w_i >= 0) (so
// -0 sets the bit and NaN clears it), bytes [scale_lo, scale_hi, sign word
// LE].  The block sum follows one of the reference's two writers exactly:
// order 0, numpy's np.mean over 32 float32 values (convert_to_b1_0_packed.py:
// 21-43: the first element, plus an 8-way pairwise sum of the other 31);
// order 1, a left-to-right sum (tests/c_ops/test_b1_linear.cpp:129-163).

__global__ __launch_bounds__(256) void b1_quantize_kernel(const float *__restrict__ w, int64_t ldw, int K, int N,
                                                          uint8_t *__restrict__ out, int order) {
#pragma clang fp contract(off)
    const int nb = K / 32;
    const int64_t total = (int64_t)N * nb;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        const int64_t n = t / nb;
        const int b = (int)(t - n * nb);
        const float *src = w + n * ldw + (int64_t)b * 32;
        float a[32];
        uint32_t bits = 0;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float v = src[i];
            a[i] = __builtin_fabsf(v);
            bits |= (v >= 0.0f ? 1u : 0u) << i;
        }
        float sum;
        if (order == 0) {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = a[1 + j];
#pragma unroll
            for (int i = 8; i < 24; i += 8)
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] += a[1 + i + j];
            float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
            for (int i = 24; i < 31; ++i) res += a[1 + i];
            sum = a[0] + res;
        } else {
            sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) sum += a[i];
        }
        const _Float16 h = (_Float16)(sum / 32.0f);
        uint16_t *o = reinterpret_cast<uint16_t *>(out + t * 6);
        o[0] = __builtin_bit_cast(uint16_t, h);
        o[1] = (uint16_t)(bits & 0xffffu);
        o[2] = (uint16_t)(bits >> 16);
    }
}

// ------------------------------------------------------- pack activations --
//
// fp32 activations -> fp16 (RNE) in the K-slot pairing, once per call: u32
// word (row, 16 blk + d) holds (a[row][32 blk + d], a[row][32 blk + d + 16]).
// The GEMM then streams this straight into LDS with no per-tile conversion.

// NT: the fp32 input is read with non-temporal loads, for inputs larger
// than the Infinity Cache that are read exactly once (4608 x 15360: 65.6 vs
// 72.9 us); a cache-resident input is faster with the default policy
// (4096 x 3072: 11.5 vs 13.4 us).
template <bool NT>
__global__ __launch_bounds__(256) void b1_pack_act_kernel(const float *__restrict__ act, int64_t lda,
                                                          uint32_t *__restrict__ ah, int64_t ldw, int M, int K) {
    const int nb = K / 32;
    const int units = M * nb * 4; // (row, block, quad)
    for (int u = blockIdx.x * 256 + threadIdx.x; u < units; u += gridDim.x * 256) {
        const int c = u & 3, rb = u >> 2;
        const int row = rb / nb, blk = rb - row * nb;
        const float *src = act + (size_t)row * lda + blk * 32 + c * 4;
        const floatx4 lo = load_f4<NT>(src);
        const floatx4 hi = load_f4<NT>(src + 16);
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = pack_f16(lo[j], hi[j]);
        *reinterpret_cast<u32x4 *>(ah + (size_t)row * ldw + blk * 16 + c * 4) = v;
    }
}

// The same packing for the fp32 entry points, range-safe: a row whose
// largest |a| would overflow fp16 (>= 65520, the RNE rounding threshold of
// 65504) is first multiplied by 2^-e, e >= 1 chosen so that its largest
// magnitude lands in [2^14, 2^15), and rsc[row] = 2^e tells the GEMM to
// multiply that row's outputs back.  Scaling by a power of two is exact in
// fp32 and in the fp16 rounding (short of the fp16 subnormal range, where
// values are below 2^-24 of the row's largest), so the row keeps fp16
// relative precision instead of turning into +-inf; every other row has e =
// 0, rsc = 1, and exactly the bits of b1_pack_act_kernel.  NaN inputs stay
// NaN; an inf keeps e = 0 (the reference's fp32 sums are non-finite there
// too).  One row is handled by 1, 2 or 4 waves (wpr = 1 << wpr_log2) of a
// 4-wave work-group, each lane holding up to U (block, quad) units of 8
// elements in registers, so the row is read once; U == 0: any length, read
// twice.
template <int U, bool NT>
__global__ __launch_bounds__(256) void b1_pack_rows_kernel(const float *__restrict__ act, int64_t lda,
                                                           uint32_t *__restrict__ ah, int64_t ldw,
                                                           float *__restrict__ rsc, int M, int K, int wpr_log2) {
    __shared__ float wmax[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wpr = 1 << wpr_log2;
    const int row = blockIdx.x * (4 >> wpr_log2) + (wave >> wpr_log2);
    const int sub = wave & (wpr - 1);
    const bool valid = row < M;
    const int units = K / 8; // (block, quad): elements 32 blk + 4 c .. +3 and 16 later
    const float *xr = act + (size_t)(valid ? row : 0) * lda;
    uint32_t *pr = ah + (size_t)(valid ? row : 0) * ldw;
    auto col = [](int u) { return (u >> 2) * 32 + (u & 3) * 4; };
    auto amax4 = [](float m, const floatx4 &v) {
        return __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fmaxf(__builtin_fabsf(v[0]), __builtin_fabsf(v[1]))),
                               __builtin_fmaxf(__builtin_fabsf(v[2]), __builtin_fabsf(v[3])));
    };
    const int stride = 64 * wpr; // units between a lane's consecutive units
    const int u0 = sub * 64 + lane;

    floatx4 lo[U > 0 ? U : 1], hi[U > 0 ? U : 1];
    float m = 0.0f;
    if constexpr (U > 0) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int u = u0 + i * stride;
            if (valid && u < units) {
                lo[i] = load_f4<NT>(xr + col(u));
                hi[i] = load_f4<NT>(xr + col(u) + 16);
            } else {
                lo[i] = hi[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int i = 0; i < U; ++i) m = amax4(amax4(m, lo[i]), hi[i]);
    } else {
        for (int u = u0; valid && u < units; u += stride)
            m = amax4(amax4(m, load_f4<NT>(xr + col(u))), load_f4<NT>(xr + col(u) + 16));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o));
    if (wpr > 1) {
        if (lane == 0) wmax[wave] = m;
        __syncthreads();
        const int w0 = wave & ~(wpr - 1);
        for (int j = 0; j < wpr; ++j) m = __builtin_fmaxf(m, wmax[w0 + j]);
    }
    // e = 0 unless the row overflows fp16; then m = 2^E (1.f), E >= 15 and
    // e = E - 14 (at most 113, so 2^-e and 2^e are normal floats)
    int e = 0;
    if (m >= 65520.0f && m <= 3.40282347e38f) e = (int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xff) - 127 - 14;
    const float down = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
    if (valid && sub == 0 && lane == 0) rsc[row] = __builtin_bit_cast(float, (uint32_t)(127 + e) << 23);
    auto store = [&](int u, floatx4 l, floatx4 h) {
        if (e) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                l[j] *= down;
                h[j] *= down;
            }
        }
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = pack_f16(l[j], h[j]);
        *reinterpret_cast<u32x4 *>(pr + (u >> 2) * 16 + (u & 3) * 4) = v;
    };
    if constexpr (U > 0) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int u = u0 + i * stride;
            if (valid && u < units) store(u, lo[i], hi[i]);
        }
    } else {
        for (int u = u0; valid && u < units; u += stride)
            store(u, load_f4<NT>(xr + col(u)), load_f4<NT>(xr + col(u) + 16));
    }
}

// Exact recomputation of the rows that the paths converting fp32
// activations inside their own kernel (the fused-conversion GEMM and the
// small-M kernels, used without a workspace) cannot take in fp16: a row
// holding an |a| >= 65520 (or an inf) is computed again in the reference's
// scalar order, the arithmetic of b1_exact_kernel, so its outputs are
// EXACT mode's bit for bit.  One work-group per row; other rows only cost a
// read (16-byte aligned rows: the callers' fp32 kernels require them).  The
// non-finite counter is corrected by the change in the count of non-finite
// values the row's outputs make.
constexpr int kFixKC = 2048; // activations staged in LDS per pass
__global__ __launch_bounds__(256) void b1_fixup_rows_kernel(LinearArgs p) {
#pragma clang fp contract(off)
    __shared__ float as[kFixKC];
    const int row = blockIdx.x;
    const float *xr = p.act + (size_t)row * p.lda;
    int over = 0;
    for (int k = threadIdx.x * 4; k < p.K; k += 1024) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(xr + k);
#pragma unroll
        for (int j = 0; j < 4; ++j) over |= __builtin_fabsf(v[j]) >= 65520.0f;
    }
    if (!__syncthreads_or(over)) return;
    const int nb = p.K / 32;
    int delta = 0;
    for (int n0 = 0; n0 < p.N; n0 += 256) {
        const int n = n0 + threadIdx.x;
        const uint16_t *wr = reinterpret_cast<const uint16_t *>(p.w + (size_t)(n < p.N ? n : 0) * nb * 6);
        float sum = 0.0f;
        for (int kc = 0; kc < p.K; kc += kFixKC) {
            const int klen = min(kFixKC, p.K - kc);
            __syncthreads();
            for (int i = threadIdx.x; i < klen; i += 256) as[i] = xr[kc + i];
            __syncthreads();
            for (int b = 0; b < klen / 32; ++b) {
                const uint16_t *blk = wr + (size_t)(kc / 32 + b) * 3;
                const float scale = (float)__builtin_bit_cast(_Float16, blk[0]);
                const uint32_t bits = (uint32_t)blk[1] | ((uint32_t)blk[2] << 16);
                float bs = 0.0f;
                for (int i = 0; i < 32; ++i) {
                    const float a = as[b * 32 + i];
                    bs = ((bits >> i) & 1u) ? bs + a : bs - a;
                }
                sum = sum + scale * bs;
            }
        }
        if (n < p.N) {
            float *o = p.out + (size_t)row * p.ldo + n;
            delta += !__builtin_isfinite(sum) - !__builtin_isfinite(*o);
            *o = sum;
        }
    }
    if (p.nonfinite && delta) atomicAdd(p.nonfinite, delta);
}

// ------------------------------------------------------------- gemm (lds) --
//
// Wide-tile GEMM over pre-packed fp16 activations.  Work-group tile BM x BN,
// NW = BN/WN waves side by side along N (each wave BM x WN; all waves share
// the activation rows, so no weight column is expanded twice).  K advances
// in stages of 128 (4 blocks).  Both operands of a stage go global -> LDS
// directly, with no VGPR staging, into three-slot rings fetched two stages
// ahead: activations with buffer_load_dwordx4 … lds (rows of 256 bytes, 16-
// byte chunk c of row r at position c ^ (r & 15), so the 16 lanes one
// ds_read_b128 phase serves hit 16 different bank groups of the 64), and
// the 24 packed bytes per weight column and stage with two
// buffer_load_dwordx3 … lds (12 bytes per lane, landing at a 16-byte lane
// stride).
//
// The grid is persistent (one work-group per CU, tiles strided by the grid
// size, in 4 x 8 tile groups so that the work-groups resident on one XCD
// share both activation rows and weight columns in its L2): the first two
// stages of a work-group's next tile are fetched before the current tile's
// results are stored.  The MFMA takes the expanded weights as its A operand
// and the activations as its B operand, so each lane's accumulator holds
// runs of 4 consecutive output columns and the epilogue writes 16-byte
// vectors.

template <int BM, int BN, int WN, int STAGES_>
struct GemmLdsCfg {
    static constexpr int NW = BN / WN, NT = NW * 64;
    static constexpr int MT = BM / 32, NTL = WN / 32;
    static constexpr int STAGES = STAGES_;            // ring slots, fetched one stage ahead
    static constexpr int KC = 128;                    // K per stage (4 blocks)
    static constexpr int ROWB = KC * 2;               // LDS bytes per activation row
    static constexpr int ASTAGE = BM * ROWB;          // activation bytes per slot
    static constexpr int LPW = ASTAGE / 1024 / NW;    // 1 KB activation loads per wave
    static constexpr int CG = WN / 64;                // 64-column weight load groups per wave
    static constexpr int BWAVE = CG * 2 * 1024;       // weight bytes per wave per slot
    static constexpr int BSTAGE = NW * BWAVE;         // weight bytes per slot
    // Weight slots take the bottom of LDS and activation slots follow; then
    // two tile-parity buffers of the BM rows' output scales (row scales of
    // range-safe packing, when the launch has them).
    static constexpr int ABASE = STAGES * BSTAGE;
    static constexpr int RSC = STAGES * (ASTAGE + BSTAGE);
    static constexpr int LDS = RSC + 2 * BM * 4;
    static constexpr int GROUP_M = 4;                 // tile grouping along M
    static constexpr int EPI_STORES = MT * NTL * 4;   // 16-byte stores per lane, full tile
    static_assert(ASTAGE % (1024 * NW) == 0, "activation loads must split evenly");
    static_assert(WN % 64 == 0, "weight loads cover 64 columns, one per lane");
    static_assert(LDS <= 160 * 1024, "gfx950 LDS");
    // The previous tile's stores are counted in vmcnt waits when the count
    // fits its 6 bits; otherwise a tile starts by draining them.
    static constexpr bool COUNT_STORES = EPI_STORES <= 63;
    // 8 waves: 2 per SIMD, 256 registers each.  4 waves (128-column wave
    // tiles, 256 accumulators): 1 per SIMD with 512.
    static constexpr int WAVES_PER_SIMD = NW >= 8 ? 2 : 1;
    static_assert(STAGES == 3, "the three-slot ring is the verified configuration");
};

// Two waves per SIMD (8 waves, one work-group per CU): 256 registers a wave.
// EPI selects what the epilogue writes (GemmEpi):
//   0  out = y
//   1  out = residual + gate[n] * y (fp32 multiply, then add)
//   2  SwiGLU over a weight matrix of 2H rows, gate rows [0, H) and value
//      rows [H, 2H): the GEMM runs over the rows in the order gate block b
//      (32 rows), value block b, ... so that one wave's two 32-column
//      accumulator tiles hold a gate and its value for the same outputs;
//      out[m][j] = silu(y[m][j]) * y[m][H + j], H columns.
template <int BM, int BN, int WN, int STAGES, int EPI>
__global__ __launch_bounds__((BN / WN) * 64, (BN / WN) >= 8 ? 2 : 1) void b1_gemm_kernel(const uint16_t *__restrict__ ah,
                                                                    const uint8_t *__restrict__ w, int K, int N,
                                                                    int M, float *__restrict__ out, int64_t ldo,
                                                                    int32_t *nonfinite, int tiles_m, int tiles_n,
                                                                    int vec_store, GemmEpi epi, int ksplit,
                                                                    int64_t pstride) {
    using C = GemmLdsCfg<BM, BN, WN, STAGES>;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // The wave index is made visibly uniform: LDS-DMA destinations go
    // through M0 and must not depend on the lane.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, g = lane >> 5;
    // Work unit u: K range `split` = u / (tiles_m tiles_n) of ksplit equal
    // ranges, output tile u % (tiles_m tiles_n).  With ksplit > 1 a unit's
    // plain product goes to partial slice `split` (out + split * pstride),
    // which a separate pass sums.
    const int nstage = K / C::KC / ksplit; // stages per unit, a multiple of STAGES
    const int ntiles = tiles_m * tiles_n;
    const int nunits = ntiles * ksplit;
    const uint32_t rs = (uint32_t)(K / 32) * 6;
    const uint8_t *abase = reinterpret_cast<const uint8_t *>(ah);

    // Tile t -> (m0, n0): groups of GROUP_M tile rows, column-major inside a
    // group, so a run of consecutive tiles covers GROUP_M x (run/GROUP_M).
    auto tile_origin = [&](int t, int &m0, int &n0) {
        const int group = t / (C::GROUP_M * tiles_n);
        const int first_m = group * C::GROUP_M;
        const int gsize = min(C::GROUP_M, tiles_m - first_m);
        const int tin = t - first_m * tiles_n;
        m0 = (first_m + tin % gsize) * BM;
        n0 = (tin / gsize) * BN;
    };

    // Activation loads: load j of a stage fills LDS bytes [1024 j, +1024)
    // of the slot = rows 4j..4j+3; lane L writes position L % 16 of row
    // 4j + L / 16, which holds chunk (L % 16) ^ (row & 15).  Rows past M
    // read row M-1.  Weight loads: lane L fetches 12 bytes (blocks 0-1, then
    // 2-3 of the stage) of column n0 + 64 wave + L; columns past N read
    // row N-1.  Neither is ever stored.
    uint32_t aoff[C::LPW];
    uint32_t boff[C::CG];
    auto setup = [&](int m0, int n0) {
#pragma unroll
        for (int i = 0; i < C::LPW; ++i) {
            const int row = 4 * (wave * C::LPW + i) + (lane >> 4);
            const int c = (lane & 15) ^ (row & 15);
            aoff[i] = ((uint32_t)min(m0 + row, M - 1) * (uint32_t)K + (uint32_t)c * 8) * 2;
        }
#pragma unroll
        for (int cg = 0; cg < C::CG; ++cg) {
            const int c = min(n0 + wave * WN + cg * 64 + lane, N - 1);
            int row = c;
            if constexpr (EPI == 2) {
                // GEMM column c -> weight row: 64-column block b holds gate
                // rows 32b.. then value rows H + 32b..
                const int b = c >> 6, within = c & 63;
                row = within < 32 ? 32 * b + within : epi.glu_h + 32 * b + (within - 32);
            }
            if constexpr (EPI == 3) {
                // the same order over the SwiGLU columns [split, N)
                if (epi.act == 2 && c >= epi.split) {
                    const int b = (c - epi.split) >> 6, within = (c - epi.split) & 63;
                    row = epi.split + (within < 32 ? 32 * b + within : epi.glu_h + 32 * b + (within - 32));
                }
            }
            boff[cg] = (uint32_t)row * rs;
        }
    };
    // Buffer loads: the operand in the resource, the lane's 32-bit offset in
    // a VGPR and the stage offset in an SGPR, so no load needs address
    // arithmetic (with 64-bit global addresses, one v_lshl_add_u64 each).
    // The host keeps both operands under 2^32 bytes (gemm_packed_ok).
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(abase), (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), kBufferFlags);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w), (short)0, (int)((uint32_t)N * rs), kBufferFlags);
    auto issue = [&](int ks, int slot) {
        uint8_t *sa = smem + C::ABASE + slot * C::ASTAGE + wave * C::LPW * 1024;
        uint8_t *sw = smem + slot * C::BSTAGE + wave * C::BWAVE;
        const uint32_t aso = (uint32_t)ks * C::ROWB, wso = (uint32_t)ks * 24;
#pragma unroll
        for (int i = 0; i < C::LPW; ++i) dma_buf_lds16s(ars, sa + i * 1024, aoff[i], aso);
#pragma unroll
        for (int cg = 0; cg < C::CG; ++cg) {
            dma_buf_lds12s(wrs, sw + cg * 2048, boff[cg], wso);
            dma_buf_lds12s(wrs, sw + cg * 2048 + 1024, boff[cg], wso + 12);
        }
    };

    // Fragment offsets: lane (li, g) reads row li (+32 mt) at chunk
    // c = 4b + 2h + g, stored at position c ^ (li & 15); its weight column
    // nt*32 + li sits at a 16-byte stride in each 1 KB half of the wave's
    // weight area.
    // The lane parts of the LDS addresses are kept as LDS pointers, one set
    // for slots 0-1 and one for slot 2, so that every slot, row-tile and
    // block offset is a ds_read immediate (< 64 KiB).
    typedef const __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8 *const lbase = (lds_u8 *)smem;
    lds_u8 *fa01[4][2], *fa2[4][2];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t f = li * C::ROWB + (((4 * b + 2 * h + g) ^ (li & 15)) * 16);
            fa01[b][h] = lbase + C::ABASE + f;
            fa2[b][h] = lbase + C::ABASE + 2 * C::ASTAGE + f;
        }
    lds_u8 *const qa = lbase + wave * C::BWAVE + li * 16;
    static_assert(C::ASTAGE + (C::MT - 1) * 32 * C::ROWB + 64 < 65536, "fragment immediates");

    floatx16 acc[C::MT][C::NTL];

    // One stage = 8 steps (block b = step/2, half h = step%2).  Software
    // pipelined: the wave's own weight dwords of the whole stage are read at
    // its top, activation fragments two steps ahead (three buffers), and the
    // weights of step+1 are expanded while the MFMAs of step run.  A
    // scheduling fence per step keeps the compiler from hoisting every read
    // of the stage.  (With the fragments read one step ahead, the compiler
    // issued them just before the step's last MFMA and the next step waited
    // for them: 1-1.5 % slower at the headline shape.)
    auto compute = [&](int slot, auto &&after_first_reads) {
        lds_u8 *sq = qa + slot * C::BSTAGE;
        auto read_frags = [&](int step, half8 (&af)[C::MT]) {
            const int b = step >> 1, h = step & 1;
            lds_u8 *fb = slot == 2 ? fa2[b][h] : fa01[b][h] + slot * C::ASTAGE;
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
                af[mt] = *reinterpret_cast<const __attribute__((address_space(3))) half8 *>(fb + mt * 32 * C::ROWB);
        };
        // weight column nt*32 + li: blocks 0-1 in the first 1 KB half of its
        // load group, blocks 2-3 in the second, 12 bytes each
        uint32_t d[C::NTL][2][3];
#pragma unroll
        for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
            for (int bp = 0; bp < 2; ++bp) {
                const __attribute__((address_space(3))) uint32_t *q =
                    reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(
                        sq + (nt >> 1) * 2048 + bp * 1024 + (nt & 1) * 512);
                d[nt][bp][0] = q[0];
                d[nt][bp][1] = q[1];
                d[nt][bp][2] = q[2];
            }
        half8 af[3][C::MT];
        read_frags(0, af[0]);
        read_frags(1, af[1]);
        after_first_reads();
        // the expanded weights of a step: block b = step / 2 has its scale
        // and sign word at 6 (b % 2) bytes into its 12-byte pair; lane group
        // g takes dwords 8h + 4g .. +3 of the block (elements d, d + 16)
        uint32_t s2[C::NTL], wg[C::NTL];
        u32x4 bw[2][C::NTL];
        auto expand = [&](int step, u32x4 (&bo)[C::NTL]) {
            const int b = step >> 1, h = step & 1;
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt) {
                if (h == 0) {
                    const uint32_t *dd = d[nt][b >> 1];
                    if ((b & 1) == 0) {
                        s2[nt] = dup_lo16(dd[0]);
                        // the sign word shifted right by 4g in one funnel
                        // shift; its bits above 27 are not those of the
                        // plain shift, but only bits 8h + j and 16 + 8h + j
                        // (<= 27) reach the mask
                        wg[nt] = __builtin_amdgcn_alignbit(dd[1], dd[0], 16 + 4 * g);
                    } else {
                        s2[nt] = dup_hi16(dd[1]);
                        wg[nt] = dd[2] >> (4 * g);
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) bo[nt][j] = wpair(wg[nt], 15 - 8 * h - j, s2[nt]);
            }
        };
        expand(0, bw[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int step = 0; step < 8; ++step) {
            if (step + 2 < 8) read_frags(step + 2, af[(step + 2) % 3]);
            if (step + 1 < 8) expand(step + 1, bw[(step + 1) & 1]);
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt) {
                const half8 bf = __builtin_bit_cast(half8, bw[step & 1][nt]);
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf, af[step % 3][mt], acc[mt][nt], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Epilogue.  Accumulator (n, m) layout of the 32x32 MFMA with weights as
    // A: lane column li = token m0 + 32 mt + li, rows 8*(v/4) + 4*g + v%4 =
    // output columns; v = 4q..4q+3 are 4 consecutive columns.  Stored as one
    // 16-byte vector each, one store instruction would cover a quarter of 32
    // lines (32 rows x 32 bytes).  Full tiles instead go through LDS and are
    // stored as whole 128-byte lines (below).  Non-finite outputs are
    // counted only when the caller passed a counter.
    //
    // The transpose area is the wave's own 2 KB weight area of the last
    // stage's slot (slot 2: the stage count is a multiple of 3), free from
    // the wave's last read of it until the wave itself refills it during the
    // next tile's first stage.  It holds 16 rows of 128 bytes, 16-byte chunk
    // c of row r at position c ^ (r & 7).  The LDS serves 16-byte accesses
    // 8 lanes at a time over 128 bytes of banks: the 8 lanes of a write hold
    // 8 consecutive rows (one chunk each), those of a read one row's 8
    // chunks, both conflict-free (c ^ ((r >> 1) & 7) paired the rows of a
    // write: 1.57 M conflict cycles per launch at M=4096 K=3072 N=12288, at
    // no measurable cost in time).  Then 8 lanes store one row's 128 bytes, a
    // whole line (261.3 -> 252.2 us at M=4096 K=3072 N=12288 for the plain
    // fp32 output).
    typedef __attribute__((address_space(3))) uint8_t lds_u8w;
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    lds_u8w *const tb = (lds_u8w *)smem + 2 * C::BSTAGE + wave * C::BWAVE;
    static_assert(C::STAGES == 3 && 16 * 128 <= C::BWAVE, "the transpose area");
    const int rr0 = lane >> 3, cc = lane & 7;
    // Rows 16 half .. 16 half + 15 of a 32-row piece, 128 bytes each: the
    // lanes holding them (li >> 4 == half) write their four chunks v[j] at
    // chunk 2j + g of row li & 15; then every lane reads chunk cc of rows
    // rr0 and rr0 + 8 into vr.
    auto transpose = [&](const u32x4(&v)[4], int half, u32x4(&vr)[2]) {
        if ((li >> 4) == half) {
            const int r = li & 15;
#pragma unroll
            for (int j = 0; j < 4; ++j) *(lds_u32x4 *)(tb + r * 128 + ((2 * j + g) ^ (r & 7)) * 16) = v[j];
        }
        // Every lane reads below.  Without this fence the compiler moved the
        // reads into the branch above, where only the writing half of the
        // wave runs them.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int rr = rr0 + 8 * k;
            vr[k] = *(const lds_u32x4 *)(tb + rr * 128 + (cc ^ (rr & 7)) * 16);
        }
    };
    // accumulator tile (mt, nt) of lane (li, g) as raw words, chunk q =
    // columns 8q + 4g .. +3 (element values are copied out first: a bit cast
    // of a vector element reads element 0 in this clang)
    auto acc_chunks = [&](int mt, int nt, u32x4(&v)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x = acc[mt][nt][4 * q + e];
                v[q][e] = __builtin_bit_cast(uint32_t, x);
            }
    };
    // A row stride in bytes, opaque to the compiler: the store offsets
    // derived from it are then computed in each epilogue rather than hoisted
    // out of the tile loop into scalar registers the main loop would carry.
    auto stride_bytes = [](int64_t ld) {
        int b = (int)ld * 4;
        asm volatile("" : "+s"(b));
        return b;
    };
    auto count_tile = [&](int &bad) {
        if (nonfinite != nullptr) {
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                    for (int v = 0; v < 16; ++v) bad += !__builtin_isfinite(acc[mt][nt][v]);
        }
    };
    // The fp32 tile through the transpose, whole-line buffer stores into the
    // wave's columns of `out` (row stride ldo, ldb = 4 ldo bytes; 128 rows
    // span < 2^31 bytes).  32 stores per lane.
    auto store_f32_lines = [&](int m0, int n0, float *__restrict__ out, int ldb) {
        const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
            out + (size_t)m0 * ldo + n0 + wave * WN, (short)0, (int)(BM * ldo * 4), kBufferFlags);
        const int lvoff = rr0 * ldb + 16 * cc;
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    u32x4 v[4], vr[2];
                    acc_chunks(mt, nt, v);
                    transpose(v, half, vr);
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const int ro = (mt * 32 + 16 * half + 8 * k) * ldb + nt * 128;
                        store16_guarded<kStoreNT>(vr[k], ors, lvoff, ro);
                    }
                }
    };

    // Returns what the tile-start vmcnt waits may assume about the stores
    // left in flight: 0 none, 1 unknown (wait for all), 2 EPI_STORES vector
    // stores per lane, 3 EPI_STORES / 2.
    auto epilogue = [&](int m0, int n0, float *__restrict__ out) -> int {
        int bad = 0;
        const bool cnt = nonfinite != nullptr;
        if constexpr (EPI == 2) {
            // lane (li, g): tile nt=0 holds gates, nt=1 their values, 4
            // consecutive outputs per register quad
            const int H = epi.glu_h;
            const int jb = (n0 >> 1) + wave * 32;
            const bool fullg = vec_store && m0 + BM <= M && jb + 32 <= H;
            if (fullg) {
                // The wave's 32 outputs of a row are one 128-byte line: made
                // by every lane, then through the transpose as whole lines
                // (16 stores per lane).
                if (cnt) {
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                        for (int v = 0; v < 16; ++v)
                            bad += !__builtin_isfinite(acc[mt][0][v]) + !__builtin_isfinite(acc[mt][1][v]);
                }
                const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
                    out + (size_t)m0 * ldo + jb, (short)0, (int)(BM * ldo * 4), kBufferFlags);
                const int ldb = stride_bytes(ldo);
                const int lvoff = rr0 * ldb + 16 * cc;
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt) {
                    u32x4 v[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float o = mul_f32(silu_f32(acc[mt][0][4 * q + r]), acc[mt][1][4 * q + r]);
                            v[q][r] = __builtin_bit_cast(uint32_t, o);
                        }
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        u32x4 vr[2];
                        transpose(v, half, vr);
#pragma unroll
                        for (int k = 0; k < 2; ++k)
                            store16_guarded<kStoreNT>(vr[k], ors, lvoff, (mt * 32 + 16 * half + 8 * k) * ldb);
                    }
                }
                count_nonfinite(nonfinite, bad);
                return 3;
            }
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) {
                const int m = m0 + mt * 32 + li;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = jb + 8 * q + 4 * g;
                    floatx4 o;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float gt = acc[mt][0][4 * q + r], vl = acc[mt][1][4 * q + r];
                        o[r] = mul_f32(silu_f32(gt), vl);
                        if (cnt && m < M && j + r < H) bad += !__builtin_isfinite(gt) + !__builtin_isfinite(vl);
                    }
                    if (m < M) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (j + r < H) out[(size_t)m * ldo + j + r] = o[r];
                    }
                }
            }
            count_nonfinite(nonfinite, bad);
            return 1;
        }
        if constexpr (EPI == 1) {
            const bool fullr = vec_store && m0 + BM <= M && n0 + BN <= N;
            if (fullr) {
                // y through the transpose; the residual read as whole lines
                // at the same positions, P of the 16 (mt, nt, half) pieces
                // ahead; out = residual + gate * y stored as whole lines.
                // The residual may be `out` itself: each element is read by
                // the lane that later writes it, and every piece's loads are
                // issued before any store of a later piece.
                count_tile(bad);
                const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
                    out + (size_t)m0 * ldo + n0 + wave * WN, (short)0, (int)(BM * ldo * 4), kBufferFlags);
                const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<float *>(epi.res) + (size_t)m0 * epi.ldr + n0 + wave * WN, (short)0,
                    (int)(BM * epi.ldr * 4), kBufferFlags);
                const int ldb = stride_bytes(ldo), lrb = stride_bytes(epi.ldr);
                const int lvoff = rr0 * ldb + 16 * cc, lroff = rr0 * lrb + 16 * cc;
                floatx4 gq[C::NTL];
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt)
                    gq[nt] = *reinterpret_cast<const floatx4 *>(epi.gate + n0 + wave * WN + nt * 32 + 4 * cc);
                constexpr int NP = C::MT * C::NTL * 2, P = 4;
                u32x4 rv[NP][2];
                auto load_res = [&](int j) {
                    const int mt = j / (2 * C::NTL), nt = (j >> 1) % C::NTL, half = j & 1;
#pragma unroll
                    for (int k = 0; k < 2; ++k)
                        rv[j][k] = __builtin_amdgcn_raw_buffer_load_b128(
                            rrs, lroff, (mt * 32 + 16 * half + 8 * k) * lrb + nt * 128, 0);
                };
#pragma unroll
                for (int j = 0; j < P; ++j) load_res(j);
#pragma unroll
                for (int j = 0; j < NP; ++j) {
                    if (j + P < NP) load_res(j + P);
                    const int mt = j / (2 * C::NTL), nt = (j >> 1) % C::NTL, half = j & 1;
                    u32x4 v[4], vr[2];
                    acc_chunks(mt, nt, v);
                    transpose(v, half, vr);
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        u32x4 o;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t yu = vr[k][e], ru = rv[j][k][e];
                            const float gv = gq[nt][e];
                            const float ov =
                                gate_residual(__builtin_bit_cast(float, ru), gv, __builtin_bit_cast(float, yu));
                            o[e] = __builtin_bit_cast(uint32_t, ov);
                        }
                        const int ro = (mt * 32 + 16 * half + 8 * k) * ldb + nt * 128;
                        store16_guarded<kStoreNT>(o, ors, lvoff, ro);
                    }
                }
                count_nonfinite(nonfinite, bad);
                return 2;
            }
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) {
                const int m = m0 + mt * 32 + li;
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int n = n0 + wave * WN + nt * 32 + 8 * q + 4 * g;
                        if (m < M) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                if (n + r < N) {
                                    const float yv = acc[mt][nt][4 * q + r];
                                    bad += cnt && !__builtin_isfinite(yv);
                                    out[(size_t)m * ldo + n + r] =
                                        gate_residual(epi.res[(size_t)m * epi.ldr + n + r], epi.gate[n + r], yv);
                                }
                            }
                        }
                    }
                }
            }
            count_nonfinite(nonfinite, bad);
            return 1;
        }
        if constexpr (EPI == 3) {
            // Columns below split: fp32.  From split on, the packed fp16
            // activations of the next linear: a packed block's dword d holds
            // columns (d, d + 16) of its 32, and lane (li, g) holds columns
            // 8q + 4g + r of each 32-column tile, so registers 4q + r and
            // 4q + 8 + r (q < 2) form dword 8q + 4g + r and 4 consecutive
            // dwords are one 16-byte chunk.  split and N are multiples of 32
            // (64 for SwiGLU), so a tile (a wave's 64 columns for SwiGLU) is
            // wholly one kind.
            static_assert(C::NTL == 2, "SwiGLU pairs one gate and one value tile per wave");
            const int wb = n0 + wave * WN; // wave-uniform
            const bool pcols = wb >= epi.split;
            if (vec_store && m0 + BM <= M && n0 + BN <= N && !(epi.act == 2 && pcols) &&
                (pcols || wb + WN <= epi.split)) {
                // A full tile whose wave columns are all of one kind: whole
                // lines through the transpose.
                count_tile(bad);
                if (!pcols) {
                    store_f32_lines(m0, n0, out, stride_bytes(ldo));
                    count_nonfinite(nonfinite, bad);
                    return 2;
                }
                // The wave's two blocks are 128 consecutive bytes of a packed
                // row: block nt's dwords 8q + 4g .. +3 are its chunk
                // 2 (2 nt + q) + g.  The values are made by every lane before
                // the transpose, which writes half the lanes at a time.
                const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                    epi.pk + (size_t)m0 * epi.ldpw + ((wb - epi.split) >> 5) * 16, (short)0,
                    (int)(BM * epi.ldpw * 4), kBufferFlags);
                const int lpb = stride_bytes(epi.ldpw);
                const int lpoff = rr0 * lpb + 16 * cc;
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt) {
                    u32x4 v[4];
#pragma unroll
                    for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                        for (int q = 0; q < 2; ++q)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float y0 = acc[mt][nt][4 * q + r], y1 = acc[mt][nt][4 * q + 8 + r];
                                v[2 * nt + q][r] = epi.act ? pack_f16(gelu_tanh(y0), gelu_tanh(y1)) : pack_f16(y0, y1);
                            }
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        u32x4 vr[2];
                        transpose(v, half, vr);
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            const int ro = (mt * 32 + 16 * half + 8 * k) * lpb;
                            store16_guarded<0>(vr[k], prs, lpoff, ro);
                        }
                    }
                }
                count_nonfinite(nonfinite, bad);
                return 3;
            }
            if (epi.act == 2 && pcols) {
                // tile 0 holds the gates, tile 1 their values, of the 32
                // outputs of packed block (wb - split) / 64
                if (wb < N) {
                    uint32_t *const pb = epi.pk + ((wb - epi.split) >> 6) * 16 + 4 * g;
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt) {
                        const int m = m0 + mt * 32 + li;
                        if (m >= M) continue;
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            u32x4 v;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float g0 = acc[mt][0][4 * q + r], v0 = acc[mt][1][4 * q + r];
                                const float g1 = acc[mt][0][4 * q + 8 + r], v1 = acc[mt][1][4 * q + 8 + r];
                                if (cnt)
                                    bad += !__builtin_isfinite(g0) + !__builtin_isfinite(v0) +
                                           !__builtin_isfinite(g1) + !__builtin_isfinite(v1);
                                v[r] = pack_f16(mul_f32(silu_f32(g0), v0), mul_f32(silu_f32(g1), v1));
                            }
                            *reinterpret_cast<u32x4 *>(pb + (size_t)m * epi.ldpw + 8 * q) = v;
                        }
                    }
                }
            } else {
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
                    const int cb = wb + nt * 32; // wave-uniform
                    if (cb >= N) continue;
                    if (cb >= epi.split) {
                        uint32_t *const pb = epi.pk + ((cb - epi.split) >> 5) * 16 + 4 * g;
#pragma unroll
                        for (int mt = 0; mt < C::MT; ++mt) {
                            const int m = m0 + mt * 32 + li;
                            if (m >= M) continue;
#pragma unroll
                            for (int q = 0; q < 2; ++q) {
                                u32x4 v;
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    const float y0 = acc[mt][nt][4 * q + r], y1 = acc[mt][nt][4 * q + 8 + r];
                                    if (cnt) bad += !__builtin_isfinite(y0) + !__builtin_isfinite(y1);
                                    v[r] = epi.act ? pack_f16(gelu_tanh(y0), gelu_tanh(y1)) : pack_f16(y0, y1);
                                }
                                *reinterpret_cast<u32x4 *>(pb + (size_t)m * epi.ldpw + 8 * q) = v;
                            }
                        }
                    } else {
#pragma unroll
                        for (int mt = 0; mt < C::MT; ++mt) {
                            const int m = m0 + mt * 32 + li;
                            if (m >= M) continue;
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                floatx4 o;
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    o[r] = acc[mt][nt][4 * q + r];
                                    if (cnt) bad += !__builtin_isfinite(o[r]);
                                }
                                *reinterpret_cast<floatx4 *>(out + (size_t)m * ldo + cb + 8 * q + 4 * g) = o;
                            }
                        }
                    }
                }
            }
            count_nonfinite(nonfinite, bad);
            return 1;
        }
        const bool full = vec_store && m0 + BM <= M && n0 + BN <= N;
        if (full) {
            count_tile(bad);
            store_f32_lines(m0, n0, out, 4 * (int)ldo);
        } else {
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) {
                const int m = m0 + mt * 32 + li;
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int n = n0 + wave * WN + nt * 32 + 8 * q + 4 * g;
                        if (m < M) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                if (n + r < N) {
                                    bad += cnt && !__builtin_isfinite(acc[mt][nt][4 * q + r]);
                                    out[(size_t)m * ldo + n + r] = acc[mt][nt][4 * q + r];
                                }
                            }
                        }
                    }
                }
            }
        }
        count_nonfinite(nonfinite, bad);
        return full ? 2 : 1;
    };

    int unit = xcd_tile(blockIdx.x, gridDim.x);
    int m0, n0, kst0;   // tile origin; first global stage of the unit's K range
    float *uout;        // where the unit's epilogue writes
    auto unit_origin = [&](int u) {
        const int split = u / ntiles;
        tile_origin(u - split * ntiles, m0, n0);
        kst0 = split * nstage;
        uout = out + (size_t)split * (size_t)pstride;
    };
    // Row scales of the tile (epi.rsc, range-safe packing): waves 0 .. BM/64
    // - 1 copy the BM values into the tile's parity buffer, ahead of its first
    // stage, so they count as part of that stage in the vmcnt waits.
    const bool rows_scaled = epi.rsc != nullptr && ksplit == 1;
    int parity = 0;
    auto issue_rsc = [&](int par) {
        static_assert(BM % 64 == 0 && BM / 64 <= C::NW, "one wave copies 64 row scales");
        if (rows_scaled && wave < BM / 64)
            dma_lds4(epi.rsc + min(m0 + 64 * wave + lane, M - 1), smem + C::RSC + par * BM * 4 + wave * 256);
    };
    unit_origin(unit);
    setup(m0, n0);
    issue_rsc(parity);
    issue(kst0, 0);
    int prev_stores = 0; // what the previous epilogue left in flight (its return value)
    for (;;) {
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int j = 0; j < C::NTL; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        // Pipeline (stage s in slot s % 3), loads one stage ahead.  At the
        // top of stage s the wave waits for its own loads of stage s, then
        // the barrier publishes every wave's part of stage s and retires all
        // reads of stage s-1, and stage s+1's loads go to slot (s+1) % 3 (its
        // last reader was stage s-2).  Vector memory operations retire in
        // issue order and loads and stores share vmcnt, so "stage s has
        // landed" is "at most the operations issued after it are
        // outstanding": none within a tile; at a tile's first stage the
        // previous tile's 32 (or 16) vector stores per lane, issued after
        // this tile's stage 0 (a gate-residual epilogue also issued loads
        // there, which only adds to the operations after that stage).  Those
        // stores thus drain under the tile's first stage of MFMA work.  A
        // ragged previous tile stored a variable count with scalar stores:
        // wait for everything.  (Loads two stages ahead, the third slot
        // refilled as soon as it is read, measured 0.7-1.1 % slower on the
        // shapes that run this kernel, and so did the next tile's first two
        // stages fetched before the stores.)  Unrolled by three so that
        // slots are compile-time; the stage count is a multiple of three, so
        // the loop has no exit mid-body.
        for (int s = 0; s < nstage; s += STAGES) {
#pragma unroll
            for (int u = 0; u < STAGES; ++u) {
                if (C::COUNT_STORES && s == 0 && u == 0 && prev_stores == 2)
                    wait_vmcnt<(C::COUNT_STORES ? C::EPI_STORES : 0)>();
                else if (C::COUNT_STORES && s == 0 && u == 0 && prev_stores == 3)
                    wait_vmcnt<(C::COUNT_STORES ? C::EPI_STORES / 2 : 0)>();
                else
                    wait_vmcnt<0>();
                lds_barrier();
                // the stage's first fragment reads go out before the next
                // stage's loads, so the loads issue under their latency
                compute(u, [&] {
                    if (s + u + 1 < nstage) issue(kst0 + s + u + 1, (u + 1) % STAGES);
                });
            }
        }

        // Slots 0 and 1 were last read before the final barrier: fetch the
        // next tile's first stage now, then store this tile.
        const int cm0 = m0, cn0 = n0, cpar = parity;
        float *const cout = uout;
        unit += gridDim.x;
        const bool more = unit < nunits;
        if (more) {
            unit_origin(unit);
            setup(m0, n0);
            parity ^= 1;
            issue_rsc(parity);
            issue(kst0, 0);
        }
        if (rows_scaled) {
            // this tile's rows: token m0 + 32 mt + li in every accumulator
            // element of lane (li, g), sub-tile mt; the scales landed before
            // the tile's last barrier (its last stage waits for everything)
            const float *rs = reinterpret_cast<const float *>(smem + C::RSC + cpar * BM * 4);
            float sc[C::MT];
            int any = 0;
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) {
                sc[mt] = rs[32 * mt + li];
                any |= sc[mt] != 1.0f;
            }
            if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[mt][nt][v] *= sc[mt];
            }
        }
        prev_stores = epilogue(cm0, cn0, cout);
        if (!more) break;
    }
}

// ---------------------------------------------------------------- gemm16 --
//
// The same GEMM over 144 x 384 or 128 x 384 tiles with 16x16x32 MFMAs, for
// shapes whose 128 x 512 tiles quantise badly on 256 CUs (gemm_tiles picks):
// at M = 4608 (Flux image + text tokens) N = 3072 gives 216 tiles of
// 128 x 512 (one round at 84 % of the CUs) but exactly 256 of 144 x 384, and
// N = 9216 gives 648 (2.53 rounds, run as 3) but exactly 768 (3 full
// rounds); at M = 4096 (Klein image tokens) N = 3072 gives 192 tiles of
// 128 x 512 but 256 of 128 x 384, N = 9216 2.25 rounds of 128 x 512 (run
// as 2 plus a round of 64-row tiles) but 3 full rounds of 128 x 384.  A
// 144 x 384 tile is 0.84 of a 128 x 512 one, a 128 x 384 tile 0.75.
//
// Eight waves side by side along N, each BM tokens x BN / 8 columns (144 x 48:
// 9 x 3 tiles of 16x16), weights as the MFMA's A operand (16 output columns
// x 32 K), tokens as B.  Lane (li, g) of a 16x16x32 operand holds K indices
// 8g .. 8g + 7 of row li: with the K-slot pairing, dword t of them is
// packed word 4g + t of the 32-element block (elements 4g + t and
// 4g + t + 16), i.e. 16-byte chunk g of the block's 64 bytes of packed
// activations, and on the weight side the sign bits 4g + t and 4g + t + 16:
// the sign word shifted right by 4g, then one shift by 15 - t and one bit
// op per dword, as in the 32x32 kernel.  The accumulator's lane (li, g)
// holds output columns 4g .. 4g + 3 of token li: one 16-byte store.
//
// Pipeline and LDS as in b1_gemm_kernel: K in stages of 128 (4 blocks), a
// three-slot ring fetched one stage ahead with buffer loads straight into
// LDS, one barrier per stage with counted vmcnt waits.  A stage is BM rows
// x 256 bytes of activations (BM / 4 loads of 1 KB) and BN columns x 24
// bytes of weights (BN / 64 column groups, two 12-byte loads each): the
// first BN / 64 waves load a weight group and some activation kilobytes,
// the others only activation kilobytes (144 x 384: 6 loads a wave; 128 x
// 384: 6 and 4).  Activation row r's chunk c sits at position c ^ (r & 15),
// so the 16 lanes of a fragment read (rows li, one chunk) hit distinct
// banks.  Full tiles only (M % BM, N % BN, K % 384 == 0); EPI 0 plain, 1
// gate-residual (GemmEpi); row scales of range-safe packing as in the
// 32x32 kernel.
template <int BM_, int BN_>
struct Gemm16Cfg {
    static constexpr int BM = BM_, BN = BN_, NW = 8, NT = NW * 64;
    static constexpr int WN = BN / NW, MT = BM / 16, NTL = WN / 16;
    static constexpr int STAGES = 3, KC = 128, ROWB = 256;
    static constexpr int ASTAGE = BM * ROWB;            // activation bytes per slot
    static constexpr int NWG = BN / 64;                 // 64-column weight load groups
    static constexpr int BSTAGE = NWG * 2048;           // weight bytes per slot
    static constexpr int ABASE = STAGES * BSTAGE;       // weights first
    static constexpr int RSC = ABASE + STAGES * ASTAGE;
    static constexpr int RSCN = (BM + 63) / 64 * 64;    // row scales per parity (64 per copying wave)
    static constexpr int LDS = RSC + 2 * RSCN * 4;
    static constexpr int GROUP_M = 4;
    // Loads per wave per stage: waves 0 .. NWG - 1 load a weight group (2
    // loads) and AW activation kilobytes, the others AO activation
    // kilobytes; AW is the split with the fewest loads on the busiest wave
    // (144 x 384: 4 + 2 and 6; 128 x 384: 4 + 2 and 4).  The waits count no
    // loads (every wait inside a tile is for everything), so the counts need
    // not be equal.
    static constexpr int ALOADS = ASTAGE / 1024;
    static constexpr int split_aw() {
        int best = -1, cost = 1 << 30;
        for (int aw = 0; aw * NWG <= ALOADS; ++aw) {
            const int rest = ALOADS - aw * NWG;
            if (NW == NWG ? rest != 0 : rest % (NW - NWG) != 0) continue;
            const int ao = NW == NWG ? 0 : rest / (NW - NWG);
            const int c = aw + 2 > ao ? aw + 2 : ao;
            if (c < cost) cost = c, best = aw;
        }
        return best;
    }
    static constexpr int AW = split_aw();
    static constexpr int AO = NW == NWG ? 0 : (ALOADS - AW * NWG) / (NW - NWG);
    static constexpr int LOADS = AW > AO ? AW : AO;    // activation offsets a wave keeps
    static constexpr int EPI_STORES = MT * NTL;         // 16-byte stores per lane, full tile
    static_assert(BM % 16 == 0 && WN % 16 == 0 && BN % 64 == 0 && NWG <= NW, "tile shape");
    static_assert(AW >= 0 && AW * NWG + AO * (NW - NWG) == ALOADS, "the loads cover the stage");
    static_assert(LDS <= 160 * 1024, "gfx950 LDS");
    static_assert(EPI_STORES <= 63, "vmcnt holds 6 bits");
    static_assert((MT - 1) * 16 * ROWB + 16 * ROWB <= 65536, "fragment immediates");
};

template <int BM, int BN, int EPI>
__global__ __launch_bounds__((Gemm16Cfg<BM, BN>::NT), 2) void b1_gemm16_kernel(const uint16_t *__restrict__ ah,
                                                                     const uint8_t *__restrict__ w, int K, int N, int M,
                                                                     float *__restrict__ out, int64_t ldo,
                                                                     int32_t *nonfinite, int tiles_m, int tiles_n,
                                                                     int vec_store, GemmEpi epi) {
    using C = Gemm16Cfg<BM, BN>;
    static_assert(EPI >= 0 && EPI <= 3, "plain, gate-residual, SwiGLU and packed-output epilogues");
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, g = lane >> 4;
    const int nstage = K / C::KC; // a multiple of STAGES
    const int ntiles = tiles_m * tiles_n;
    const uint32_t rs = (uint32_t)(K / 32) * 6;

    auto tile_origin = [&](int t, int &m0, int &n0) {
        const int group = t / (C::GROUP_M * tiles_n);
        const int first_m = group * C::GROUP_M;
        const int gsize = min(C::GROUP_M, tiles_m - first_m);
        const int tin = t - first_m * tiles_n;
        m0 = (first_m + tin % gsize) * C::BM;
        n0 = (tin / gsize) * C::BN;
    };

    // Loads of a stage.  Activation load j (0 .. BM / 4 - 1) fills LDS bytes
    // [1024 j, +1024) of the slot: rows 4j .. 4j + 3, lane L at position
    // L % 16 of row 4j + L / 16, holding chunk (L % 16) ^ (row & 15).  Waves
    // w < NWG issue loads AW w .. + AW - 1, the others AW NWG + AO (w - NWG)
    // .. + AO - 1.  Weight group q (waves q < NWG): lane L fetches 12 bytes
    // (blocks 0-1, then 2-3 of the stage) of column n0 + 64 q + L.  Rows and
    // columns past the matrix cannot occur (full tiles).
    // whether tile column n0's columns are SwiGLU [gate | value] pairs (EPI 2,
    // or EPI 3 with act 2 from split on; split % BN == 0 there)
    auto swiglu_tile = [&](int n0) { return EPI == 2 || (EPI == 3 && epi.act == 2 && n0 >= epi.split); };
    // whether tile column n0 is wholly packed GELU or plain (EPI 3, act 0 or
    // 1, from split on)
    auto packed_tile = [&](int n0) { return EPI == 3 && epi.act != 2 && n0 >= epi.split; };
    const bool wload = wave < C::NWG;
    const int a_first = wload ? C::AW * wave : C::AW * C::NWG + C::AO * (wave - C::NWG);
    uint32_t aoff[C::LOADS];
    uint32_t boff = 0;
    auto setup = [&](int m0, int n0) {
#pragma unroll
        for (int i = 0; i < C::LOADS; ++i) {
            const int row = 4 * (a_first + i) + (lane >> 4);
            const int c = (lane & 15) ^ (row & 15);
            aoff[i] = ((uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)c * 8) * 2;
        }
        int row = n0 + 64 * (wload ? wave : 0) + lane;
        if (swiglu_tile(n0)) {
            // SwiGLU: the tile's 24 16-column tiles are the gates and the
            // values of its 192 outputs in 12 groups of 16.  Waves 4h + r,
            // r < 3, hold [gate 6h + 2r, its value, gate 6h + 2r + 1]
            // (groups 6h + 2r and 6h + 2r + 1 are packed block 3h + r);
            // wave 4h + 3 holds the values of groups 6h + 1, 6h + 3 and
            // 6h + 5 (the epilogue passes them to the block's wave).  Each
            // weight row keeps its place within its 16-column MFMA tile.
            const int base = EPI == 3 ? epi.split : 0;
            const int tc = row - n0, sub = tc >> 4, pos = tc & 15;
            const int w = sub / 3, t = sub - 3 * w, h = w >> 2, r = w & 3;
            const int grp = r < 3 ? 6 * h + 2 * r + (t == 2) : 6 * h + 2 * t + 1;
            const bool value = r < 3 ? t == 1 : true;
            row = base + (value ? epi.glu_h : 0) + (n0 - base) / 2 + 16 * grp + pos;
        } else if (packed_tile(n0)) {
            // Packed columns: the tile's 12 blocks of 32 columns, each a low
            // and a high 16-column half.  Waves 4h + r, r < 3, hold [low and
            // high half of block 6h + 2r, low half of block 6h + 2r + 1];
            // wave 4h + 3 holds the high halves of blocks 6h + 1, 6h + 3 and
            // 6h + 5 (the epilogue passes them on).  Each weight row keeps
            // its place within its 16-column MFMA tile.
            const int tc = row - n0, sub = tc >> 4, pos = tc & 15;
            const int w = sub / 3, t = sub - 3 * w, h = w >> 2, r = w & 3;
            const int blk = 6 * h + (r < 3 ? 2 * r + (t == 2) : 2 * t + 1);
            const int half = r < 3 ? t == 1 : 1;
            row = n0 + 32 * blk + 16 * half + pos;
        }
        boff = (uint32_t)row * rs;
    };
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(ah), (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), kBufferFlags);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w), (short)0, (int)((uint32_t)N * rs), kBufferFlags);
    auto issue = [&](int ks, int slot) {
        uint8_t *sa = smem + C::ABASE + slot * C::ASTAGE + a_first * 1024;
        const uint32_t aso = (uint32_t)ks * C::ROWB, wso = (uint32_t)ks * 24;
        if (wload) {
#pragma unroll
            for (int i = 0; i < C::AW; ++i) dma_buf_lds16s(ars, sa + i * 1024, aoff[i], aso);
            uint8_t *sw = smem + slot * C::BSTAGE + wave * 2048;
            dma_buf_lds12s(wrs, sw, boff, wso);
            dma_buf_lds12s(wrs, sw + 1024, boff, wso + 12);
        } else {
#pragma unroll
            for (int i = 0; i < C::AO; ++i) dma_buf_lds16s(ars, sa + i * 1024, aoff[i], aso);
        }
    };

    // Fragment addresses.  Activations: lane (li, g), block j of the stage,
    // row tile mt: row 16 mt + li, chunk 4 j + g at position (4 j + g) ^ li,
    // 256-byte rows; one LDS pointer per (slot, j), the row tile an
    // immediate.  Weights: the wave's 16-column chunk q = 3 wave + nt of the
    // tile lies in load group q / 4 at column (q % 4) 16 + li, 16 bytes a
    // column in each 1 KB half.
    typedef const __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8 *const lbase = (lds_u8 *)smem;
    // Slots 0 and 1 share one pointer set (slot 1 an immediate away) when
    // their offsets stay below the 64 KiB immediate range; slot 2 has its own.
    constexpr bool SHARE01 = C::ASTAGE + (C::MT - 1) * 16 * C::ROWB < 65536;
    lds_u8 *fa[2][4];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            fa[sl][j] = lbase + C::ABASE + (sl ? 2 : 0) * C::ASTAGE + li * C::ROWB + (((4 * j + g) ^ li) * 16);
    auto frag_ptr = [&](int slot, int j) -> lds_u8 * {
        if constexpr (SHARE01) return slot == 2 ? fa[1][j] : fa[0][j] + slot * C::ASTAGE;
        return fa[0][j] + slot * C::ASTAGE;
    };
    // Weights: with 4 column tiles a wave (NTL % 4 == 0) they are one load
    // group's consecutive 256-byte quarters, an immediate apart.
    lds_u8 *qw[C::NTL % 4 == 0 ? 1 : C::NTL];
    if constexpr (C::NTL % 4 == 0) {
        qw[0] = lbase + (C::NTL * wave >> 2) * 2048 + li * 16;
    } else {
#pragma unroll
        for (int nt = 0; nt < C::NTL; ++nt) {
            const int q = C::NTL * wave + nt;
            qw[nt] = lbase + (q >> 2) * 2048 + ((q & 3) * 16 + li) * 16;
        }
    }
    auto wcol_ptr = [&](int nt) -> lds_u8 * {
        if constexpr (C::NTL % 4 == 0) return qw[0] + (nt >> 2) * 2048 + (nt & 3) * 256;
        return qw[nt];
    };

    floatx4 acc[C::MT][C::NTL];

    // One stage: 4 steps (blocks) x MT row tiles.  The wave's weight dwords
    // of blocks 0-1 are read at the stage top and those of blocks 2-3, into
    // the same registers, once step 1's weights have been expanded (during
    // step 0); activation fragments stream through a ring of 4, three row
    // tiles ahead (across steps); the weights of step j + 1 are expanded one
    // 16-column tile per row tile at the start of step j, while its MFMAs
    // run.  A scheduling fence per row tile keeps the compiler from hoisting
    // every read of the stage.
    static_assert(C::NTL + 1 < C::MT, "weight reads of blocks 2-3 inside step 0");
    auto compute = [&](int slot, auto &&after_first_reads) {
        uint32_t d[C::NTL][3];
        auto read_w = [&](int bp) {
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt) {
                const __attribute__((address_space(3))) uint32_t *q =
                    reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(
                        wcol_ptr(nt) + slot * C::BSTAGE + bp * 1024);
                d[nt][0] = q[0];
                d[nt][1] = q[1];
                d[nt][2] = q[2];
            }
        };
        read_w(0);
        constexpr int R = 4, DIST = 3, NF = 4 * C::MT;
        half8 af[R];
        auto read_frag = [&](int f) {
            const int j = f / C::MT, mt = f % C::MT;
            af[f % R] = *reinterpret_cast<const __attribute__((address_space(3))) half8 *>(frag_ptr(slot, j) +
                                                                                            mt * 16 * C::ROWB);
        };
#pragma unroll
        for (int f = 0; f < DIST; ++f) read_frag(f);
        after_first_reads();
        // LATE: with 4 column tiles a wave, one buffer of expanded weights:
        // tile nt of step j + 1 is expanded into tile nt's registers right
        // after step j's last MFMA with them (two buffers would not fit
        // beside 128 accumulators without spills)
        constexpr bool LATE = C::NTL >= 4;
        u32x4 bw[LATE ? 1 : 2][C::NTL];
        // block j's scale and sign word sit at 6 (j % 2) bytes into the
        // 12-byte pair held in d
        auto expand = [&](int j, int nt, u32x4 &bo) {
            const uint32_t *dd = d[nt];
            uint32_t s2, wg;
            if ((j & 1) == 0) {
                s2 = dup_lo16(dd[0]);
                // the sign word of block j, shifted right by 4g (bits above
                // 27 are not those of the plain shift; only bits t and
                // 16 + t, t < 4, reach the mask)
                wg = __builtin_amdgcn_alignbit(dd[1], dd[0], 16 + 4 * g);
            } else {
                s2 = dup_hi16(dd[1]);
                wg = dd[2] >> (4 * g);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) bo[t] = wpair(wg, 15 - t, s2);
        };
#pragma unroll
        for (int nt = 0; nt < C::NTL; ++nt) expand(0, nt, bw[0][nt]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int j = f / C::MT, mt = f % C::MT;
            if (f + DIST < NF) read_frag(f + DIST);
            if constexpr (LATE) {
                if (j == 1 && mt == 0) read_w(1);
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, bw[0][nt]),
                                                                         af[f % R], acc[mt][nt], 0, 0, 0);
                    if (j + 1 < 4 && mt == C::MT - 1) expand(j + 1, nt, bw[0][nt]);
                }
            } else {
                if (j + 1 < 4 && mt < C::NTL) expand(j + 1, mt, bw[(j + 1) & 1][mt]);
                if (j == 0 && mt == C::NTL) read_w(1);
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, bw[j & 1][nt]),
                                                                         af[f % R], acc[mt][nt], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    auto count_tile = [&](int &bad) {
        if (nonfinite != nullptr) {
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) bad += !__builtin_isfinite(acc[mt][nt][v]);
        }
    };
    auto stride_bytes = [](int64_t ld) {
        int b = (int)ld * 4;
        asm volatile("" : "+s"(b));
        return b;
    };
    // Lane (li, g) of tile (mt, nt): token m0 + 16 mt + li, columns
    // n0 + WN wave + 16 nt + 4 g .. + 3: one 16-byte store each (MT NTL per
    // lane), half a line per 4 lanes.  Without vec_store (out, or the
    // residual and gate, or the packed rows, not 16-byte aligned) the same
    // values go out as scalar stores.  Returns the vector stores per lane it
    // left in flight (0 after scalar stores).
    auto epilogue = [&](int m0, int n0) -> int {
        int bad = 0;
        count_tile(bad);
        if constexpr (EPI == 2 || EPI == 3) {
            if (swiglu_tile(n0)) {
                // SwiGLU (the layout of setup): wave 4h + 3 passes its three
                // value tiles through LDS (slots 1 and 2's activation area:
                // slot 1's is idle from the last stage's barrier to the next
                // tile's first, slot 2's once every wave has finished the
                // last stage, hence the barrier before the writes); wave
                // 4h + r, r < 3, then holds block 3h + r: low
                // group silu(tile 0) * tile 1, high group silu(tile 2) *
                // the passed values, silu(gate) * value as the producer pass
                // computes it, and stores it row tile by row tile (fp32: two
                // 16-byte stores, the line's halves; packed: one, dwords
                // 4g .. 4g + 3 of the block's row).
                static_assert(C::NTL == 3 && C::NW == 8 && 6 * C::MT * 1024 <= 2 * C::ASTAGE, "the SwiGLU exchange");
                typedef __attribute__((address_space(3))) uint8_t lds8;
                typedef __attribute__((address_space(3))) floatx4 lds_f4;
                const int h = wave >> 2, r = wave & 3;
                lds8 *const xa = (lds8 *)smem + C::ABASE + C::ASTAGE + h * (3 * C::MT * 1024) + lane * 16;
                // the area runs into slot 2's, which slower waves may still
                // be reading for the tile's last stage
                lds_barrier();
                if (r == 3) {
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                        for (int t = 0; t < 3; ++t) *(lds_f4 *)(xa + (t * C::MT + mt) * 1024) = acc[mt][t];
                }
                wait_lgkmcnt0();
                lds_barrier();
                if (r == 3) {
                    count_nonfinite(nonfinite, bad);
                    return 0;
                }
                // the block's first output
                const int ob = (n0 - (EPI == 3 ? epi.split : 0)) / 2 + 32 * (3 * h + r);
                auto swiglu = [&](float gt, float vl) { return mul_f32(silu_f32(gt), vl); };
                // the block's low and high outputs of row tile mt, element e
                auto block_out = [&](int mt, floatx4 &lo, floatx4 &hi) {
                    const floatx4 v = *(const lds_f4 *)(xa + (r * C::MT + mt) * 1024);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo[e] = swiglu(acc[mt][0][e], acc[mt][1][e]);
                        const float ve = v[e];
                        hi[e] = swiglu(acc[mt][2][e], ve);
                    }
                };
                if constexpr (EPI == 2) {
                    if (!vec_store) {
#pragma unroll
                        for (int mt = 0; mt < C::MT; ++mt) {
                            floatx4 lo, hi;
                            block_out(mt, lo, hi);
                            const size_t m = (size_t)(m0 + 16 * mt + li);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                out[m * ldo + ob + 4 * g + e] = lo[e];
                                out[m * ldo + ob + 16 + 4 * g + e] = hi[e];
                            }
                        }
                        count_nonfinite(nonfinite, bad);
                        return 0;
                    }
                    const int ldb = stride_bytes(ldo);
                    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
                        out + (size_t)m0 * ldo, (short)0, (int)(C::BM * ldo * 4), kBufferFlags);
                    const int lvoff = li * ldb + 16 * g;
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt) {
                        floatx4 lo, hi;
                        block_out(mt, lo, hi);
                        u32x4 a, b;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x0 = lo[e], x1 = hi[e];
                            a[e] = __builtin_bit_cast(uint32_t, x0);
                            b[e] = __builtin_bit_cast(uint32_t, x1);
                        }
                        store16_guarded<kStoreNT>(a, ors, lvoff, mt * 16 * ldb + ob * 4);
                        store16_guarded<kStoreNT>(b, ors, lvoff, mt * 16 * ldb + ob * 4 + 64);
                    }
                    count_nonfinite(nonfinite, bad);
                    return 2 * C::MT;
                } else {
                    // packed: output column c of a row is half (c / 16) % 2 of
                    // dword 16 (c / 32) + c % 16: the block is dwords ob / 2 ..
                    // + 15 of the row
                    if (!vec_store) {
#pragma unroll
                        for (int mt = 0; mt < C::MT; ++mt) {
                            floatx4 lo, hi;
                            block_out(mt, lo, hi);
                            const size_t m = (size_t)(m0 + 16 * mt + li);
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                epi.pk[m * epi.ldpw + ob / 2 + 4 * g + e] = pack_f16_rounded(lo[e], hi[e]);
                        }
                        count_nonfinite(nonfinite, bad);
                        return 0;
                    }
                    const int lpb = stride_bytes(epi.ldpw);
                    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                        epi.pk + (size_t)m0 * epi.ldpw, (short)0, (int)(C::BM * epi.ldpw * 4), kBufferFlags);
                    const int lpoff = li * lpb + 16 * g;
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt) {
                        floatx4 lo, hi;
                        block_out(mt, lo, hi);
                        u32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = pack_f16_rounded(lo[e], hi[e]);
                        store16_guarded<0>(v, prs, lpoff, mt * 16 * lpb + ob * 2);
                    }
                    count_nonfinite(nonfinite, bad);
                    return C::MT;
                }
            }
        }
        if constexpr (EPI == 3) {
            if (packed_tile(n0)) {
                // A wholly packed tile (the layout of setup): wave 4h + 3
                // applies the activation to its three high halves and passes
                // them through LDS (slots 1 and 2's activation area, after a
                // barrier: slot 2 holds the last stage);
                // wave 4h + r, r < 3, then holds blocks 6h + 2r and 6h + 2r +
                // 1, a 128-byte line of each row, and stores it row tile by
                // row tile as two 16-byte stores (dwords 4g .. 4g + 3 of each
                // block).
                static_assert(C::NTL == 3 && C::NW == 8 && 6 * C::MT * 1024 <= 2 * C::ASTAGE, "the block exchange");
                typedef __attribute__((address_space(3))) uint8_t lds8;
                typedef __attribute__((address_space(3))) floatx4 lds_f4;
                auto act = [&](float y) { return epi.act ? gelu_tanh(y) : y; };
                const int h = wave >> 2, r = wave & 3;
                lds8 *const xa = (lds8 *)smem + C::ABASE + C::ASTAGE + h * (3 * C::MT * 1024) + lane * 16;
                lds_barrier(); // (as in the SwiGLU exchange: slot 2's area)
                if (r == 3) {
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                        for (int t = 0; t < 3; ++t) {
                            floatx4 v;
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = act(acc[mt][t][e]);
                            *(lds_f4 *)(xa + (t * C::MT + mt) * 1024) = v;
                        }
                }
                wait_lgkmcnt0();
                lds_barrier();
                if (r == 3) {
                    count_nonfinite(nonfinite, bad);
                    return 0;
                }
                // the line's first byte in the packed row: block 6h + 2r
                const int cb = (n0 - epi.split) * 2 + 64 * (6 * h + 2 * r);
                auto line = [&](int mt, u32x4 &a, u32x4 &b) {
                    const floatx4 v = *(const lds_f4 *)(xa + (r * C::MT + mt) * 1024);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float ve = v[e];
                        a[e] = pack_f16_rounded(act(acc[mt][0][e]), act(acc[mt][1][e]));
                        b[e] = pack_f16_rounded(act(acc[mt][2][e]), ve);
                    }
                };
                if (!vec_store) {
#pragma unroll
                    for (int mt = 0; mt < C::MT; ++mt) {
                        u32x4 a, b;
                        line(mt, a, b);
                        uint32_t *rowp = epi.pk + (size_t)(m0 + 16 * mt + li) * epi.ldpw + cb / 4 + 4 * g;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            rowp[e] = a[e];
                            rowp[16 + e] = b[e];
                        }
                    }
                    count_nonfinite(nonfinite, bad);
                    return 0;
                }
                const int lpb = stride_bytes(epi.ldpw);
                const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                    epi.pk + (size_t)m0 * epi.ldpw, (short)0, (int)(C::BM * epi.ldpw * 4), kBufferFlags);
                const int lpoff = li * lpb + 16 * g;
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt) {
                    u32x4 a, b;
                    line(mt, a, b);
                    store16_guarded<0>(a, prs, lpoff, mt * 16 * lpb + cb);
                    store16_guarded<0>(b, prs, lpoff, mt * 16 * lpb + cb + 64);
                }
                count_nonfinite(nonfinite, bad);
                return 2 * C::MT;
            }
            // A tile of fp32 columns, or one the split point crosses (the
            // plain layout).  Columns below epi.split: fp32 into out.  From
            // split on: fp16 (of GELU-tanh when epi.act) into the packed rows of epi.pk
            // (ldpw dwords apart), as the next linear reads them: column
            // split + 32 b + e of a row is half e / 16 of dword 16 b + e % 16.
            // split % 32 == 0 and tiles are 16-column aligned, so a tile is
            // one half of one block, and lane (li, g) holds that half of
            // dwords 16 b + 4 g .. + 3.  When the block's other half is in
            // the same wave the low tile writes the four dwords as one
            // 16-byte store; a half whose partner lies in the next or the
            // previous wave (a wave has 3 tiles) goes out as four 2-byte
            // stores, the two halves meeting in L2.
            const int wb = n0 + C::WN * wave; // wave-uniform
            auto act = [&](float y) { return epi.act ? gelu_tanh(y) : y; };
            if (!vec_store) {
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const size_t m = (size_t)(m0 + 16 * mt + li);
                            const int n = wb + 16 * nt + 4 * g + e;
                            const float y = acc[mt][nt][e];
                            if (n < epi.split) {
                                out[m * ldo + n] = y;
                            } else {
                                const int c = n - epi.split;
                                const uint16_t h = half_bits(act(y));
                                reinterpret_cast<uint16_t *>(epi.pk + m * epi.ldpw + (c >> 5) * 16 + (c & 15))[(c >> 4) & 1] = h;
                            }
                        }
                count_nonfinite(nonfinite, bad);
                return 0;
            }
            const int ldb = stride_bytes(ldo), lpb = stride_bytes(epi.ldpw);
            const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
                out + (size_t)m0 * ldo, (short)0, (int)(C::BM * ldo * 4), kBufferFlags);
            const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                epi.pk + (size_t)m0 * epi.ldpw, (short)0, (int)(C::BM * epi.ldpw * 4), kBufferFlags);
            const int lvoff = li * ldb + 16 * g, lpoff = li * lpb + 16 * g;
            // Each tile's part, decided once (wave-uniform): 0 fp32, 1 the low
            // half of a block whose high half is the next tile (one 16-byte
            // store for both), 2 that high half (nothing more), 3 a lone
            // half (2-byte stores).  The stores go out row tile by row tile,
            // so the two halves of a 128-byte line leave within a few
            // instructions of each other, in this wave or in its neighbour:
            // ordered tile by tile, 30 % more bytes reached memory (lines
            // written in parts).
            int kind[C::NTL], off[C::NTL];
            int nst = 0; // vector stores per lane (wave-uniform)
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt) {
                const int cb = wb + 16 * nt; // the tile's first column
                const int c = cb - epi.split, hi = (c >> 4) & 1;
                if (cb < epi.split) {
                    kind[nt] = 0;
                    off[nt] = cb * 4;
                    nst += C::MT;
                } else if (hi == 0 && nt + 1 < C::NTL) {
                    kind[nt] = 1;
                    off[nt] = (c >> 5) * 64; // the block's first dword, in bytes
                    nst += C::MT;
                } else if (hi == 1 && nt > 0) {
                    kind[nt] = 2;
                    off[nt] = 0;
                } else {
                    kind[nt] = 3;
                    off[nt] = (c >> 5) * 64 + 2 * hi;
                    nst += 4 * C::MT;
                }
            }
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
                    if (kind[nt] == 0) {
                        u32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x = acc[mt][nt][e];
                            v[e] = __builtin_bit_cast(uint32_t, x);
                        }
                        store16_guarded<kStoreNT>(v, ors, lvoff, mt * 16 * ldb + off[nt]);
                    } else if (kind[nt] == 1) {
                        u32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float y0 = acc[mt][nt][e], y1 = acc[mt][(nt + 1) % C::NTL][e];
                            v[e] = pack_f16(act(y0), act(y1));
                        }
                        store16_guarded<0>(v, prs, lpoff, mt * 16 * lpb + off[nt]);
                    } else if (kind[nt] == 3) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float y = acc[mt][nt][e];
                            const uint16_t h = half_bits(act(y));
                            __builtin_amdgcn_raw_buffer_store_b16(h, prs, lpoff, mt * 16 * lpb + off[nt] + 4 * e,
                                                                  0);
                        }
                    }
                }
            count_nonfinite(nonfinite, bad);
            return nst;
        }
        if (!vec_store) {
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const size_t m = (size_t)(m0 + 16 * mt + li);
                        const int n = n0 + C::WN * wave + 16 * nt + 4 * g + e;
                        float y = acc[mt][nt][e];
                        if constexpr (EPI == 1) y = gate_residual(epi.res[m * epi.ldr + n], epi.gate[n], y);
                        out[m * ldo + n] = y;
                    }
            count_nonfinite(nonfinite, bad);
            return 0;
        }
        const int ldb = stride_bytes(ldo);
        const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
            out + (size_t)m0 * ldo + n0 + C::WN * wave, (short)0, (int)(C::BM * ldo * 4), kBufferFlags);
        const int lvoff = li * ldb + 16 * g;
        if constexpr (EPI == 0) {
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NTL; ++nt) {
                    u32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x = acc[mt][nt][e];
                        v[e] = __builtin_bit_cast(uint32_t, x);
                    }
                    store16_guarded<kStoreNT>(v, ors, lvoff, mt * 16 * ldb + nt * 64);
                }
        } else {
            // out = residual + gate[n] * y, the residual read at the same
            // places P tiles ahead; it may be `out` itself: each element is
            // read by the lane that writes it, before that write
            const int lrb = stride_bytes(epi.ldr);
            const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(epi.res) + (size_t)m0 * epi.ldr + n0 + C::WN * wave, (short)0,
                (int)(C::BM * epi.ldr * 4), kBufferFlags);
            const int lroff = li * lrb + 16 * g;
            floatx4 gq[C::NTL];
#pragma unroll
            for (int nt = 0; nt < C::NTL; ++nt)
                gq[nt] = *reinterpret_cast<const floatx4 *>(epi.gate + n0 + C::WN * wave + 16 * nt + 4 * g);
            constexpr int NP = C::MT * C::NTL, P = 6;
            u32x4 rv[NP];
            auto load_res = [&](int p) {
                const int mt = p / C::NTL, nt = p % C::NTL;
                rv[p] = __builtin_amdgcn_raw_buffer_load_b128(rrs, lroff, mt * 16 * lrb + nt * 64, 0);
            };
#pragma unroll
            for (int p = 0; p < P; ++p) load_res(p);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                if (p + P < NP) load_res(p + P);
                const int mt = p / C::NTL, nt = p % C::NTL;
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // elements copied out before any bit cast (a bit cast of
                    // a vector element reads element 0 in this clang)
                    const float y = acc[mt][nt][e];
                    const uint32_t ru = rv[p][e];
                    const float ov = gate_residual(__builtin_bit_cast(float, ru), gq[nt][e], y);
                    o[e] = __builtin_bit_cast(uint32_t, ov);
                }
                store16_guarded<kStoreNT>(o, ors, lvoff, mt * 16 * ldb + nt * 64);
            }
        }
        count_nonfinite(nonfinite, bad);
        return C::EPI_STORES;
    };

    int unit = xcd_tile(blockIdx.x, gridDim.x);
    int m0, n0;
    const bool rows_scaled = epi.rsc != nullptr;
    int parity = 0;
    // Row scales of the tile: waves 0 .. RSCN / 64 - 1 copy 64 each (entries
    // past BM are never read), ahead of the tile's first stage.  The
    // buffer form of the copy: with a global-form LDS copy in the kernel the
    // compiler makes every LDS wait a full lgkmcnt(0), which here would also
    // wait for the fragment reads issued ahead.
    const __amdgpu_buffer_rsrc_t rsrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(epi.rsc), (short)0, rows_scaled ? M * 4 : 0, kBufferFlags);
    auto issue_rsc = [&](int par) {
        if (rows_scaled && wave < C::RSCN / 64)
            dma_buf_lds4(rsrs, smem + C::RSC + par * C::RSCN * 4 + wave * 256,
                         (uint32_t)min(m0 + 64 * wave + lane, M - 1) * 4u);
    };
    tile_origin(unit, m0, n0);
    setup(m0, n0);
    issue_rsc(parity);
    issue(0, 0);
    // what the previous epilogue left in flight: EPI_STORES vector stores per
    // lane, or (a SwiGLU tile, or a packed-output wave that wrote one or two
    // blocks) MT
    bool prev_stores = false, prev_part = false;
    for (;;) {
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int j = 0; j < C::NTL; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        // Loads one stage ahead, as in b1_gemm_kernel.  At the top of stage s
        // the wave waits for its own loads of stage s (nothing newer, except
        // at a tile's first stage the previous tile's stores, issued after
        // this tile's stage 0; a gate-residual epilogue also issued its loads
        // there, which only adds to the newer operations), then the barrier
        // publishes every wave's part and retires all reads of stage s - 1,
        // and stage s + 1 goes to the slot stage s - 2 held.  (Two stages
        // ahead measured 0.5-1.8 % slower at the M = 4608 shapes.)
        for (int s = 0; s < nstage; s += C::STAGES) {
#pragma unroll
            for (int u = 0; u < C::STAGES; ++u) {
                if (s == 0 && u == 0 && prev_stores)
                    wait_vmcnt<C::EPI_STORES>();
                else if ((EPI == 2 || EPI == 3) && s == 0 && u == 0 && prev_part)
                    wait_vmcnt<C::MT>();
                else
                    wait_vmcnt<0>(); // (after scalar stores, or in the first tile, everything)
                lds_barrier();
                compute(u, [&] {
                    if (s + u + 1 < nstage) issue(s + u + 1, (u + 1) % C::STAGES);
                });
            }
        }
        // Slot 0 was last read before the final barrier: fetch the next
        // tile's first stage now, then store this tile.
        const int cm0 = m0, cn0 = n0, cpar = parity;
        unit += gridDim.x;
        const bool more = unit < ntiles;
        if (more) {
            tile_origin(unit, m0, n0);
            setup(m0, n0);
            parity ^= 1;
            issue_rsc(parity);
            issue(0, 0);
        }
        if (rows_scaled) {
            const float *rsp = reinterpret_cast<const float *>(smem + C::RSC + cpar * C::RSCN * 4);
            float sc[C::MT];
            int any = 0;
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) {
                sc[mt] = rsp[16 * mt + li];
                any |= sc[mt] != 1.0f;
            }
            if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < C::NTL; ++nt)
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[mt][nt][v] *= sc[mt];
            }
        }
        const int ns = epilogue(cm0, cn0);
        prev_stores = ns >= C::EPI_STORES;
        prev_part = (EPI == 2 || EPI == 3) && ns >= C::MT;
        if (!more) break;
    }
}

// Split-K reduction: out[m][n] = sum over s = 0..S-1, in that order, of
// part[s][m][n] (slices pstride apart, rows ldp apart, ldp % 4 == 0), with
// the non-finite count of the sums.
// rsc: row scales of range-safe packing (or nullptr), applied to the sum.
__global__ __launch_bounds__(256) void b1_splitk_reduce_kernel(const float *__restrict__ part, int64_t ldp,
                                                               int64_t pstride, int S, int M, int N,
                                                               float *__restrict__ out, int64_t ldo,
                                                               int32_t *nonfinite, int vec,
                                                               const float *__restrict__ rsc) {
    const int q = (N + 3) / 4; // 4-column units per row
    const int64_t units = (int64_t)M * q;
    int bad = 0;
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
        const int m = (int)(u / q), c = (int)(u - (int64_t)m * q) * 4;
        const float *src = part + (size_t)m * ldp + c;
        floatx4 sum = *reinterpret_cast<const floatx4 *>(src);
        for (int sp = 1; sp < S; ++sp) {
            const floatx4 v = *reinterpret_cast<const floatx4 *>(src + (size_t)sp * pstride);
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[r] += v[r];
        }
        if (rsc) {
            const float sc = rsc[m];
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[r] *= sc;
        }
        float *dst = out + (size_t)m * ldo + c;
        if (vec && c + 4 <= N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) bad += nonfinite && !__builtin_isfinite(sum[r]);
            *reinterpret_cast<floatx4 *>(dst) = sum;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (c + r < N) {
                    bad += nonfinite && !__builtin_isfinite(sum[r]);
                    dst[r] = sum[r];
                }
        }
    }
    count_nonfinite(nonfinite, bad);
}

// ----------------------------------------------------------------- gemv --
//
// Small M (<= 16).  Persistent work-groups (one per CU); wave w owns a K
// slice of kGvBPW blocks and accumulates every 16-row group of its
// work-group over that slice (split-K); the waves' partial tiles are then
// summed in LDS in a fixed order.  MFMA 16x16x32 f16 with the tokens on the
// A side (rows >= M are zero) and the weight rows on the B side.
//
// Block-interleaved K: inside a quad of 4 consecutive blocks, lane group g
// (lanes 16g..16g+15) always works on block 4q+g, and MFMA t (t = 0..3) of
// the quad covers fp16 dwords 4t..4t+3 of that block (elements d and d+16,
// d = 4t..4t+3).  Each lane therefore needs only its own 6-byte block of its
// own row, which it fetches as two aligned dwords; all of a wave's weight
// loads are issued before any is consumed, so the kernel pays one HBM round
// trip rather than one per row group.

constexpr int kGvWaves = 8;                    // waves per work-group
constexpr int kGvQuads = 3;                    // 4-block quads per wave per pass
constexpr int kGvBPW = 4 * kGvQuads;           // blocks per wave per pass
constexpr int kGvChunk = kGvWaves * kGvBPW;    // blocks per pass (K 3072)
constexpr int kGvMaxRG = 6;                    // 16-row groups per WG, max
constexpr int kGvAUnits = 6;                   // activation units per lane per batch
constexpr int kGvWaveLds = kGvBPW * 4 * 16 * 16; // fp16 fragments of one wave (12 KB)
constexpr int kGvLds = kGvWaves * kGvWaveLds;  // 96 KB; the reduction reuses it

// Row groups [rg0, rg1) of work-group bid when `groups` are split over nwg
// work-groups as evenly as possible (the first groups % nwg get one more).
// 32-bit: a 64-bit division costs each work-group some 130 scalar
// instructions before its first load.
__device__ __forceinline__ void wg_row_groups(int groups, int nwg, int bid, int &rg0, int &rg1) {
    const int q = groups / nwg, r = groups - q * nwg;
    rg0 = bid * q + min(bid, r);
    rg1 = rg0 + q + (bid < r ? 1 : 0);
}

// The activation slice of a wave (Mp token slots x 12 blocks) is read with
// coalesced float4 loads in units (block, t, token) -- token fastest, so
// each unit pair covers 64 contiguous bytes of one token row -- converted to
// fp16 pairs and written to the wave's LDS area already in MFMA fragment
// order (fragment (q, t) = 64 lanes x 16 bytes), from which every lane then
// reads its 12 fragments with ds_read_b128.
__global__ __launch_bounds__(kGvWaves * 64) void b1_gemv_kernel(LinearArgs p, int groups, int mp_log2) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int nwg = gridDim.x, bid = blockIdx.x;
    int rg0, rg1;
    wg_row_groups(groups, nwg, bid, rg0, rg1);
    const int nrg = rg1 - rg0;
    const int nb = p.K / 32;
    const size_t rs = (size_t)nb * 6;
    const int mp = 1 << mp_log2; // token slots, power of two >= M
    uint8_t *abuf = gsm + wave * kGvWaveLds;
    // Block 4q+g has the parity of g (the slice start and 4q are even).  An
    // even block starts a 4-byte aligned 8-byte window; an odd block sits at
    // byte 2 of the window that starts 2 bytes before it.
    const int odd = g & 1;
    const uint32_t sel_word = odd ? 0x07060504u : 0x05040302u;
    const uint32_t sel_scale = odd ? 0x03020302u : 0x01000100u;

    floatx4 acc[kGvMaxRG];
#pragma unroll
    for (int r = 0; r < kGvMaxRG; ++r) acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int kb0 = 0; kb0 < nb; kb0 += kGvChunk) {
        const int wb0 = kb0 + wave * kGvBPW;

        // Packed weights first, so their latency overlaps the activation
        // traffic: the 6-byte block 4q+g of row (rg0 + r) * 16 + col.
        uint32_t wd[kGvMaxRG][kGvQuads][2];
#pragma unroll
        for (int r = 0; r < kGvMaxRG; ++r) {
            const int n = (rg0 + r) * 16 + col;
#pragma unroll
            for (int q = 0; q < kGvQuads; ++q) {
                const int blk = wb0 + 4 * q + g;
                if (r < nrg && n < p.N && blk < nb) {
                    const uint32_t *src = reinterpret_cast<const uint32_t *>(
                        p.w + (size_t)n * rs + (size_t)blk * 6 - 2 * odd);
                    wd[r][q][0] = src[0];
                    wd[r][q][1] = src[1];
                } else {
                    wd[r][q][0] = wd[r][q][1] = 0u;
                }
            }
        }

        // Activations -> fp16 fragments in LDS.  Unit u = (bl*4 + t)*mp + tok
        // loads a[tok][32 (wb0+bl) + 4t .. +3] and the 4 elements 16 later.
        const int units = 48 << mp_log2;
        for (int base = 0; base < units; base += 64 * kGvAUnits) {
            floatx4 lo[kGvAUnits], hi[kGvAUnits];
#pragma unroll
            for (int i = 0; i < kGvAUnits; ++i) {
                const int u = min(base + i * 64 + lane, units - 1);
                const int tok = min(u & (mp - 1), p.M - 1);
                const int bt = u >> mp_log2;
                const int blk = min(wb0 + (bt >> 2), nb - 1);
                const float *src = p.act + (size_t)tok * p.lda + (size_t)blk * 32 + 4 * (bt & 3);
                lo[i] = *reinterpret_cast<const floatx4 *>(src);
                hi[i] = *reinterpret_cast<const floatx4 *>(src + 16);
            }
#pragma unroll
            for (int i = 0; i < kGvAUnits; ++i) {
                const int u = base + i * 64 + lane;
                const int tok = u & (mp - 1), bt = u >> mp_log2;
                const int bl = bt >> 2, t = bt & 3;
                if (u < units) {
                    const bool ok = wb0 + bl < nb;
                    u32x4 v;
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = ok ? pack_f16(lo[i][j], hi[i][j]) : 0u;
                    *reinterpret_cast<u32x4 *>(abuf + ((((bl >> 2) * 4 + t) * 64) + (bl & 3) * 16 + tok) * 16) = v;
                }
            }
        }
        // Same-wave LDS accesses complete in order; no barrier is needed
        // between this wave's writes and its reads.
        u32x4 af[kGvQuads][4];
#pragma unroll
        for (int q = 0; q < kGvQuads; ++q)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const u32x4 v = *reinterpret_cast<const u32x4 *>(abuf + ((q * 4 + t) * 64 + lane) * 16);
                af[q][t] = col < p.M ? v : u32x4{0u, 0u, 0u, 0u};
            }

#pragma unroll
        for (int q = 0; q < kGvQuads; ++q) {
            uint32_t s2[kGvMaxRG], w[kGvMaxRG];
#pragma unroll
            for (int r = 0; r < kGvMaxRG; ++r) {
                s2[r] = __builtin_amdgcn_perm(wd[r][q][1], wd[r][q][0], sel_scale);
                w[r] = __builtin_amdgcn_perm(wd[r][q][1], wd[r][q][0], sel_word);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < kGvMaxRG; ++r) {
                    if (r < nrg) {
                        u32x4 bd;
#pragma unroll
                        for (int j = 0; j < 4; ++j) bd[j] = wpair(w[r], 15 - 4 * t - j, s2[r]);
                        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8, af[q][t]), __builtin_bit_cast(half8, bd), acc[r], 0, 0, 0);
                    }
                }
            }
        }
    }

    // Cross-wave (split-K) reduction in a fixed order, in LDS reused from the
    // activation fragments, then store.  16x16 accumulator layout: lane
    // column = lane & 15 (weight row), rows 4*(lane >> 4) + v (tokens).
    __syncthreads();
    floatx4 *red = reinterpret_cast<floatx4 *>(gsm); // [wave][rg][lane]
#pragma unroll
    for (int r = 0; r < kGvMaxRG; ++r)
        if (r < nrg) red[(wave * kGvMaxRG + r) * 64 + lane] = acc[r];
    __syncthreads();
    int bad = 0;
    for (int e = tid; e < nrg * 256; e += kGvWaves * 64) {
        const int c = e & 15, tok = (e >> 4) & 15, r = e >> 8;
        const int ln = 16 * (tok >> 2) + c, v = tok & 3;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kGvWaves; ++w) s += red[(w * kGvMaxRG + r) * 64 + ln][v];
        const int n = (rg0 + r) * 16 + c;
        if (tok < p.M && n < p.N) {
            bad += !__builtin_isfinite(s);
            p.out[(size_t)tok * p.ldo + n] = s;
        }
    }
    count_nonfinite(p.nonfinite, bad);
}


// The small-M kernel for K % 256 == 0 (rows are then 16-byte multiples):
// the same per-wave K slices and cross-wave reduction as b1_gemv_kernel, with
// every load a whole-instruction DMA and no work-group barrier before the
// reduction.
//  * Weights: each wave stages, for every row of its work-group's row
//    groups, exactly its own K slice (72 bytes: 12 blocks, fetched as the 5
//    aligned 16-byte chunks that cover it) into its own LDS area, rows 80
//    bytes apart.  A wave therefore waits only for its own DMAs (vmcnt),
//    row group by row group, and never for the other waves.
//  * Activations, packed fp16 (PACKED): fragment (q, t) of the MFMA A
//    operand is 16 token slots x 32 K, S <= 16 slots in use (the power of
//    two >= M).  S <= 8: one 1 KB DMA per slot, the token's 12 blocks as
//    they lie in its row; S = 16: each 1 KB DMA carries one fragment in
//    fragment order (g3_issue_act).  Tokens past M and slots past S zero.
//  * Activations, fp32 (!PACKED): lane (g, tok) takes the 8 elements of its
//    fragment slot (S = 8: from the slot slices DMAs staged in LDS,
//    g3_issue_act_f32; S = 16: straight from the fp32 rows) and converts
//    them to fp16 pairs (round to nearest even) in registers; a lane that
//    met an |a| >= 65520 (beyond the fp16 range) flags its token, and after
//    the reduction the work-group computes its rows of flagged tokens again
//    in the reference's scalar arithmetic (EXACT mode's bits), correcting
//    the non-finite count.  (Loading the fragment slots straight from the
//    rows touches a separate 64-byte line per lane; staging the slices
//    takes 11.1 -> 10.1 us at M=8 K=3072 N=18432.)
//  * Order of the loads: activations first, then the weight row groups, so
//    that vmcnt (which retires in issue order) tells when each has landed.
// One pass covers 96 blocks (K 3072, 12 per wave); longer K runs more
// passes over the same LDS areas.
constexpr int kG3Chunk = kGvWaves * kGvBPW;                    // 96 blocks per pass
constexpr int kG3RowCh = 5;                                    // 16-byte chunks per row per wave
constexpr int kG3RowB = kG3RowCh * 16;                         // 80: wave-private row stride
constexpr int kG3WInst = (kGvMaxRG * 16 * kG3RowCh + 63) / 64; // 8 weight DMAs per wave

// The weight DMAs of a wave's slices: DMA i's lane takes slot 64 i + lane of
// the rows x kG3RowCh chunks, and with 64 = 12 kG3RowCh + 4 that slot is row
// row0 + 12 i + (4 i + ch0) / 5, chunk (4 i + ch0) % 5 (row0, ch0: slot
// lane's).  So each DMA's offset is the lane's base plus a uniform term and
// one select: no division or wide multiply per DMA.
static_assert(kG3RowCh == 5, "slot arithmetic for 5 chunks a row");
struct SliceDmas {
    int row0, ch0;
    uint32_t base, inrow0; // offset and in-row byte of slot lane at K offset 0
    // rows from global row `first`, rs bytes a row; slice0: the wave's first
    // byte in a row
    __device__ __forceinline__ SliceDmas(int lane, int first, uint32_t rs, uint32_t slice0) {
        row0 = lane / kG3RowCh;
        ch0 = lane - row0 * kG3RowCh;
        inrow0 = slice0 + (uint32_t)ch0 * 16u;
        base = (uint32_t)(first + row0) * rs + inrow0;
    }
    // DMA i's offset kofs bytes into the rows, or an out-of-range one for a
    // slot past `rows` rows or past a row's rs bytes
    __device__ __forceinline__ uint32_t off(int i, int rows, uint32_t rs, uint32_t kofs) const {
        const int m = (4 * i) % 5, qi = (4 * i) / 5;
        const bool carry = ch0 + m >= 5;
        const int row = row0 + 12 * i + qi + (carry ? 1 : 0);
        const uint32_t inrow = kofs + inrow0 + 16u * (uint32_t)m - (carry ? 80u : 0u);
        const uint32_t o = base + kofs + (uint32_t)(12 * i + qi) * rs + 16u * (uint32_t)m + (carry ? rs - 80u : 0u);
        return ((row < rows) & (inrow < rs)) ? o : 0xFFFFFFF0u;
    }
};
constexpr int kG3WLds = kG3WInst * 1024;                       // 8 KB of weights per wave
constexpr int kG3ALds = kGvBPW * 1024;                         // 12 KB of fragments per wave
constexpr int kG3WaveLds = kG3WLds + kG3ALds;
constexpr int kG3Lds = kGvWaves * kG3WaveLds;                  // 160 KB
static_assert(kG3Lds <= 160 * 1024, "gfx950 LDS");
static_assert(kGvWaves * kGvMaxRG * 64 * 16 + kGvWaves * 4 <= kG3Lds, "the reduction and its flags fit");
static_assert(kG3RowB >= 72 + 8, "a slice plus its alignment slack");

// Row group R of the chunk being decoded has landed: all DMAs covering its
// rows are done.  AHEAD more DMAs (the next chunk's, in the grouped kernel)
// were issued after them; DMAs retire in issue order.
template <int R, int AHEAD>
__device__ __forceinline__ void g3_wait_rg() {
    constexpr int j = ((R + 1) * 16 * kG3RowCh + 63) / 64;
    wait_vmcnt<kG3WInst - j + AHEAD>();
}
template <int AHEAD>
__device__ __forceinline__ void g3_wait(int r) {
    switch (r) {
    case 0: g3_wait_rg<0, AHEAD>(); break;
    case 1: g3_wait_rg<1, AHEAD>(); break;
    case 2: g3_wait_rg<2, AHEAD>(); break;
    case 3: g3_wait_rg<3, AHEAD>(); break;
    case 4: g3_wait_rg<4, AHEAD>(); break;
    default: g3_wait_rg<5, AHEAD>(); break;
    }
}

// Decode and MFMA of row group r of a pass into its accumulator, from a
// wave's staged rows (wbuf, 80 bytes apart) and its activation fragments af.
// The slice of wave w starts 8 (w odd) bytes into its first chunk; block
// 4q + g sits at 6 (4q + g) bytes into the slice, read as the aligned 8-byte
// window that holds it (2 bytes earlier for odd g).
// FRESH: acc holds nothing yet; the first MFMA adds to a constant zero.
template <bool FRESH = false>
__device__ __forceinline__ void g3_decode_rg(const uint8_t *wbuf, int r, int wave, int lane,
                                             const u32x4 (&af)[kGvQuads][4], floatx4 &acc) {
    const int col = lane & 15, g = lane >> 4, odd = g & 1;
    const uint32_t sel_word = odd ? 0x07060504u : 0x05040302u;
    const uint32_t sel_scale = odd ? 0x03020302u : 0x01000100u;
    const int wshift = 8 * (wave & 1);
    uint32_t wd[kGvQuads][2];
#pragma unroll
    for (int q = 0; q < kGvQuads; ++q) {
        const __attribute__((address_space(3))) uint32_t *src =
            reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(
                (__attribute__((address_space(3))) uint8_t *)wbuf + (r * 16 + col) * kG3RowB + (4 * q + g) * 6 +
                wshift - 2 * odd);
        wd[q][0] = src[0];
        wd[q][1] = src[1];
    }
#pragma unroll
    for (int q = 0; q < kGvQuads; ++q) {
        const uint32_t s2 = __builtin_amdgcn_perm(wd[q][1], wd[q][0], sel_scale);
        const uint32_t w = __builtin_amdgcn_perm(wd[q][1], wd[q][0], sel_word);
        // MFMA t takes pairs 4t .. 4t + 3; one 64-bit shift serves t and t + 2
        u32x4 bd[4];
        wpair_quads<0>(w, w >> 8, s2, bd[0], bd[2]);
        wpair_quads<1>(w, w >> 8, s2, bd[1], bd[3]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, af[q][t]),
                                                         __builtin_bit_cast(half8, bd[t]),
                                                         FRESH && q == 0 && t == 0 ? floatx4{0.f, 0.f, 0.f, 0.f} : acc,
                                                         0, 0, 0);
    }
}

// Row groups [0, nrg) of a pass, each decoded as soon as its own DMAs have
// landed (AHEAD: DMAs issued after this pass's).
template <int AHEAD>
__device__ __forceinline__ void g3_decode(const uint8_t *wbuf, int nrg, int wave, int lane, const u32x4 (&af)[kGvQuads][4],
                                          floatx4 (&acc)[kGvMaxRG]) {
#pragma unroll
    for (int r = 0; r < kGvMaxRG; ++r) {
        if (r < nrg) {
            g3_wait<AHEAD>(r);
            g3_decode_rg(wbuf, r, wave, lane, af, acc[r]);
        }
    }
}

// The activation DMAs of a wave's pass (packed fp16, S slots).  S <= 8: one
// 1 KB DMA per token slot, contiguous in the token's row from the wave's
// first block (its 12 blocks are the first 768 bytes), landing at abuf +
// 1040 t; the row stride of 65 16-byte chunks puts the 8 slots' chunks of a
// fragment read in distinct bank groups.  Lanes past K and slots past M read
// zeros.  (Fragment-ordered DMAs touch a separate 64-byte line per lane, and
// the whole-row form makes the weight DMAs, issued after them, start
// earlier: 8.28 -> 7.97 us per launch at M=8 K=3072 N=18432.)  S = 16: F =
// 16 / S fragments per 1 KB DMA in fragment order, kGvBPW fragments.
constexpr int kG3ARow = 1040;
static_assert(8 * kG3ARow <= kG3ALds, "eight contiguous token rows");
template <int S>
__device__ __forceinline__ void g3_issue_act(__amdgpu_buffer_rsrc_t ars, uint8_t *abuf, int lane, int wb0, int nb, int M,
                                             int K) {
    if constexpr (S <= 8) {
        const uint32_t inrow = (uint32_t)wb0 * 64u + (uint32_t)lane * 16u;
        const bool kin = inrow < (uint32_t)nb * 64u;
#pragma unroll
        for (int t = 0; t < S; ++t)
            dma_buf_lds16(ars, abuf + t * kG3ARow,
                          (kin && t < M) ? (uint32_t)t * (uint32_t)K * 2u + inrow : 0xFFFFFFF0u);
    } else {
        constexpr int F = (16 / S) < kGvBPW ? 16 / S : kGvBPW;
        constexpr int NA = (kGvBPW + F - 1) / F;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int sub = lane / (4 * S), within = lane % (4 * S);
            const int ag = within / S, tok = within % S;
            const int f = i * F + sub;
            const int blk = wb0 + 4 * (f >> 2) + ag;
            const bool ok = f < kGvBPW && tok < M && blk < nb;
            dma_buf_lds16(ars, abuf + i * 1024,
                          ok ? (uint32_t)tok * (uint32_t)K * 2u + (uint32_t)blk * 64u + (uint32_t)(f & 3) * 16u
                             : 0xFFFFFFF0u);
        }
    }
}

template <int S>
__device__ __forceinline__ void g3_read_act(const uint8_t *abuf, int lane, u32x4 (&af)[kGvQuads][4]) {
    const int col = lane & 15, g = lane >> 4;
#pragma unroll
    for (int q = 0; q < kGvQuads; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if constexpr (S <= 8) {
                af[q][t] = col < S ? *reinterpret_cast<const u32x4 *>(abuf + col * kG3ARow + (4 * q + g) * 64 + t * 16)
                                   : u32x4{0u, 0u, 0u, 0u};
            } else {
                constexpr int F = (16 / S) < kGvBPW ? 16 / S : kGvBPW;
                const int f = 4 * q + t;
                af[q][t] = col < S ? *reinterpret_cast<const u32x4 *>(abuf + f / F * 1024 + (f % F * 4 * S + g * S + col) * 16)
                                   : u32x4{0u, 0u, 0u, 0u};
            }
        }
}

// Cross-wave reduction of a chunk's partial tiles (waves' partials at
// `red` + wave * wstride, [rg][lane] floatx4) in wave order, then the
// outputs of row groups [0, nrg) starting at row n0 of out, times the row
// scales rsc when given; the (row, token slot) elements of S slots spread
// over the threads.  Returns the non-finite count.
template <int S>
__device__ __forceinline__ int g3_reduce_store(const uint8_t *red, int wstride, int nrg, int tid, int M, int N, int n0,
                                               float *out, int64_t ldo, const float *rsc) {
    constexpr int SE = 16 * S; // elements of a row group, a power of two
    int bad = 0;
    for (int e = tid; e < nrg * SE; e += kGvWaves * 64) {
        const int c = e & 15, tok = (e % SE) >> 4, r = e / SE;
        const int ln = 16 * (tok >> 2) + c, v = tok & 3;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < kGvWaves; ++w) sum += reinterpret_cast<const floatx4 *>(red + w * wstride)[r * 64 + ln][v];
        const int n = n0 + r * 16 + c;
        if (tok < M && n < N) {
            if (rsc) sum *= rsc[tok];
            bad += !__builtin_isfinite(sum);
            out[(size_t)tok * ldo + n] = sum;
        }
    }
    return bad;
}

// fp32 activations, at most 8 token slots, through LDS: slot t's 12 blocks
// (1536 bytes of its row from the wave's first block) land as chunk c (16
// bytes) of its first 1024 bytes at abuf + 1024 t + 16 (c ^ t), and chunk c
// of its last 512 bytes at abuf + 8192 + 1024 (t / 2) + 512 (t % 2) +
// 16 (c ^ t): two slots' tails share one DMA.  The XOR puts the 8 slots'
// copies of one chunk in distinct bank groups.  Chunks past K and slots past
// M read zeros.  frs: the rows, (M - 1) lda + K floats.
__device__ __forceinline__ void g3_issue_act_f32(__amdgpu_buffer_rsrc_t frs, uint8_t *abuf, int lane, int wb0, int nb,
                                                 int M, int64_t lda) {
    const uint32_t base = (uint32_t)wb0 * 128u, limit = (uint32_t)nb * 128u;
    const uint32_t rowb = (uint32_t)lda * 4u;
    for (int t = 0; t < M; ++t) {
        const uint32_t inrow = base + (uint32_t)(lane ^ t) * 16u;
        dma_buf_lds16(frs, abuf + 1024 * t, inrow < limit ? (uint32_t)t * rowb + inrow : 0xFFFFFFF0u);
    }
    for (int pr = 0; 2 * pr < M; ++pr) {
        const int t = 2 * pr + (lane >> 5);
        const uint32_t inrow = base + (64u + (uint32_t)((lane & 31) ^ t)) * 16u;
        dma_buf_lds16(frs, abuf + 8192 + 1024 * pr, (t < M && inrow < limit) ? (uint32_t)t * rowb + inrow : 0xFFFFFFF0u);
    }
}
static_assert(8 * 1024 + 4 * 1024 <= kG3ALds, "eight fp32 slot slices");

// Chunk c (of 96) of slot t's slice, as g3_issue_act_f32 placed it.
__device__ __forceinline__ floatx4 g3_act_f32(const uint8_t *abuf, int t, int c) {
    const int off = c < 64 ? 1024 * t + 16 * (c ^ t) : 8192 + 1024 * (t >> 1) + 512 * (t & 1) + 16 * ((c - 64) ^ t);
    return *reinterpret_cast<const floatx4 *>(abuf + off);
}

template <int S, bool PACKED>
// qr: the row groups over the work-groups as wg_row_groups splits them,
// quotient | remainder << 4, from the host (no division in the kernel).
__global__ __launch_bounds__(kGvWaves * 64) void b1_gemv3_kernel(LinearArgs p, int qr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, g = lane >> 4;
    const int bid = blockIdx.x;
    const int q = qr & 15, r = qr >> 4;
    const int rg0 = bid * q + min(bid, r);
    const int nrg = q + (bid < r ? 1 : 0);
    const int nb = p.K / 32;
    const uint32_t rs = (uint32_t)nb * 6;
    uint8_t *wbuf = gsm + wave * kG3WaveLds;
    uint8_t *abuf = wbuf + kG3WLds;
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.w), (short)0, (int)(p.N * rs), kBufferFlags);
    // this wave's slice: bytes [72 w, 72 w + 72) of a pass's row part,
    // fetched from the aligned 72 w - 8 (w odd) as kG3RowCh chunks
    const uint32_t slice0 = (uint32_t)(72 * wave) & ~15u;
    const SliceDmas wd(lane, rg0 * 16, rs, slice0);

    floatx4 acc[kGvMaxRG];
#pragma unroll
    for (int r = 0; r < kGvMaxRG; ++r) acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
    float amax = 0.0f; // fp32: the largest magnitude this lane converted

    for (int kb0 = 0; kb0 < nb; kb0 += kG3Chunk) {
        const int wb0 = kb0 + wave * kGvBPW;
        // 1. activations
        constexpr bool F32LDS = !PACKED && S <= 8;
        static_assert((S & (S - 1)) == 0, "token slots a power of two");
        floatx4 xa[PACKED || F32LDS ? 1 : kGvBPW][2];
        if constexpr (PACKED) {
            const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(p.act), (short)0, (int)((uint32_t)p.M * (uint32_t)p.K * 2u), kBufferFlags);
            g3_issue_act<S>(ars, abuf, lane, wb0, nb, p.M, p.K);
        } else if constexpr (F32LDS) {
            const __amdgpu_buffer_rsrc_t frs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(p.act), (short)0,
                (int)(((uint32_t)(p.M - 1) * (uint32_t)p.lda + (uint32_t)p.K) * 4u), kBufferFlags);
            g3_issue_act_f32(frs, abuf, lane, wb0, nb, p.M, p.lda);
        } else {
            // lane (g, col): elements 32 blk + 4 t .. +3 and 16 later of token
            // col, blk = wb0 + 4 q + g, for fragment (q, t)
#pragma unroll
            for (int f = 0; f < kGvBPW; ++f) {
                const int blk = wb0 + 4 * (f >> 2) + g;
                if (col < p.M && blk < nb) {
                    const float *src = p.act + (size_t)col * p.lda + (size_t)blk * 32 + 4 * (f & 3);
                    xa[f][0] = *reinterpret_cast<const floatx4 *>(src);
                    xa[f][1] = *reinterpret_cast<const floatx4 *>(src + 16);
                } else {
                    xa[f][0] = xa[f][1] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        // 2. this wave's slice of every row of the work-group's row groups
#pragma unroll
        for (int i = 0; i < kG3WInst; ++i) dma_buf_lds16(wrs, wbuf + i * 1024, wd.off(i, nrg * 16, rs, (uint32_t)kb0 * 6u));
        // 3. the activations (issued first) have landed when at most the
        //    weight DMAs are outstanding
        wait_vmcnt<kG3WInst>();
        u32x4 af[kGvQuads][4];
        if constexpr (PACKED) {
            g3_read_act<S>(abuf, lane, af);
        } else if constexpr (F32LDS) {
            // lane (g, col), fragment (q, t): chunks 8 blk + t and + 4 of its
            // slot's slice, blk = 4 q + g (elements 32 blk + 4 t .. +3 and 16
            // later).  Chunks past K hold the DMA's zeros.  Every lane reads:
            // one whose column is a slot past M, or past S (it reads slot
            // col mod S), gets another token's or stale values, which reach
            // only output columns that are never stored (MFMA columns are
            // independent), and its range flag is masked below.
#pragma unroll
            for (int f = 0; f < kGvBPW; ++f) {
                const int bl = 4 * (f >> 2) + g, c = 8 * bl + (f & 3);
                const floatx4 x0 = g3_act_f32(abuf, col & (S - 1), c);
                const floatx4 x1 = g3_act_f32(abuf, col & (S - 1), c + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    amax = absmax3(amax, x0[j], x1[j]);
                    af[f >> 2][f & 3][j] = pack_f16(x0[j], x1[j]);
                }
            }
        } else {
#pragma unroll
            for (int f = 0; f < kGvBPW; ++f)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    amax = absmax3(amax, xa[f][0][j], xa[f][1][j]);
                    af[f >> 2][f & 3][j] = pack_f16(xa[f][0][j], xa[f][1][j]);
                }
        }
        // 4. row group by row group, as this wave's own DMAs land
        g3_decode<0>(wbuf, nrg, wave, lane, af, acc);
        wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): LDS reads done before the next pass's DMAs
    }

    // cross-wave reduction in a fixed order; the fp32 kernel's flags of
    // tokens with an activation beyond the fp16 range (a word per wave) go
    // with the partials, after them
    __syncthreads();
    floatx4 *red = reinterpret_cast<floatx4 *>(gsm); // [wave][rg][lane]
#pragma unroll
    for (int r = 0; r < kGvMaxRG; ++r)
        if (r < nrg) red[(wave * kGvMaxRG + r) * 64 + lane] = acc[r];
    uint32_t *flags = reinterpret_cast<uint32_t *>(gsm + kGvWaves * kGvMaxRG * 64 * 16);
    if constexpr (!PACKED) {
        const uint64_t bal = __builtin_amdgcn_ballot_w64(amax >= kF16Overflow);
        const uint32_t toks = (uint32_t)((bal | (bal >> 16) | (bal >> 32) | (bal >> 48)) & 0xFFFFu) &
                              (p.M >= 16 ? 0xFFFFu : (1u << p.M) - 1u);
        if (lane == 0) flags[wave] = toks;
    }
    __syncthreads();
    int bad = g3_reduce_store<S>(gsm, kGvMaxRG * 64 * 16, nrg, tid, p.M, p.N, rg0 * 16, p.out, p.ldo,
                              PACKED ? p.rsc : nullptr);
    if constexpr (!PACKED) {
        // this work-group's rows of the flagged tokens again, after every
        // thread's stores above (a barrier only on this rare path; `all` is
        // the same in every thread)
        uint32_t all = 0;
#pragma unroll
        for (int w = 0; w < kGvWaves; ++w) all |= flags[w];
        if (all) {
            __syncthreads();
            {
#pragma clang fp contract(off)
                for (int e = tid; e < 16 * nrg * 16; e += kGvWaves * 64) {
                    const int tok = e / (nrg * 16), rr = e - tok * (nrg * 16);
                    const int n = rg0 * 16 + rr;
                    if (tok >= p.M || n >= p.N || !((all >> tok) & 1u)) continue;
                    const float *xr = p.act + (size_t)tok * p.lda;
                    const uint16_t *wr = reinterpret_cast<const uint16_t *>(p.w + (size_t)n * rs);
                    float sum = 0.0f;
                    for (int b = 0; b < nb; ++b) {
                        const float scale = (float)__builtin_bit_cast(_Float16, wr[3 * b]);
                        const uint32_t bits = (uint32_t)wr[3 * b + 1] | ((uint32_t)wr[3 * b + 2] << 16);
                        float bs = 0.0f;
                        for (int i = 0; i < 32; ++i) {
                            const float a = xr[32 * b + i];
                            bs = ((bits >> i) & 1u) ? bs + a : bs - a;
                        }
                        sum = sum + scale * bs;
                    }
                    float *o = p.out + (size_t)tok * p.ldo + n;
                    bad += !__builtin_isfinite(sum) - !__builtin_isfinite(*o);
                    *o = sum;
                }
            }
        }
    }
    count_nonfinite(p.nonfinite, bad);
}

// Several small-M linears over one activation matrix in one launch (the
// modulation projections of a step, q/k/v of the text stream at a few
// tokens): packed fp16, or at most 8 tokens of fp32 rows (F32: converted by
// each wave as it stages them, tokens beyond the fp16 range recomputed in
// EXACT arithmetic).  Each op has its own work-groups (wgstart), each
// taking at most G4Cfg::P consecutive row groups of that op in one pass:
// every wave stages its activation slice and then DMAs its K slice of those
// rows into its own LDS area, keeping kG4Ahead row groups in flight behind
// the one it decodes, with no work-group barrier until the end, where the
// waves' partial tiles are summed once, in wave order.  The per-wave K
// slices, MFMA order and reduction order are those of b1_gemv3_kernel, so
// each op's outputs equal its own small-M call bit for bit.
struct GemvGroup {
    const uint8_t *w[kGemvGroupMax];
    float *out[kGemvGroupMax];
    int64_t ldo[kGemvGroupMax];
    int N[kGemvGroupMax];           // 0 for the entries past the ops
    int wgstart[kGemvGroupMax + 1]; // first work-group of each op; wgstart[nops..] = the grid
    int rgqr[kGemvGroupMax];        // an op's row groups over its work-groups: q | r << 4
    int K, M;
    const void *act;  // packed fp16 [M][K], or fp32 [M][lda] (the F32 kernels)
    int64_t lda;      // fp32 row stride (elements)
    const float *rsc; // row scales of the packing, or nullptr
    int32_t *nonfinite;
};

// The first 8 entries of a kernel-argument array held in SGPRs: each is
// read once with a constant index and passed through an empty asm, so that
// a choice among them by a wave-uniform condition stays scalar selects and
// the entries arrive in one round of scalar loads.  (Without the asm the
// compiler folds the selects back into an indexed read of argument memory,
// a dependent scalar load of about 1 us; with an array member instead of
// named ones it moves the entries to scratch.)
template <class T>
__device__ __forceinline__ T sgpr_opaque(T x) {
    asm volatile("" : "+s"(x));
    return x;
}
template <class T>
struct Sgpr8 {
    T a0, a1, a2, a3, a4, a5, a6, a7;
    template <class U, int N>
    __device__ __forceinline__ explicit Sgpr8(const U (&a)[N])
        : a0(sgpr_opaque((T)a[0])), a1(sgpr_opaque((T)a[1])), a2(sgpr_opaque((T)a[2])), a3(sgpr_opaque((T)a[3])),
          a4(sgpr_opaque((T)a[4])), a5(sgpr_opaque((T)a[5])), a6(sgpr_opaque((T)a[6])), a7(sgpr_opaque((T)a[7])) {
        static_assert(N >= 8, "eight entries");
    }
};

// Row groups whose DMAs are in flight behind the one being decoded.  With
// two work-groups per CU (16 waves), 2 measured best for the modulation
// projections: 13.9 us per launch against 14.2-14.5 us with 1 and 14.4-14.6
// us with 4 (a timing copy, two alternating passes).  With one work-group
// per CU (8 tokens) 2 is best too: the four projections at M = 8 took
// 18.6 us against 20.3-20.4 us with 4 or 8.
constexpr int kG4Ahead = 2;

// Row groups of a one-pass work-group by token slots S and per-wave LDS
// bytes WL: the activation slice (ABytes) and the weight slices of P row
// groups (WInst DMAs of 1 KB) fill a wave's WL bytes.  WL = 10 KB (S <= 4)
// puts two work-groups on a CU, so that one's reduction and tail overlap the
// other's decode; S = 8 and 16 need the whole 20 KB.
constexpr int g4_abytes(int S) { return S <= 8 ? (S - 1) * kG3ARow + 1024 : kGvBPW * 1024; }
constexpr int g4_rows(int abytes, int wl) {
    int p = 0;
    while (abytes + ((16 * kG3RowCh * (p + 1) + 63) / 64) * 1024 <= wl) ++p;
    return p;
}
template <int S, int WL, bool F32 = false>
struct G4Cfg {
    static constexpr int ABytes = g4_abytes(S);
    static constexpr int P = g4_rows(ABytes, WL);
    static constexpr int WInst = (P * 16 * kG3RowCh + 63) / 64;
    static constexpr int Lds = kGvWaves * WL;
    static_assert(P >= 1 && ABytes % 16 == 0 && ABytes + WInst * 1024 <= WL, "a wave's LDS area");
    static_assert(P < 16, "row groups per work-group in 4 bits (GemvGroup::rgqr)");
    static_assert(P * 1024 <= WL, "the reduction fits");
    static_assert(WInst + 2 * kGemvGroupMax < 64, "vmcnt range");
    static_assert(P * 1024 * kGvWaves + kGvWaves * 4 <= kGvWaves * WL, "the reduction and its flags fit");
};
constexpr int kG4WL2 = 10 * 1024; // two work-groups per CU
constexpr int kG4WL1 = kG3WaveLds; // one

// Weight DMAs of a one-pass work-group that cover its row groups 0..r
// (a row group's 16 rows x 5 chunks are 1.25 DMAs of 64 lanes).
constexpr int g4_dmas(int r) { return (16 * kG3RowCh * (r + 1) + 63) / 64; }

// Row groups R.. of the pass: issue the DMAs of row group R + D (keeping
// D row groups in flight behind the one being decoded), wait for row group
// R's (DMAs retire in issue order: at most the hi - g4_dmas(R) issued after
// them may be outstanding), decode it, go on while R + 1 < nrg.
template <int R, int P, int WI, int D>
struct G4Decode {
    template <class Issue>
    static __device__ __forceinline__ void run(const uint8_t *wbuf, int nrg, int wave, int lane,
                                               const u32x4 (&af)[kGvQuads][4], floatx4 (&acc)[P], Issue &issue) {
        if (R < nrg) {
            constexpr int lo = g4_dmas(R + D - 1) < WI ? g4_dmas(R + D - 1) : WI;
            constexpr int hi = g4_dmas(R + D) < WI ? g4_dmas(R + D) : WI;
#pragma unroll
            for (int i = lo; i < hi; ++i) issue(i);
            wait_vmcnt<hi - g4_dmas(R)>();
            g3_decode_rg<true>(wbuf, R, wave, lane, af, acc[R]);
            G4Decode<R + 1, P, WI, D>::run(wbuf, nrg, wave, lane, af, acc, issue);
        }
    }
};
template <int P, int WI, int D>
struct G4Decode<P, P, WI, D> {
    template <class Issue>
    static __device__ __forceinline__ void run(const uint8_t *, int, int, int, const u32x4 (&)[kGvQuads][4],
                                               floatx4 (&)[P], Issue &) {}
};

// fp32 activations of the grouped kernel, S <= 8 token slots, through
// registers into the packed layout g3_read_act<S> reads: token t at abuf +
// kG3ARow t, block b's 16 dwords at 64 b, dword d the fp16 pair (element d,
// element d + 16), rounded as the single call rounds.  Job j = (t, b, q) of
// the S * 48 loads elements 32 b + 4 q .. + 3 and 16 later of token t's
// slice (the wave's 12 blocks from block wb0) and stores them packed at
// kG3ARow t + 64 b + 16 q.  Blocks past K and tokens past M read zeros.
// (Staging the fp32 slice in LDS instead takes a second KB of the wave's
// area, a row group fewer per work-group and, for a step's modulation
// projections, more work-groups than two a CU hold.)
template <int S>
struct G4ActF32 {
    static_assert(S <= 8, "at most 8 token slots");
    static constexpr int J = S * 48, R = (J + 63) / 64;
    floatx4 x[R][2];
    // frs: the rows, (M - 1) lda + K floats; rowb = lda * 4
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t frs, int lane, int wb0, int nb, int M,
                                         uint32_t rowb) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int j = r * 64 + lane, t = j / 48, bq = j - 48 * t, b = bq >> 2;
            const uint32_t off = (uint32_t)t * rowb + (uint32_t)(wb0 + b) * 128u + (uint32_t)(bq & 3) * 16u;
            const bool ok = j < J && t < M && wb0 + b < nb;
            x[r][0] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(frs, ok ? off : 0xFFFFFFF0u, 0, 0));
            x[r][1] = __builtin_bit_cast(floatx4,
                                         __builtin_amdgcn_raw_buffer_load_b128(frs, ok ? off + 64u : 0xFFFFFFF0u, 0, 0));
        }
    }
    // Returns the tokens (bit t) this lane found an element beyond the fp16
    // range in.
    __device__ __forceinline__ uint32_t store(uint8_t *abuf, int lane) const {
        uint32_t ovf = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int j = r * 64 + lane, t = j / 48, bq = j - 48 * t;
            if (j < J) {
                u32x4 v;
                float amax = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    amax = absmax3(amax, x[r][0][e], x[r][1][e]);
                    v[e] = pack_f16(x[r][0][e], x[r][1][e]);
                }
                ovf |= (uint32_t)(amax >= kF16Overflow) << t;
                *reinterpret_cast<u32x4 *>(abuf + t * kG3ARow + 64 * (bq >> 2) + 16 * (bq & 3)) = v;
            }
        }
        return ovf;
    }
};

// (__launch_bounds__' second argument is the minimum of waves per SIMD: two
// work-groups of 8 waves on a CU need 4, so at most 128 registers a wave.)
template <int S, int WL, bool F32>
__global__ __launch_bounds__(kGvWaves * 64, WL == kG4WL2 ? 4 : 2) void b1_gemv_group_kernel(GemvGroup p) {
    using C = G4Cfg<S, WL, F32>;
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = sgpr_opaque(p.K), M = sgpr_opaque(p.M);
    const void *const act = reinterpret_cast<const void *>(sgpr_opaque((uint64_t)p.act));
    const float *const rsc = reinterpret_cast<const float *>(sgpr_opaque((uint64_t)p.rsc));
    const int nb = K / 32;
    const uint32_t rs = (uint32_t)nb * 6;
    uint8_t *abuf = gsm + wave * WL;
    uint8_t *wbuf = abuf + C::ABytes;
    const uint32_t slice0 = (uint32_t)(72 * wave) & ~15u;
    // the per-op arguments, all read at the start (one round of scalar
    // loads); this work-group's op and its row groups [R0, R0 + nrg)
    static_assert(kGemvGroupMax == 8, "eight ops");
    const Sgpr8<int> wgs(p.wgstart);
    const Sgpr8<int> ns(p.N);
    const Sgpr8<uint64_t> ws(p.w);
    const Sgpr8<int> qrs(p.rgqr);
    const int bid = blockIdx.x;
    // the op is the last whose first work-group is at or before bid: a scan
    // of scalar compares and selects (indexing the entries by a computed op
    // made a tree of branches, ~270 scalar instructions before the first
    // DMA, in every wave)
    const int wgv[kGemvGroupMax] = {wgs.a0, wgs.a1, wgs.a2, wgs.a3, wgs.a4, wgs.a5, wgs.a6, wgs.a7};
    const int nv[kGemvGroupMax] = {ns.a0, ns.a1, ns.a2, ns.a3, ns.a4, ns.a5, ns.a6, ns.a7};
    const uint64_t wv[kGemvGroupMax] = {ws.a0, ws.a1, ws.a2, ws.a3, ws.a4, ws.a5, ws.a6, ws.a7};
    const int qrv[kGemvGroupMax] = {qrs.a0, qrs.a1, qrs.a2, qrs.a3, qrs.a4, qrs.a5, qrs.a6, qrs.a7};
    int op = 0, wg0 = wgv[0], N = nv[0], qr = qrv[0];
    uint64_t wq = wv[0];
#pragma unroll
    for (int k = 1; k < kGemvGroupMax; ++k) {
        const bool c = bid >= wgv[k];
        op = c ? k : op;
        wg0 = c ? wgv[k] : wg0;
        N = c ? nv[k] : N;
        wq = c ? wv[k] : wq;
        qr = c ? qrv[k] : qr;
    }
    uint8_t *const wp = reinterpret_cast<uint8_t *>(wq);
    // the op's row groups split as wg_row_groups would, from the host's
    // quotient and remainder (no division here)
    const int q = qr & 15, r = qr >> 4, local = bid - wg0;
    const int R0 = local * q + min(local, r);
    const int nrg = q + (local < r ? 1 : 0); // at most C::P (the launcher's grid)
    // 1. the activation slice, then the weight slices, D row groups ahead
    G4ActF32<F32 ? S : 1> xf; // fp32: this lane's activation chunks
    if constexpr (F32) {
        const uint32_t rowb = (uint32_t)sgpr_opaque(p.lda) * 4u;
        const __amdgpu_buffer_rsrc_t frs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void *>(act), (short)0, (int)((uint32_t)(M - 1) * rowb + (uint32_t)K * 4u), kBufferFlags);
        xf.load(frs, lane, wave * kGvBPW, nb, M, rowb);
    } else {
        const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void *>(act), (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), kBufferFlags);
        g3_issue_act<S>(ars, abuf, lane, wave * kGvBPW, nb, M, K);
    }
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(wp, (short)0, (int)((uint32_t)N * rs), kBufferFlags);
    const SliceDmas wd(lane, R0 * 16, rs, slice0);
    const int lim = min(nrg * 16, N - R0 * 16); // rows of the work-group's row groups that exist
    auto issue = [&](int i) { dma_buf_lds16(wrs, wbuf + i * 1024, wd.off(i, lim, rs, 0u)); };
    constexpr int D = kG4Ahead;
    constexpr int first = g4_dmas(D - 1) < C::WInst ? g4_dmas(D - 1) : C::WInst;
#pragma unroll
    for (int i = 0; i < first; ++i) issue(i);
    // the outputs' arguments only now, so that their scalar loads do not
    // hold back the first DMAs
    const Sgpr8<uint64_t> outs(p.out);
    const Sgpr8<int64_t> ldos(p.ldo);
    // 2. the activations (issued first) have landed when at most the weight
    //    DMAs are outstanding; the fp32 ones go to LDS packed (read back
    //    by this wave only: its LDS operations complete in order)
    wait_vmcnt<first>();
    u32x4 af[kGvQuads][4];
    uint32_t ovf = 0; // fp32: tokens (bit t) this lane found beyond the fp16 range
    if constexpr (F32) ovf = xf.store(abuf, lane);
    g3_read_act<S>(abuf, lane, af);
    // 3. row group by row group, as this wave's own DMAs land
    floatx4 acc[C::P]; // each set by its row group's decode; [nrg, P) never read
    G4Decode<0, C::P, C::WInst, D>::run(wbuf, nrg, wave, lane, af, acc, issue);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0)

    // 4. cross-wave reduction in wave order; the fp32 kernel's out-of-range
    //    token flags (a word per wave) go with the partials
    __syncthreads();
    floatx4 *red = reinterpret_cast<floatx4 *>(gsm); // [wave][P][lane]
#pragma unroll
    for (int r = 0; r < C::P; ++r)
        if (r < nrg) red[(wave * C::P + r) * 64 + lane] = acc[r];
    uint32_t *flags = reinterpret_cast<uint32_t *>(gsm + kGvWaves * C::P * 1024);
    if constexpr (F32) {
        uint32_t toks = 0;
#pragma unroll
        for (int t = 0; t < S; ++t)
            if (__builtin_amdgcn_ballot_w64(((ovf >> t) & 1u) != 0)) toks |= 1u << t;
        if (lane == 0) flags[wave] = toks;
    }
    __syncthreads();
    const uint64_t ov[kGemvGroupMax] = {outs.a0, outs.a1, outs.a2, outs.a3, outs.a4, outs.a5, outs.a6, outs.a7};
    const int64_t lv[kGemvGroupMax] = {ldos.a0, ldos.a1, ldos.a2, ldos.a3, ldos.a4, ldos.a5, ldos.a6, ldos.a7};
    uint64_t oq = ov[0];
    int64_t ldo = lv[0];
#pragma unroll
    for (int k = 1; k < kGemvGroupMax; ++k) {
        oq = k <= op ? ov[k] : oq;
        ldo = k <= op ? lv[k] : ldo;
    }
    float *const out = reinterpret_cast<float *>(oq);
    // the (row, token slot) elements of all nrg row groups spread over the
    // work-group's threads (one pass at S <= 4); each element summed over
    // the waves in wave order
    int bad = 0;
    constexpr int SE = 16 * S; // elements of a row group, a power of two
    for (int idx = tid; idx < nrg * SE; idx += kGvWaves * 64) {
        const int r = idx / SE, tok = (idx % SE) >> 4, c = idx & 15;
        const int ln = 16 * (tok >> 2) + c, v = tok & 3;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < kGvWaves; ++w) sum += red[(w * C::P + r) * 64 + ln][v];
        const int n = (R0 + r) * 16 + c;
        if (tok < M && n < N) {
            if (rsc) sum *= rsc[tok];
            bad += !__builtin_isfinite(sum);
            out[(size_t)tok * ldo + n] = sum;
        }
    }
    if constexpr (F32) {
        // this work-group's rows of the flagged tokens again in the
        // reference's scalar arithmetic (the single call's EXACT rows),
        // after every thread's stores above (a barrier only on this rare
        // path; `all` is the same in every thread)
        uint32_t all = 0;
#pragma unroll
        for (int w = 0; w < kGvWaves; ++w) all |= flags[w];
        if (all) {
            __syncthreads();
            const float *xa = static_cast<const float *>(act);
            const int64_t lda = p.lda;
            {
#pragma clang fp contract(off)
                for (int e2 = tid; e2 < S * nrg * 16; e2 += kGvWaves * 64) {
                    const int t2 = e2 / (nrg * 16), rr = e2 - t2 * (nrg * 16);
                    const int n = R0 * 16 + rr;
                    if (t2 >= M || n >= N || !((all >> t2) & 1u)) continue;
                    const float *xr = xa + (size_t)t2 * lda;
                    const uint16_t *wr = reinterpret_cast<const uint16_t *>(wp + (size_t)n * rs);
                    float sum = 0.0f;
                    for (int b = 0; b < nb; ++b) {
                        const float scale = (float)__builtin_bit_cast(_Float16, wr[3 * b]);
                        const uint32_t bits = (uint32_t)wr[3 * b + 1] | ((uint32_t)wr[3 * b + 2] << 16);
                        float bs = 0.0f;
                        for (int i = 0; i < 32; ++i) {
                            const float a = xr[32 * b + i];
                            bs = ((bits >> i) & 1u) ? bs + a : bs - a;
                        }
                        sum = sum + scale * bs;
                    }
                    float *o = out + (size_t)t2 * ldo + n;
                    bad += !__builtin_isfinite(sum) - !__builtin_isfinite(*o);
                    *o = sum;
                }
            }
        }
    }
    count_nonfinite(p.nonfinite, bad);
}

} // namespace

// ------------------------------------------------------------- launchers --

hipError_t launch_exact(const LinearArgs &a, int num_cus, hipStream_t s) {
    // rows a work-group shares its signs over: 16 or 8 while that leaves
    // at least 4 work-groups (16 waves) a CU, else 4 (a small grid needs
    // the work-groups more than the shared signs)
    const int64_t cols = (a.N + kExTN - 1) / kExTN;
    const int64_t want = 4 * (int64_t)(num_cus > 0 ? num_cus : 256);
    auto go = [&](auto kernel, int tm) {
        const dim3 grid((unsigned)cols, (unsigned)((a.M + tm - 1) / tm));
        hipLaunchKernelGGL(kernel, grid, dim3(kExTN), 0, s, a);
    };
    if (a.M > 8 && cols * ((a.M + 15) / 16) >= want)
        go(b1_exact_kernel<16>, 16);
    else if (a.M > 4 && cols * ((a.M + 7) / 8) >= want)
        go(b1_exact_kernel<8>, 8);
    else
        go(b1_exact_kernel<4>, 4);
    return hipGetLastError();
}

static bool fast_layout_ok(const LinearArgs &a) {
    return a.K % 64 == 0 && a.lda % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(a.act) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(a.w) & 3u) == 0;
}

bool gemm_supported(const LinearArgs &a) { return fast_layout_ok(a); }

namespace {
// The packed GEMM configuration: 128 x 512 tiles of 8 waves, three-slot ring,
// one work-group per CU.
constexpr int kBM = 128, kBN = 512, kWN = 64, kStages = 3, kWgPerCu = 1;
using KCfg = GemmLdsCfg<kBM, kBN, kWN, kStages>;
// Half-height tiles for the last, partial round of some shapes.
constexpr int kBMH = 64;
using KCfgH = GemmLdsCfg<kBMH, kBN, kWN, kStages>;
} // namespace

// GEMM over pre-packed activations: the stage count K/128 is a multiple of
// the ring's slot count, and byte offsets into the packed activations and
// the weights fit the kernel's 32-bit offsets.
bool gemm_packed_ok(int M, int K, int N) {
    const uint64_t act_bytes = (uint64_t)M * (uint64_t)K * 2;
    const uint64_t w_bytes = (uint64_t)N * (uint64_t)(K / 32) * 6;
    return M > 0 && K > 0 && N > 0 && K % (KCfg::KC * kStages) == 0 && act_bytes < (1ull << 32) &&
           w_bytes < (1ull << 32);
}

static size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t pack_area_bytes(int M, int K) { return round256((size_t)M * K * 2) + round256((size_t)M * 4); }

size_t gemm_workspace_bytes(const LinearArgs &a) {
    return gemm_packed_ok(a.M, a.K, a.N) && fast_layout_ok(a) ? pack_area_bytes(a.M, a.K) : 0;
}

float *pack_area_rsc(void *area, int M, int K) {
    return reinterpret_cast<float *>(static_cast<uint8_t *>(area) + round256((size_t)M * K * 2));
}

hipError_t launch_pack_rows(const float *act, int64_t lda, int M, int K, void *area, hipStream_t s) {
    return launch_pack_rows_to(act, lda, M, K, area, pack_area_rsc(area, M, K), s);
}

hipError_t launch_pack_rows_to(const float *act, int64_t lda, int M, int K, void *packed, float *rsc,
                               hipStream_t s) {
    const int units = K / 8;
    int wl = 0, per = 0;
    for (wl = 0; wl <= 2; ++wl) {
        per = (units + (64 << wl) - 1) / (64 << wl);
        if (per <= 8) break;
    }
    if (wl > 2) {
        wl = 2;
        per = 0; // read twice
    }
    const int rows_per_wg = 4 >> wl;
    const dim3 grid((M + rows_per_wg - 1) / rows_per_wg);
    const bool nt = (uint64_t)M * (uint64_t)K * 4 > kNtInputBytes;
    uint32_t *pk = static_cast<uint32_t *>(packed);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, act, lda, pk, (int64_t)K / 2, rsc, M, K, wl);
    };
#define B1_PACK_ROWS(U)                                                                                         \
    (nt ? go(b1_pack_rows_kernel<U, true>) : go(b1_pack_rows_kernel<U, false>))
    if (per == 0) B1_PACK_ROWS(0);
    else if (per <= 1) B1_PACK_ROWS(1);
    else if (per <= 2) B1_PACK_ROWS(2);
    else if (per <= 4) B1_PACK_ROWS(4);
    else if (per <= 6) B1_PACK_ROWS(6);
    else B1_PACK_ROWS(8);
#undef B1_PACK_ROWS
    return hipGetLastError();
}

hipError_t launch_fixup_rows(const LinearArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(b1_fixup_rows_kernel, dim3(a.M), dim3(256), 0, s, a);
    return hipGetLastError();
}

bool pack_supported(const float *act, int64_t lda, int M, int K) {
    return K % 32 == 0 && lda >= K && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(act) & 15u) == 0 &&
           (uint64_t)M * (uint64_t)(K / 32) * 4 < (1ull << 31);
}

hipError_t launch_pack(const float *act, int64_t lda, int M, int K, void *packed, int64_t ldp, hipStream_t s) {
    const int units = M * (K / 32) * 4;
    const int pgrid = (units + 255) / 256 < 65535 ? (units + 255) / 256 : 65535;
    const bool nt = (uint64_t)M * (uint64_t)K * 4 > kNtInputBytes;
    hipLaunchKernelGGL(nt ? b1_pack_act_kernel<true> : b1_pack_act_kernel<false>, dim3(pgrid), dim3(256), 0, s, act,
                       lda, static_cast<uint32_t *>(packed), ldp / 2, M, K);
    return hipGetLastError();
}

// Split-K: how many K ranges to split a plain GEMM into, 1 for none.  A
// split pays only when the 128 x 512 tiles leave most CUs idle (fewer than
// half busy): it multiplies the work units by S, then a separate pass sums
// S fp32 partial products.  Model, in microseconds: a 384-K unit of a tile
// takes ~10.9; the partials cost their write and read at ~5 TB/s plus ~3
// for the extra launch.  S divides K / 384, at most 16.
int gemm_splits(int M, int K, int N, int num_cus) {
    if (num_cus <= 0 || !gemm_packed_ok(M, K, N) || N % 4) return 1;
    const int tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    const int slots = num_cus * kWgPerCu;
    if (2 * tiles > slots) return 1;
    const int units = K / (KCfg::KC * kStages);
    int best = 1;
    double best_us = 0;
    for (int sp = 1; sp <= 16 && sp <= units; ++sp) {
        if (units % sp) continue;
        const double rounds = (double)((tiles * sp + slots - 1) / slots);
        double us = rounds * (units / sp) * 10.9;
        if (sp > 1) us += 2.0 * sp * (double)M * N * 4 / 5e6 + 3.0;
        if (sp == 1 || us < best_us) {
            best = sp;
            best_us = us;
        }
    }
    return best;
}

size_t gemm_split_bytes(int M, int N, int splits) {
    return splits > 1 ? (size_t)splits * (size_t)M * (size_t)((N + 3) & ~3) * sizeof(float) : 0;
}

// Rounds of the 128 x 512 kernel's persistent grid, in units of one round
// of full tiles: ceil(tiles / slots), or, where launch_gemm_packed_t runs
// the last partial round as 64-row tiles, the full rounds plus ~0.6.
static double gemm_rounds128(int M, int N, int num_cus) {
    const int tiles_n = (N + kBN - 1) / kBN, tiles = ((M + kBM - 1) / kBM) * tiles_n;
    const int slots = num_cus * kWgPerCu;
    const int full = tiles / slots * slots, head_rows = full / tiles_n;
    const int tail_tiles = ((M - head_rows * kBM + kBMH - 1) / kBMH) * tiles_n;
    if (full > 0 && full < tiles && tiles_n < slots && head_rows > 0 && tail_tiles <= slots)
        return full / slots + 0.6;
    return (double)((tiles + slots - 1) / slots);
}

int gemm_tiles(int M, int K, int N, int num_cus) {
    if (num_cus <= 0 || !gemm_packed_ok(M, K, N) || K % (Gemm16Cfg<128, 384>::KC * Gemm16Cfg<128, 384>::STAGES))
        return 0;
    if (gemm_splits(M, K, N, num_cus) > 1) return 0;
    // rounds of the persistent grid in units of a 128 x 512 round (a BM x BN
    // tile counts BM BN / 65536 of one); strictly fewer to leave the
    // 128 x 512 kernel
    double best = gemm_rounds128(M, N, num_cus);
    int kind = 0;
    auto consider = [&](int id, int bm, int bn) {
        if (M % bm || N % bn) return;
        const int tiles = (M / bm) * (N / bn);
        const double r = (double)((tiles + num_cus - 1) / num_cus) * (double)(bm * bn) / (double)(kBM * kBN);
        if (r < best) {
            best = r;
            kind = id;
        }
    };
    consider(1, 144, 384);
    consider(2, 128, 384);
    return kind;
}

template <int BM, int BN, int EPI>
static hipError_t launch_gemm16_t(const void *packed, const uint8_t *w, int K, int N, int M, float *out, int64_t ldo,
                                  int32_t *nonfinite, int num_cus, const GemmEpi &epi, hipStream_t s) {
    using C = Gemm16Cfg<BM, BN>;
    auto kernel = &b1_gemm16_kernel<BM, BN, EPI>;
    static std::once_flag attr_once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(attr_once, [kernel] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
    });
    if (attr_err != hipSuccess) return attr_err;
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    // 16-byte rows, and BM rows of a buffer resource under 2^31 bytes
    int vec_store = al16(out) && ldo % 4 == 0 && ldo < (int64_t(1) << 21);
    if (EPI == 1)
        vec_store = vec_store && al16(epi.res) && al16(epi.gate) && epi.ldr % 4 == 0 && epi.ldr < (int64_t(1) << 21);
    if (EPI == 3)
        vec_store = (epi.split == 0 || vec_store) && al16(epi.pk) && epi.ldpw % 4 == 0 &&
                    epi.ldpw < (int64_t(1) << 21);
    const int tiles_m = M / C::BM, tiles_n = N / C::BN, tiles = tiles_m * tiles_n;
    const int grid = tiles < num_cus ? tiles : num_cus; // persistent
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(C::NT), C::LDS, s, static_cast<const uint16_t *>(packed), w, K, N, M,
                       out, ldo, nonfinite, tiles_m, tiles_n, vec_store, epi);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_gemm_packed_t(const void *packed, const uint8_t *w, int K, int N, int M, float *out,
                                       int64_t ldo, int32_t *nonfinite, int num_cus, const GemmEpi &epi,
                                       hipStream_t s, int ksplit = 1, float *partials = nullptr) {
    // (with ksplit > 1 the row scales epi.rsc go to the reduction, not the
    // GEMM, which writes plain partial products)
    // (a packed SwiGLU output on 16x16 tiles needs the split point on a
    // tile boundary, every tile wholly fp32 or wholly SwiGLU pairs; otherwise
    // it runs the 128 x 512 kernel)
    {
        const bool tiles_ok = !(EPI == 3 && epi.act == 2 && epi.split % 384 != 0);
        if (!(ksplit > 1 && partials != nullptr) && tiles_ok) {
            const int t = gemm_tiles(M, K, N, num_cus);
            if (t == 1) return launch_gemm16_t<144, 384, EPI>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s);
            if (t == 2) return launch_gemm16_t<128, 384, EPI>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s);
        }
    }
    auto kernel = &b1_gemm_kernel<kBM, kBN, kWN, kStages, EPI>;
    static std::once_flag attr_once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(attr_once, [kernel] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, KCfg::LDS);
    });
    if (attr_err != hipSuccess) return attr_err;
    const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
    const bool split = EPI == 0 && ksplit > 1 && partials != nullptr;
    const int units = tiles_m * tiles_n * (split ? ksplit : 1);
    const int slots = num_cus > 0 ? num_cus * kWgPerCu : units;
    const int grid = units < slots ? units : slots; // persistent
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (split) {
        // the units' plain products into the partial slices, then their sum
        const int64_t ldp = (N + 3) & ~3;
        const int64_t pstride = (int64_t)M * ldp;
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(KCfg::NT), KCfg::LDS, s, static_cast<const uint16_t *>(packed),
                           w, K, N, M, partials, ldp, nullptr, tiles_m, tiles_n,
                           (int)(al16(partials) && ldp < (int64_t(1) << 22)), epi, ksplit, pstride);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t q = (int64_t)M * ((N + 3) / 4);
        const int64_t want = (q + 255) / 256, cap = (int64_t)(num_cus > 0 ? num_cus : 256) * 8;
        const int rgrid = (int)(want < cap ? want : cap);
        hipLaunchKernelGGL(b1_splitk_reduce_kernel, dim3(rgrid), dim3(256), 0, s, partials, ldp, pstride, ksplit, M,
                           N, out, ldo, nonfinite, (int)(al16(out) && ldo % 4 == 0), epi.rsc);
        return hipGetLastError();
    }
    int vec_store = al16(out) && ldo % 4 == 0 && ldo < (int64_t(1) << 22);
    if (EPI == 1)
        vec_store = vec_store && al16(epi.res) && al16(epi.gate) && epi.ldr % 4 == 0 && epi.ldr < (int64_t(1) << 22);
    if (EPI == 3)
        // each part the epilogue writes: 16-byte aligned rows (the caller
        // checks these) and 128 rows under 2^31 bytes for the buffer stores
        vec_store = (epi.split == 0 || (al16(out) && ldo % 4 == 0 && ldo < (int64_t(1) << 22))) &&
                    (epi.split >= N || (al16(epi.pk) && epi.ldpw % 4 == 0 && epi.ldpw < (int64_t(1) << 22)));
    // The persistent grid runs ceil(tiles / slots) rounds.  When the whole
    // tile rows that fit in the full rounds leave at most one round of
    // 64-row tiles, those rows run with 128-row tiles (still the same
    // number of rounds) and the rest as 64-row tiles in a second launch:
    // twice the tiles, each ~0.6 of a 128-row tile's time (at M=4608 K=3072
    // N=12288: 768 tiles in 3 rounds, then 192 half tiles instead of 96;
    // at M=4096 N=9216: 504 tiles in 2 rounds, then 144 half tiles instead
    // of a third round of 72).  Every output is the same sum in the same
    // order.
    const int tiles = tiles_m * tiles_n;
    const int full = num_cus > 0 ? tiles / slots * slots : 0;
    const int head_rows = full / tiles_n;                        // whole tile rows in the full rounds
    const int tail_tiles = ((M - head_rows * kBM + kBMH - 1) / kBMH) * tiles_n;
    if (full > 0 && full < tiles && tiles_n < slots && head_rows > 0 && tail_tiles <= slots) {
        auto tail = &b1_gemm_kernel<kBMH, kBN, kWN, kStages, EPI>;
        static std::once_flag tail_once;
        static hipError_t tail_err = hipSuccess;
        std::call_once(tail_once, [tail] {
            tail_err = hipFuncSetAttribute(reinterpret_cast<const void *>(tail),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, KCfgH::LDS);
        });
        if (tail_err != hipSuccess) return tail_err;
        const int ms = head_rows * kBM;
        const int hunits = head_rows * tiles_n;
        hipLaunchKernelGGL(kernel, dim3(hunits < slots ? hunits : slots), dim3(KCfg::NT), KCfg::LDS, s,
                           static_cast<const uint16_t *>(packed), w, K, N, ms, out, ldo, nonfinite, head_rows, tiles_n,
                           vec_store, epi, 1, (int64_t)0);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        GemmEpi et = epi;
        if (et.res) et.res += (size_t)ms * (size_t)et.ldr;
        if (et.pk) et.pk += (size_t)ms * (size_t)et.ldpw;
        if (et.rsc) et.rsc += ms;
        const int mt = M - ms, tm = (mt + kBMH - 1) / kBMH;
        hipLaunchKernelGGL(tail, dim3(tm * tiles_n), dim3(KCfgH::NT), KCfgH::LDS, s,
                           static_cast<const uint16_t *>(packed) + (size_t)ms * (size_t)K, w, K, N, mt,
                           out ? out + (size_t)ms * (size_t)ldo : out, ldo, nonfinite, tm, tiles_n, vec_store, et, 1,
                           (int64_t)0);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(KCfg::NT), KCfg::LDS, s, static_cast<const uint16_t *>(packed), w,
                       K, N, M, out, ldo, nonfinite, tiles_m, tiles_n, vec_store, epi, 1, (int64_t)0);
    return hipGetLastError();
}

hipError_t launch_gemm_packed(const void *packed, const uint8_t *w, int K, int N, int M, float *out, int64_t ldo,
                              int32_t *nonfinite, int num_cus, hipStream_t s) {
    return launch_gemm_packed_t<0>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, GemmEpi{}, s);
}

hipError_t launch_gemm_packed_split(const void *packed, const uint8_t *w, int K, int N, int M, float *out,
                                    int64_t ldo, int32_t *nonfinite, int num_cus, int splits, void *partials,
                                    hipStream_t s, const float *rsc) {
    GemmEpi epi;
    epi.rsc = rsc;
    return launch_gemm_packed_t<0>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s, splits,
                                   static_cast<float *>(partials));
}

hipError_t launch_gemm_packed_epi(const void *packed, const uint8_t *w, int K, int N, int M, float *out,
                                  int64_t ldo, int32_t *nonfinite, int num_cus, int kind, const GemmEpi &epi,
                                  hipStream_t s) {
    switch (kind) {
    case 0: return launch_gemm_packed_t<0>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s);
    case 1: return launch_gemm_packed_t<1>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s);
    case 2: return launch_gemm_packed_t<2>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s);
    case 3: return launch_gemm_packed_t<3>(packed, w, K, N, M, out, ldo, nonfinite, num_cus, epi, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(const LinearArgs &a, int num_cus, void *workspace, size_t ws_bytes, hipStream_t s) {
    const size_t need = gemm_workspace_bytes(a);
    if (need == 0 || workspace == nullptr || ws_bytes < need) {
        // Fused-conversion kernel: no workspace needed; rows its fp16
        // conversion overflows are then computed exactly.
        constexpr int BM = 128, BN = 512, WM = 128, WN = 64;
        using C = GemmCfg<BM, BN, WM, WN>;
        const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
        hipLaunchKernelGGL((b1_gemm_fused_kernel<BM, BN, WM, WN>), dim3(tiles_m * tiles_n), dim3(C::NT), 0, s, a,
                           tiles_n);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? launch_fixup_rows(a, s) : e;
    }
    hipError_t e = launch_pack_rows(a.act, a.lda, a.M, a.K, workspace, s);
    if (e != hipSuccess) return e;
    const float *rsc = pack_area_rsc(workspace, a.M, a.K);
    // the split-K partials after the packing, when the workspace holds them
    const int splits = gemm_splits(a.M, a.K, a.N, num_cus);
    if (splits > 1 && ws_bytes >= need + gemm_split_bytes(a.M, a.N, splits))
        return launch_gemm_packed_split(workspace, a.w, a.K, a.N, a.M, a.out, a.ldo, a.nonfinite, num_cus, splits,
                                        static_cast<uint8_t *>(workspace) + need, s, rsc);
    GemmEpi epi;
    epi.rsc = rsc;
    return launch_gemm_packed_epi(workspace, a.w, a.K, a.N, a.M, a.out, a.ldo, a.nonfinite, num_cus, 0, epi, s);
}

size_t gemm_workspace_bytes_total(const LinearArgs &a, int num_cus) {
    const size_t pack = gemm_workspace_bytes(a);
    if (pack == 0) return 0;
    const int splits = gemm_splits(a.M, a.K, a.N, num_cus);
    return splits > 1 ? pack + gemm_split_bytes(a.M, a.N, splits) : pack;
}

hipError_t launch_quantize(const float *w, int64_t ldw, int K, int N, void *packed, int order, hipStream_t s) {
    const int64_t total = (int64_t)N * (K / 32);
    const int64_t want = (total + 255) / 256;
    const int grid = (int)(want < 65535 ? want : 65535);
    hipLaunchKernelGGL(b1_quantize_kernel, dim3(grid), dim3(256), 0, s, w, ldw, K, N, static_cast<uint8_t *>(packed),
                       order);
    return hipGetLastError();
}

hipError_t launch_norm_mod(const float *x, int64_t ldx, int H, int rows, const float *scale, const float *shift,
                           float eps, float *y, int64_t ldy, void *packed, hipStream_t s) {
    const dim3 grid((rows + 3) / 4);
    uint32_t *pk = static_cast<uint32_t *>(packed);
    if (H <= 512 * 6)
        hipLaunchKernelGGL(b1_norm_mod_kernel<6>, grid, dim3(256), 0, s, x, ldx, H, rows, scale, shift, eps, y, ldy, pk);
    else if (H <= 512 * 24)
        hipLaunchKernelGGL(b1_norm_mod_kernel<24>, grid, dim3(256), 0, s, x, ldx, H, rows, scale, shift, eps, y, ldy,
                           pk);
    else
        hipLaunchKernelGGL(b1_norm_mod_kernel<0>, grid, dim3(256), 0, s, x, ldx, H, rows, scale, shift, eps, y, ldy, pk);
    return hipGetLastError();
}

hipError_t launch_epi(const float *y, int64_t ldy, int M, int N, int kind, const GemmEpi &epi, float *out,
                      int64_t ldo, hipStream_t s) {
    const int cols = kind == 2 ? epi.glu_h : N;
    const int64_t units = (int64_t)M * cols;
    const int64_t want = (units + 255) / 256;
    const int grid = (int)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(b1_epi_kernel, dim3(grid), dim3(256), 0, s, y, ldy, M, cols, kind, epi.gate, epi.res, epi.ldr,
                       epi.glu_h, out, ldo);
    return hipGetLastError();
}

hipError_t launch_epi_packed(const float *y, int64_t ldy, int M, int N, const GemmEpi &epi, float *out,
                             int64_t ldo, hipStream_t s) {
    if (epi.split > 0) {
        const hipError_t e = hipMemcpy2DAsync(out, (size_t)ldo * sizeof(float), y, (size_t)ldy * sizeof(float),
                                              (size_t)epi.split * sizeof(float), (size_t)M,
                                              hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return e;
    }
    if (epi.split >= N) return hipSuccess;
    const float *src = y + epi.split;
    const int64_t ldp = epi.ldpw * 2;
    switch (epi.act) {
    case 0: return launch_pack(src, ldy, M, N - epi.split, epi.pk, ldp, s);
    case 1: return launch_gelu_pack(src, ldy, M, N - epi.split, epi.pk, ldp, s);
    case 2: return launch_swiglu_pack(src, ldy, M, epi.glu_h, epi.pk, ldp, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gelu(const float *x, int64_t ldx, float *y, int64_t ldy, int cols, int rows, hipStream_t s) {
    const int64_t units = (int64_t)rows * (cols / 4);
    const int64_t want = (units + 1023) / 1024; // 4 units a thread
    const int grid = (int)(want < 65535 ? want : 65535);
    const bool nt = (uint64_t)rows * (uint64_t)cols * 4 > kNtInputBytes;
    hipLaunchKernelGGL(nt ? b1_gelu_kernel<true> : b1_gelu_kernel<false>, dim3(grid), dim3(256), 0, s, x, ldx, y, ldy,
                       cols, rows);
    return hipGetLastError();
}

hipError_t launch_gelu_pack(const float *act, int64_t lda, int M, int K, void *packed, int64_t ldp,
                            hipStream_t s) {
    const int units = M * (K / 32) * 4;
    const int pgrid = (units + 255) / 256 < 65535 ? (units + 255) / 256 : 65535;
    const bool nt = (uint64_t)M * (uint64_t)K * 4 > kNtInputBytes;
    hipLaunchKernelGGL(nt ? b1_gelu_pack_kernel<true> : b1_gelu_pack_kernel<false>, dim3(pgrid), dim3(256), 0, s,
                       act, lda, static_cast<uint32_t *>(packed), ldp / 2, M, K);
    return hipGetLastError();
}

hipError_t launch_swiglu_pack(const float *act, int64_t lda, int M, int H, void *packed, int64_t ldp,
                              hipStream_t s) {
    const int units = M * (H / 32) * 4;
    const int pgrid = (units + 255) / 256 < 65535 ? (units + 255) / 256 : 65535;
    const bool nt = (uint64_t)M * (uint64_t)H * 8 > kNtInputBytes;
    hipLaunchKernelGGL(nt ? b1_swiglu_pack_kernel<true> : b1_swiglu_pack_kernel<false>, dim3(pgrid), dim3(256), 0,
                       s, act, lda, static_cast<uint32_t *>(packed), ldp / 2, M, H);
    return hipGetLastError();
}

bool gemv_supported(const LinearArgs &a) { return a.M <= kGemvMaxM && fast_layout_ok(a); }

static hipError_t gemv_attrs() {
    static std::once_flag attr_once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(attr_once, [] {
        const void *g3[] = {
            reinterpret_cast<const void *>(&b1_gemv3_kernel<8, false>),
            reinterpret_cast<const void *>(&b1_gemv3_kernel<16, false>),
            reinterpret_cast<const void *>(&b1_gemv3_kernel<1, true>),
            reinterpret_cast<const void *>(&b1_gemv3_kernel<2, true>),
            reinterpret_cast<const void *>(&b1_gemv3_kernel<4, true>),
            reinterpret_cast<const void *>(&b1_gemv3_kernel<8, true>),
            reinterpret_cast<const void *>(&b1_gemv3_kernel<16, true>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<1, kG4WL2, false>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<2, kG4WL2, false>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<4, kG4WL2, false>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<8, kG4WL1, false>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<16, kG4WL1, false>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<1, kG4WL2, true>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<2, kG4WL2, true>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<4, kG4WL2, true>),
            reinterpret_cast<const void *>(&b1_gemv_group_kernel<8, kG4WL1, true>),
        };
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void *>(&b1_gemv_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kGvLds);
        for (const void *f : g3)
            if (attr_err == hipSuccess)
                attr_err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kG3Lds);
    });
    return attr_err;
}

// Weights staged through LDS when rows are 16-byte multiples and the weight
// bytes fit a buffer resource's 31-bit range.
static bool gemv_staged(int K, int N) {
    return K % 256 == 0 && (uint64_t)N * (uint64_t)(K / 32) * 6 < (1ull << 31);
}

// One work-group per CU, at most kGvMaxRG row groups each, at least one.
static_assert(kGvMaxRG < 16, "row groups per work-group in 4 bits");
static void gemv_grid(int N, int num_cus, int *nwg_out, int *groups_out, int *qr_out = nullptr) {
    const int groups = (N + 15) / 16;
    int nwg = num_cus > 0 ? num_cus : 256;
    const int need = (groups + kGvMaxRG - 1) / kGvMaxRG;
    if (nwg < need) nwg = need;
    if (nwg > groups) nwg = groups;
    *nwg_out = nwg;
    *groups_out = groups;
    if (qr_out) {
        const int q = groups / nwg; // 1 .. kGvMaxRG
        *qr_out = q | (groups - q * nwg) << 4;
    }
}

static hipError_t gemv_group_run(const void *act, int64_t lda, const float *rsc, bool f32, int K, int M,
                                 const GemvGroupOp *ops, int nops, int32_t *nonfinite, int num_cus, hipStream_t s);

hipError_t launch_gemv(const LinearArgs &a, int num_cus, hipStream_t s) {
    const hipError_t attr_err = gemv_attrs();
    if (attr_err != hipSuccess) return attr_err;
    // up to 4 tokens at K <= 3072: the grouped kernel with one op (the same
    // bits; 7.6 against 8.3 us at M = 1, 8.2 against 8.4 at M = 4, K = 3072,
    // N = 18432, graph replay; from 5 tokens on b1_gemv3_kernel<8, false>
    // is as fast or faster: 8.8 against 9.05 us at M = 8)
    {
        const GemvGroupOp op{a.w, a.N, a.out, a.ldo};
        if (a.M <= 4 && gemv_group_ok(a.M, a.K, &op, 1) && gemv_group_f32_ok(a.act, a.lda, a.M, a.K))
            return gemv_group_run(a.act, a.lda, nullptr, true, a.K, a.M, &op, 1, a.nonfinite, num_cus, s);
    }
    int nwg, groups, qr;
    gemv_grid(a.N, num_cus, &nwg, &groups, &qr);
    if (gemv_staged(a.K, a.N)) {
        // converts and repairs out-of-range tokens itself
        LinearArgs b = a;
        b.rsc = nullptr;
        // up to 8 tokens whose rows lie in a buffer resource: through LDS
        if (a.M <= 8 && ((uint64_t)(a.M - 1) * (uint64_t)a.lda + (uint64_t)a.K) * 4u < (1ull << 31))
            hipLaunchKernelGGL((b1_gemv3_kernel<8, false>), dim3(nwg), dim3(kGvWaves * 64), kG3Lds, s, b, qr);
        else
            hipLaunchKernelGGL((b1_gemv3_kernel<16, false>), dim3(nwg), dim3(kGvWaves * 64), kG3Lds, s, b, qr);
        return hipGetLastError();
    }
    int mp_log2 = 0;
    while ((1 << mp_log2) < a.M) ++mp_log2;
    hipLaunchKernelGGL(b1_gemv_kernel, dim3(nwg), dim3(kGvWaves * 64), kGvLds, s, a, groups, mp_log2);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? launch_fixup_rows(a, s) : e;
}

bool gemv_packed_ok(int M, int K, int N) {
    return M >= 1 && M <= kGemvMaxM && gemm_packed_ok(M, K, N) && gemv_staged(K, N) &&
           (uint64_t)M * (uint64_t)K * 2 < (1ull << 31);
}

hipError_t launch_gemv_packed(const void *packed, const uint8_t *w, int K, int N, int M, float *out, int64_t ldo,
                              int32_t *nonfinite, int num_cus, hipStream_t s, const float *rsc) {
    const hipError_t attr_err = gemv_attrs();
    if (attr_err != hipSuccess) return attr_err;
    const LinearArgs a{static_cast<const float *>(packed), K, w, K, N, M, out, ldo, nonfinite, rsc};
    int nwg, groups, qr;
    gemv_grid(N, num_cus, &nwg, &groups, &qr);
    const dim3 grid(nwg), block(kGvWaves * 64);
    if (M <= 1)
        hipLaunchKernelGGL((b1_gemv3_kernel<1, true>), grid, block, kG3Lds, s, a, qr);
    else if (M <= 2)
        hipLaunchKernelGGL((b1_gemv3_kernel<2, true>), grid, block, kG3Lds, s, a, qr);
    else if (M <= 4)
        hipLaunchKernelGGL((b1_gemv3_kernel<4, true>), grid, block, kG3Lds, s, a, qr);
    else if (M <= 8)
        hipLaunchKernelGGL((b1_gemv3_kernel<8, true>), grid, block, kG3Lds, s, a, qr);
    else
        hipLaunchKernelGGL((b1_gemv3_kernel<16, true>), grid, block, kG3Lds, s, a, qr);
    return hipGetLastError();
}

bool gemv_group_ok(int M, int K, const GemvGroupOp *ops, int nops) {
    if (nops < 1 || nops > kGemvGroupMax || M < 1 || M > kGemvMaxM || K < 1 || K > kG3Chunk * 32) return false;
    int64_t groups = 0;
    for (int i = 0; i < nops; ++i) {
        if (ops[i].N < 1 || !gemv_staged(K, ops[i].N)) return false;
        groups += (ops[i].N + 15) / 16;
    }
    return groups <= INT32_MAX;
}

// Both forms of the grouped launch: packed fp16 activations (with the row
// scales of a range-safe packing) or, at most 8 tokens, fp32 rows.
static hipError_t gemv_group_run(const void *act, int64_t lda, const float *rsc, bool f32, int K, int M,
                                 const GemvGroupOp *ops, int nops, int32_t *nonfinite, int num_cus, hipStream_t s) {
    const hipError_t attr_err = gemv_attrs();
    if (attr_err != hipSuccess) return attr_err;
    GemvGroup p{};
    int groups[kGemvGroupMax] = {};
    int gs = 0; // row groups of all the ops
    for (int o = 0; o < kGemvGroupMax; ++o) {
        const GemvGroupOp &op = ops[o < nops ? o : 0];
        p.w[o] = op.w;
        p.out[o] = op.out;
        p.ldo[o] = o < nops ? op.ldo : 0;
        p.N[o] = o < nops ? op.N : 0;
        groups[o] = o < nops ? (op.N + 15) / 16 : 0;
        gs += groups[o];
    }
    p.K = K;
    p.M = M;
    p.act = act;
    p.lda = lda;
    p.rsc = rsc;
    p.nonfinite = nonfinite;
    // work-groups per op: in proportion to its row groups over the CUs'
    // slots (two per CU where a work-group takes half the LDS), at least
    // ceil(groups / P) so that one pass holds them, at most its row groups
    const int cus = num_cus > 0 ? num_cus : 256;
    auto launch = [&](auto kern, int P, int per_cu, int lds) {
        const int64_t slots = (int64_t)per_cu * cus;
        int nwg = 0;
        for (int o = 0; o < kGemvGroupMax; ++o) {
            p.wgstart[o] = nwg;
            if (o >= nops) continue;
            const int g = groups[o];
            int64_t k = (int64_t)g * slots / gs;
            if (k < (g + P - 1) / P) k = (g + P - 1) / P;
            if (k > g) k = g;
            if (k < 1) k = 1;
            const int q = g / (int)k; // 1 .. P
            p.rgqr[o] = q | (g - q * (int)k) << 4;
            nwg += (int)k;
        }
        p.wgstart[kGemvGroupMax] = nwg;
        hipLaunchKernelGGL(kern, dim3(nwg), dim3(kGvWaves * 64), lds, s, p);
    };
    if (f32) {
        if (M <= 1)
            launch(b1_gemv_group_kernel<1, kG4WL2, true>, G4Cfg<1, kG4WL2, true>::P, 2, G4Cfg<1, kG4WL2, true>::Lds);
        else if (M <= 2)
            launch(b1_gemv_group_kernel<2, kG4WL2, true>, G4Cfg<2, kG4WL2, true>::P, 2, G4Cfg<2, kG4WL2, true>::Lds);
        else if (M <= 4)
            launch(b1_gemv_group_kernel<4, kG4WL2, true>, G4Cfg<4, kG4WL2, true>::P, 2, G4Cfg<4, kG4WL2, true>::Lds);
        else
            launch(b1_gemv_group_kernel<8, kG4WL1, true>, G4Cfg<8, kG4WL1, true>::P, 1, G4Cfg<8, kG4WL1, true>::Lds);
    } else if (M <= 1) {
        launch(b1_gemv_group_kernel<1, kG4WL2, false>, G4Cfg<1, kG4WL2>::P, 2, G4Cfg<1, kG4WL2>::Lds);
    } else if (M <= 2) {
        launch(b1_gemv_group_kernel<2, kG4WL2, false>, G4Cfg<2, kG4WL2>::P, 2, G4Cfg<2, kG4WL2>::Lds);
    } else if (M <= 4) {
        launch(b1_gemv_group_kernel<4, kG4WL2, false>, G4Cfg<4, kG4WL2>::P, 2, G4Cfg<4, kG4WL2>::Lds);
    } else if (M <= 8) {
        launch(b1_gemv_group_kernel<8, kG4WL1, false>, G4Cfg<8, kG4WL1>::P, 1, G4Cfg<8, kG4WL1>::Lds);
    } else {
        launch(b1_gemv_group_kernel<16, kG4WL1, false>, G4Cfg<16, kG4WL1>::P, 1, G4Cfg<16, kG4WL1>::Lds);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_group(const void *packed, const float *rsc, int K, int M, const GemvGroupOp *ops, int nops,
                             int32_t *nonfinite, int num_cus, hipStream_t s) {
    return gemv_group_run(packed, K, rsc, false, K, M, ops, nops, nonfinite, num_cus, s);
}

bool gemv_group_f32_ok(const float *act, int64_t lda, int M, int K) {
    return M >= 1 && M <= kGemvGroupF32MaxM && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(act) & 15) == 0 &&
           ((uint64_t)(M - 1) * (uint64_t)lda + (uint64_t)K) * 4u < (1ull << 31);
}

hipError_t launch_gemv_group_f32(const float *act, int64_t lda, int K, int M, const GemvGroupOp *ops, int nops,
                                 int32_t *nonfinite, int num_cus, hipStream_t s) {
    return gemv_group_run(act, lda, nullptr, true, K, M, ops, nops, nonfinite, num_cus, s);
}

} // namespace b1
