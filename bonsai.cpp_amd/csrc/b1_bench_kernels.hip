// Measurement kernels for bench.py (not part of the B1_0 linear): the time a
// launch takes to read a given number of bytes from HBM and do nothing else,
// the floor against which the small-M kernels' per-launch times are read.
// Built into lib/libb1bench.so, separate from the library proper.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Work-group b reads 16-byte words [b * per, (b + 1) * per) of src (the last
// one fewer), four loads in flight per lane, and folds them into one word
// that it writes to sink[b] only when it equals `magic` (an argument, so the
// compiler cannot drop the loads; a match only writes the sink).
__global__ __launch_bounds__(1024) void b1bench_read_kernel(const u32x4 *__restrict__ src, size_t n16, size_t per,
                                                           uint32_t *sink, uint32_t magic) {
    const size_t lo = (size_t)blockIdx.x * per;
    const size_t hi = lo + per < n16 ? lo + per : n16;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (size_t i = lo + threadIdx.x; i < hi; i += 4 * (size_t)blockDim.x) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const size_t j = i + (size_t)u * blockDim.x;
            v[u] = j < hi ? src[j] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u];
    }
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == magic) sink[blockIdx.x] = x;
}

} // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, src 16-byte aligned) with nwg work-groups
// of `block` threads (block <= 1024); sink holds nwg words.  0 on success.
int b1bench_read(const void *src, size_t bytes, void *sink, int nwg, int block, hipStream_t stream) {
    if (!src || !sink || bytes % 16 || ((uintptr_t)src & 15) || nwg < 1 || block < 64 || block > 1024 ||
        block % 64)
        return 1;
    const size_t n16 = bytes / 16, per = (n16 + nwg - 1) / nwg;
    hipLaunchKernelGGL(b1bench_read_kernel, dim3(nwg), dim3(block), 0, stream, static_cast<const u32x4 *>(src), n16,
                       per, static_cast<uint32_t *>(sink), 0x9E3779B9u);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

} // extern "C"
