// The reference's single-op harness (tests/c_ops/test_b1_linear.cpp) on the
// MI355X library: same command line, same files.
//
//   b1_linear_hip <act.bin> <weight.bin> <out.bin> [batch] [in_dim] [out_dim] [mode]
//
//   act.bin    fp32 [batch * in_dim] (row-major)
//   weight.bin fp32 [out_dim * in_dim] (row-major), packed to B1_0 on the
//              device by bonsai_b1_quantize_f32 with the left-to-right block
//              sum of the reference harness's own writer (:129-163)
//   out.bin    fp32 [batch * out_dim]
//   mode       auto (default) | exact | gemm | gemv
//
// Defaults and checks follow the reference harness (:177-213): batch 1,
// in_dim 64, out_dim 32; the element counts of the inputs must match.
// Exit status: 0 on success, 1 on a usage or input error, 2 on a device or
// library error, 3 when the output holds NaN/Inf (the reference aborts).
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "bonsai_b1.h"

static float *read_float_bin(const char *path, size_t *count) {
    FILE *f = fopen(path, "rb");
    if (!f) {
        perror(path);
        return NULL;
    }
    fseek(f, 0, SEEK_END);
    const long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (size < 0) {
        fclose(f);
        return NULL;
    }
    float *data = (float *)malloc(size > 0 ? (size_t)size : 1);
    const size_t got = data ? fread(data, 1, (size_t)size, f) : 0;
    fclose(f);
    if (!data || got != (size_t)size) {
        fprintf(stderr, "short read of %s\n", path);
        free(data);
        return NULL;
    }
    *count = (size_t)size / sizeof(float);
    return data;
}

static int write_float_bin(const char *path, const float *data, size_t count) {
    FILE *f = fopen(path, "wb");
    if (!f) {
        perror(path);
        return 0;
    }
    const size_t put = fwrite(data, sizeof(float), count, f);
    fclose(f);
    return put == count;
}

#define HIP_OK(call)                                                                \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));       \
            return 2;                                                               \
        }                                                                           \
    } while (0)

int main(int argc, char **argv) {
    if (argc < 4) {
        fprintf(stderr, "Usage: %s <act.bin> <weight.bin> <out.bin> [batch] [in_dim] [out_dim] [mode]\n", argv[0]);
        fprintf(stderr, "  act.bin    : float32 [batch * in_dim]\n");
        fprintf(stderr, "  weight.bin : float32 [out_dim * in_dim]\n");
        fprintf(stderr, "  out.bin    : float32 [batch * out_dim]\n");
        fprintf(stderr, "  mode       : auto | exact | gemm | gemv\n");
        return 1;
    }
    const int batch = argc > 4 ? atoi(argv[4]) : 1;
    const int in_dim = argc > 5 ? atoi(argv[5]) : 64;
    const int out_dim = argc > 6 ? atoi(argv[6]) : 32;
    int mode = BONSAI_B1_MODE_AUTO;
    if (argc > 7) {
        if (!strcmp(argv[7], "exact")) mode = BONSAI_B1_MODE_EXACT;
        else if (!strcmp(argv[7], "gemm")) mode = BONSAI_B1_MODE_GEMM;
        else if (!strcmp(argv[7], "gemv")) mode = BONSAI_B1_MODE_GEMV;
        else if (strcmp(argv[7], "auto")) {
            fprintf(stderr, "unknown mode %s\n", argv[7]);
            return 1;
        }
    }
    printf("Testing b1_linear: batch=%d in_dim=%d out_dim=%d\n", batch, in_dim, out_dim);
    if (batch <= 0 || in_dim <= 0 || out_dim <= 0 || in_dim % BONSAI_B1_BLOCK_SIZE) {
        fprintf(stderr, "Error: need batch, out_dim > 0 and in_dim a positive multiple of %d\n",
                BONSAI_B1_BLOCK_SIZE);
        return 1;
    }

    size_t act_count = 0, weight_count = 0;
    float *act = read_float_bin(argv[1], &act_count);
    float *weight = read_float_bin(argv[2], &weight_count);
    if (!act || !weight) {
        fprintf(stderr, "Error reading input files\n");
        return 1;
    }
    printf("  Read %zu floats from %s\n", act_count, argv[1]);
    printf("  Read %zu floats from %s\n", weight_count, argv[2]);
    if (act_count != (size_t)batch * in_dim) {
        fprintf(stderr, "Error: expected act_count=%zu, got %zu\n", (size_t)batch * in_dim, act_count);
        return 1;
    }
    if (weight_count != (size_t)out_dim * in_dim) {
        fprintf(stderr, "Error: expected weight_count=%zu, got %zu\n", (size_t)out_dim * in_dim, weight_count);
        return 1;
    }

    hipStream_t s;
    HIP_OK(hipStreamCreate(&s));
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    const size_t packed_bytes = (size_t)out_dim * (in_dim / BONSAI_B1_BLOCK_SIZE) * BONSAI_B1_BLOCK_BYTES;
    float *d_act = NULL, *d_w = NULL, *d_out = NULL;
    void *d_packed = NULL;
    int32_t *d_bad = NULL;
    HIP_OK(hipMalloc((void **)&d_act, act_count * sizeof(float)));
    HIP_OK(hipMalloc((void **)&d_w, weight_count * sizeof(float)));
    HIP_OK(hipMalloc((void **)&d_out, (size_t)batch * out_dim * sizeof(float)));
    HIP_OK(hipMalloc(&d_packed, packed_bytes));
    HIP_OK(hipMalloc((void **)&d_bad, sizeof(int32_t)));
    HIP_OK(hipMemcpyAsync(d_act, act, act_count * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_OK(hipMemcpyAsync(d_w, weight, weight_count * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_OK(hipMemsetAsync(d_bad, 0, sizeof(int32_t), s));

    printf("  Quantizing weights to B1_0...\n");
    int st = bonsai_b1_quantize_f32(d_w, in_dim, in_dim, out_dim, d_packed, BONSAI_B1_SUM_SEQUENTIAL, s);
    if (st != BONSAI_B1_OK) {
        fprintf(stderr, "bonsai_b1_quantize_f32: %s\n", bonsai_b1_status_string(st));
        return 2;
    }

    printf("  Running b1_linear...\n");
    B1Weights w = {d_packed, in_dim, out_dim, packed_bytes, dev};
    B1LinearUserData ud;
    st = bonsai_b1_linear(d_act, &w, batch, d_out, &ud, mode, d_bad, s);
    if (st != BONSAI_B1_OK) {
        fprintf(stderr, "bonsai_b1_linear: %s\n", bonsai_b1_status_string(st));
        return 2;
    }
    const size_t out_count = (size_t)batch * out_dim;
    float *out = (float *)malloc(out_count * sizeof(float));
    int32_t bad = 0;
    if (!out) return 2;
    HIP_OK(hipMemcpyAsync(out, d_out, out_count * sizeof(float), hipMemcpyDeviceToHost, s));
    HIP_OK(hipMemcpyAsync(&bad, d_bad, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    HIP_OK(hipStreamSynchronize(s));
    if (!write_float_bin(argv[3], out, out_count)) return 1;
    printf("  Written %zu floats to %s\n", out_count, argv[3]);

    (void)hipFree(d_act);
    (void)hipFree(d_w);
    (void)hipFree(d_out);
    (void)hipFree(d_packed);
    (void)hipFree(d_bad);
    (void)hipStreamDestroy(s);
    free(act);
    free(weight);
    free(out);
    if (bad) {
        fprintf(stderr, "B1_FATAL_OUT: %d non-finite outputs\n", bad);
        return 3;
    }
    printf("  OK\n");
    return 0;
}
