/* A plain C caller of libxpuint8: no Python and no torch, only the HIP
 * runtime and include/xpuint8.h, the way the reference's native callers would
 * bind the library.  It prepares a weight and runs the one-call INT8 linear
 * on a stream of its own, then checks two argument errors.
 *
 *   linear_consumer DIR M N K
 *
 * reads DIR/x.bin (bf16 [M,K]), DIR/w.bin (bf16 [N,K]) and DIR/b.bin (bf16
 * [N]); writes DIR/w8.bin (int8 [N,K]), DIR/ws.bin (fp32 [N]) and DIR/y.bin
 * (bf16 [M,N]).  Exit status 0 on success. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "xpuint8.h"

#define HIP_OK(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess) {                                                   \
            fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));            \
            return 2;                                                             \
        }                                                                         \
    } while (0)

static void *read_file(const char *dir, const char *name, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    void *p = malloc(bytes);
    size_t got = p ? fread(p, 1, bytes, f) : 0;
    fclose(f);
    if (got != bytes) {
        free(p);
        return NULL;
    }
    return p;
}

static int write_file(const char *dir, const char *name, const void *p, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f) return 1;
    size_t put = fwrite(p, 1, bytes, f);
    fclose(f);
    return put != bytes;
}

int main(int argc, char **argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s DIR M N K\n", argv[0]);
        return 2;
    }
    const char *dir = argv[1];
    const int64_t M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
    const size_t xb = (size_t)(M * K) * 2, wb = (size_t)(N * K) * 2, bb = (size_t)N * 2;
    const size_t yb = (size_t)(M * N) * 2;
    void *hx = read_file(dir, "x.bin", xb), *hw = read_file(dir, "w.bin", wb);
    void *hb = read_file(dir, "b.bin", bb);
    if (!hx || !hw || !hb) {
        fprintf(stderr, "cannot read the inputs in %s\n", dir);
        return 2;
    }
    if (xpuint8_init() != 0) {
        fprintf(stderr, "xpuint8_init: %s\n", xpuint8_last_error());
        return 1;
    }
    printf("device: %s\n", xpuint8_device_name());

    void *dx, *dw, *db, *dy, *dws, *dw8, *work = NULL;
    HIP_OK(hipMalloc(&dx, xb));
    HIP_OK(hipMalloc(&dw, wb));
    HIP_OK(hipMalloc(&db, bb));
    HIP_OK(hipMalloc(&dy, yb));
    HIP_OK(hipMalloc(&dw8, (size_t)(N * K)));
    HIP_OK(hipMalloc(&dws, (size_t)N * 4));
    HIP_OK(hipMemcpy(dx, hx, xb, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dw, hw, wb, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(db, hb, bb, hipMemcpyHostToDevice));

    hipStream_t s;
    HIP_OK(hipStreamCreate(&s));
    if (xpuint8_prepare_weight_stream(s, dw, (int8_t *)dw8, (float *)dws, N, K) != 0) {
        fprintf(stderr, "prepare_weight: %s\n", xpuint8_last_error());
        return 1;
    }
    const int64_t need = xpuint8_linear_workspace_size(M, N, K);
    if (need < 0) {
        fprintf(stderr, "linear_workspace_size: %s\n", xpuint8_last_error());
        return 1;
    }
    if (need > 0) HIP_OK(hipMalloc(&work, (size_t)need));
    if (xpuint8_linear_stream(s, dx, (const int8_t *)dw8, (const float *)dws, db, 1, dy, M, N,
                              K, work, need) != 0) {
        fprintf(stderr, "linear: %s\n", xpuint8_last_error());
        return 1;
    }
    HIP_OK(hipStreamSynchronize(s));

    /* argument errors come back as codes and messages, before any device work */
    if (xpuint8_linear_stream(s, dx, (const int8_t *)dw8, (const float *)dws, db, 1, dy, M, N,
                              K + 16, work, need) != 3 ||
        strstr(xpuint8_last_error(), "256") == NULL) {
        fprintf(stderr, "K %% 256 != 0 not rejected as expected: %s\n", xpuint8_last_error());
        return 1;
    }
    if (need > 0 &&
        xpuint8_linear_stream(s, dx, (const int8_t *)dw8, (const float *)dws, db, 1, dy, M, N,
                              K, work, need - 1) == 0) {
        fprintf(stderr, "a short workspace was accepted\n");
        return 1;
    }

    void *hy = malloc(yb), *hw8 = malloc((size_t)(N * K)), *hws = malloc((size_t)N * 4);
    HIP_OK(hipMemcpy(hy, dy, yb, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hw8, dw8, (size_t)(N * K), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hws, dws, (size_t)N * 4, hipMemcpyDeviceToHost));
    if (write_file(dir, "y.bin", hy, yb) || write_file(dir, "w8.bin", hw8, (size_t)(N * K)) ||
        write_file(dir, "ws.bin", hws, (size_t)N * 4)) {
        fprintf(stderr, "cannot write the outputs in %s\n", dir);
        return 2;
    }
    HIP_OK(hipStreamDestroy(s));
    HIP_OK(hipFree(dx));
    HIP_OK(hipFree(dw));
    HIP_OK(hipFree(db));
    HIP_OK(hipFree(dy));
    HIP_OK(hipFree(dw8));
    HIP_OK(hipFree(dws));
    if (work) HIP_OK(hipFree(work));
    free(hx);
    free(hw);
    free(hb);
    free(hy);
    free(hw8);
    free(hws);
    printf("ok\n");
    return 0;
}
