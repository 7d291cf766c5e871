/* fft_c_abi.c -- the C ABI driven from plain C, the way a Rust (or any FFI)
 * binding of include/ferrum_gpu.h drives it: no Python, no C++.
 *
 * Checks, on GPU 0:
 *   1. an impulse at 0 transforms to all ones (N = 1024, batch 4, host path);
 *   2. a seeded batch (the library's on-device generator) survives a forward +
 *      normalised inverse round trip on device buffers, and the forward
 *      result's bin 0 equals the input sum (DFT definition at k = 0);
 *   3. a 2D impulse transforms to all ones (64 x 64).
 * Exit status 0 on success; prints one line per check.
 *
 * Build: make -C ferrum-gpu_amd/csrc example  (gcc; links libferrum_gpu.so):
 * the executable fft_c_abi, and libfft_c_abi.so exporting the same checks as
 * fft_c_abi_example() for callers that run them in-process (the GPU tests). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "ferrum_gpu.h"

#define CHECK(call)                                                                   \
    do {                                                                              \
        int rc_ = (call);                                                             \
        if (rc_ != FG_OK) {                                                           \
            fprintf(stderr, "%s failed (%d): %s\n", #call, rc_, fg_last_error());     \
            return 1;                                                                 \
        }                                                                             \
    } while (0)

static double max_abs_diff_from(const float* z, size_t n, float re, float im) {
    double m = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double d = fabs((double)z[2 * i] - re) + fabs((double)z[2 * i + 1] - im);
        if (d > m) m = d;
    }
    return m;
}

int fft_c_abi_example(void) {
    int count = 0;
    CHECK(fg_device_count(&count));
    if (count < 1) {
        fprintf(stderr, "no GPU visible\n");
        return 2;
    }
    fg_device_t dev;
    CHECK(fg_device_open(0, &dev));

    /* 1. impulse -> all ones, through the host-memory entry point */
    const uint32_t log_n = 10;
    const size_t n = (size_t)1 << log_n, batch = 4, total = n * batch;
    float* x = (float*)calloc(2 * total, sizeof(float));
    float* y = (float*)malloc(2 * total * sizeof(float));
    if (!x || !y) return 1;
    for (size_t b = 0; b < batch; ++b) x[2 * b * n] = 1.0f;
    CHECK(fg_fft_1d_c2c_pow2_host(dev, x, y, total, log_n, FG_FORWARD, 0));
    double e1 = max_abs_diff_from(y, total, 1.0f, 0.0f);
    printf("impulse -> ones (N=%zu, batch %zu): max |error| %.3g\n", n, batch, e1);

    /* 2. seeded device-resident round trip */
    fg_fft_plan_t plan;
    CHECK(fg_fft_plan_1d(dev, log_n, batch, &plan));
    void *d_in, *d_mid, *d_out;
    CHECK(fg_alloc_zeros(dev, 8 * total, &d_in));
    CHECK(fg_alloc_zeros(dev, 8 * total, &d_mid));
    CHECK(fg_alloc_zeros(dev, 8 * total, &d_out));
    CHECK(fg_fill_uniform_c64(dev, d_in, total, 1, NULL));
    CHECK(fg_fft_exec(plan, d_in, d_mid, FG_FORWARD, 0, NULL));
    CHECK(fg_fft_exec(plan, d_mid, d_out, FG_INVERSE, 1, NULL));
    CHECK(fg_device_sync(dev));
    float* h_in = (float*)malloc(2 * total * sizeof(float));
    float* h_mid = (float*)malloc(2 * total * sizeof(float));
    float* h_out = (float*)malloc(2 * total * sizeof(float));
    if (!h_in || !h_mid || !h_out) return 1;
    CHECK(fg_copy_d2h(dev, h_in, d_in, 8 * total));
    CHECK(fg_copy_d2h(dev, h_mid, d_mid, 8 * total));
    CHECK(fg_copy_d2h(dev, h_out, d_out, 8 * total));
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < 2 * total; ++i) {
        double d = (double)h_out[i] - h_in[i];
        num += d * d;
        den += (double)h_in[i] * h_in[i];
    }
    double rt = sqrt(num / den);
    double s_re = 0.0, s_im = 0.0;
    for (size_t i = 0; i < n; ++i) {
        s_re += h_in[2 * i];
        s_im += h_in[2 * i + 1];
    }
    double e0 = fabs(h_mid[0] - s_re) + fabs(h_mid[1] - s_im);
    printf("round trip rel-L2 %.3g; X[0] - sum(x) = %.3g\n", rt, e0);

    /* 3. 2D impulse -> all ones */
    const uint32_t log2d = 6;
    const size_t n2 = (size_t)1 << (2 * log2d);
    float* x2 = (float*)calloc(2 * n2, sizeof(float));
    float* y2 = (float*)malloc(2 * n2 * sizeof(float));
    if (!x2 || !y2) return 1;
    x2[0] = 1.0f;
    CHECK(fg_fft_2d_c2c_pow2_host(dev, x2, y2, log2d, 1, FG_FORWARD, 0));
    double e2 = max_abs_diff_from(y2, n2, 1.0f, 0.0f);
    printf("2D impulse -> ones (%zu x %zu): max |error| %.3g\n", (size_t)1 << log2d, (size_t)1 << log2d, e2);

    CHECK(fg_free(dev, d_in));
    CHECK(fg_free(dev, d_mid));
    CHECK(fg_free(dev, d_out));
    CHECK(fg_fft_plan_destroy(plan));
    CHECK(fg_device_close(dev));
    free(x); free(y); free(h_in); free(h_mid); free(h_out); free(x2); free(y2);

    const int ok = e1 < 1e-5 && rt < 1e-5 && e0 < 1e-3 && e2 < 1e-5;
    printf("%s\n", ok ? "OK" : "FAILED");
    fflush(stdout);
    return ok ? 0 : 1;
}

#ifndef FG_EXAMPLE_NO_MAIN
int main(void) { return fft_c_abi_example(); }
#endif
