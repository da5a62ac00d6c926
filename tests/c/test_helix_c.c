/* test_helix_c.c -- a C program that links libhelix.a (the CMake target
 * helix::helix) and uses nothing but include/helix/helix.h and helix_host.h,
 * the way a ggml backend or any other C host would.
 *
 *   1. Host-only context (no GPU needed): descriptor defaults, the shape gate,
 *      the scratch plan of BASELINE config 0 (L=256 S=1 H=8 P=64 N=64 G=1).
 *   2. With a GPU: config 0 encoded on both multipass paths and compared with
 *      the C oracle (oracle/helix_oracle.c, test infrastructure: the checker,
 *      never the thing tested), at the reference parity test's bounds
 *      (tests/test_metal_parity.mm:35-38, 210-218):
 *        fp32 path (backend SGMMA): y and s1 per element within 5e-6 rel + 5e-7 abs
 *        bf16 path (backend MPP):   y within 1.5e-2 rel + 3e-3 abs,
 *                                   s1 at the fp32 bound (its state stays fp32-accurate)
 *
 * Exit status 0 on success. Without a GPU the device part is skipped unless
 * --require-gpu is given; --host-only skips it on any machine.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "helix/helix.h"
#include "helix/helix_host.h"
#include "helix_oracle.h"

static int failures = 0;

#define CHECK(cond, ...)                              \
    do {                                              \
        if (!(cond)) {                                \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);             \
            fprintf(stderr, "\n");                    \
            ++failures;                               \
        }                                             \
    } while (0)

static helix_tensor dev_tensor(void* p) {
    helix_tensor t;
    t.buf = p;
    t.offset = 0;
    return t;
}

/* Largest per-element excess |got - want| / (abs + rel |want|); <= 1 passes. */
static double excess(const float* got, const float* want, size_t n, double rel, double abs_tol) {
    double worst = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double e = fabs((double)got[i] - (double)want[i]) / (abs_tol + rel * fabs((double)want[i]));
        if (!(e <= worst)) worst = e;   /* NaN propagates as a failure */
    }
    return worst;
}

static void host_checks(void) {
    helix_ctx* h = NULL;
    CHECK(helix_ctx_create_host(&h) == HELIX_OK && h, "helix_ctx_create_host");
    if (!h) return;
    helix_scan_desc d;
    helix_scan_desc_init(&d, 256, 1, 8, 64, 64, 1);
    CHECK(d.s_x[0] == 8 * 64 && d.s_x[1] == 64 && d.s_x[2] == 1, "dense x strides");
    CHECK(d.chunk == 0 && d.io_dtype == HELIX_F32, "descriptor defaults");
    d.multipass = true;
    CHECK(helix_scan_supported(h, &d), "config 0 declined: %s", helix_ctx_last_error(h));
    const size_t bytes = helix_scan_scratch_size(h, &d);
    CHECK(bytes > 0, "multipass scratch size");
    helix_plan_info pi;
    CHECK(helix_scan_plan_info(h, &d, &pi) == HELIX_OK, "plan info");
    printf("host: config 0 scratch %zu bytes, kernels %s / %s / %s\n", bytes, pi.kernel_a, pi.kernel_b,
           pi.kernel_c);
    helix_scan_desc bad = d;
    bad.n_group = 3;   /* does not divide n_head */
    CHECK(!helix_scan_supported(h, &bad), "n_group not dividing n_head accepted");
    helix_ctx_free(h);
}

static int device_checks(void) {
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || n_dev == 0) return 0;
    helix_ctx* ctx = NULL;
    if (helix_ctx_create(&ctx, NULL, NULL) != HELIX_OK) {
        fprintf(stderr, "helix_ctx_create: %s\n", helix_ctx_last_error(NULL));
        return 0;
    }
    const int L = 256, S = 1, H = 8, P = 64, N = 64, G = 1;
    const size_t nx = (size_t)S * L * H * P, nb = (size_t)S * L * G * N, ndt = (size_t)S * L * H,
                 ns = (size_t)S * H * P * N;
    float* s0 = calloc(ns, 4);
    float* x = malloc(nx * 4);
    float* dt = malloc(ndt * 4);
    float* A = malloc(H * 4);
    float* B = malloc(nb * 4);
    float* C = malloc(nb * 4);
    float* y_ref = malloc(nx * 4);
    float* s1_ref = malloc(ns * 4);
    float* y = malloc(nx * 4);
    float* s1 = malloc(ns * 4);
    /* BASELINE config 0: x ~ N(0,1), dt = softplus(N(-1, 0.5)), A = -exp(U(ln 1, ln 16)),
     * B, C ~ N(0,1)/sqrt(N), zero initial state. */
    oracle_problem_gauss(L, S, H, P, N, G, 20260101u, 0.0, -1.0, 0.5, 1.0, 16.0, s0, x, dt, A, B, C);

    helix_scan_desc d;
    helix_scan_desc_init(&d, L, S, H, P, N, G);
    d.multipass = true;
    oracle_scan(&d, s0, x, dt, A, B, C, NULL, y_ref, s1_ref, NULL);

    void *d_s0, *d_x, *d_dt, *d_A, *d_B, *d_C, *d_y, *d_s1, *d_scr;
    int ok = hipMalloc(&d_s0, ns * 4) == hipSuccess && hipMalloc(&d_x, nx * 4) == hipSuccess &&
             hipMalloc(&d_dt, ndt * 4) == hipSuccess && hipMalloc(&d_A, H * 4) == hipSuccess &&
             hipMalloc(&d_B, nb * 4) == hipSuccess && hipMalloc(&d_C, nb * 4) == hipSuccess &&
             hipMalloc(&d_y, nx * 4) == hipSuccess && hipMalloc(&d_s1, ns * 4) == hipSuccess;
    CHECK(ok, "hipMalloc");
    ok = ok && hipMemcpy(d_s0, s0, ns * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_x, x, nx * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_dt, dt, ndt * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_A, A, H * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_B, B, nb * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_C, C, nb * 4, hipMemcpyHostToDevice) == hipSuccess;
    CHECK(ok, "hipMemcpy to device");

    const helix_backend backends[2] = {HELIX_BACKEND_SGMMA, HELIX_BACKEND_MPP};
    const char* names[2] = {"fp32 path (SGMMA)", "bf16 path (MPP)"};
    const double y_rel[2] = {5e-6, 1.5e-2}, y_abs[2] = {5e-7, 3e-3};
    for (int k = 0; ok && k < 2; ++k) {
        d.backend = backends[k];
        const size_t sb = helix_scan_scratch_size(ctx, &d);
        d_scr = NULL;
        if (sb && hipMalloc(&d_scr, sb) != hipSuccess) {
            CHECK(0, "hipMalloc scratch");
            break;
        }
        const helix_status st =
            helix_scan_encode(ctx, NULL, &d, dev_tensor(d_s0), dev_tensor(d_x), dev_tensor(d_dt), dev_tensor(d_A),
                              dev_tensor(d_B), dev_tensor(d_C), HELIX_TENSOR_NULL, dev_tensor(d_y),
                              dev_tensor(d_s1), sb ? dev_tensor(d_scr) : HELIX_TENSOR_NULL);
        CHECK(st == HELIX_OK, "%s encode: %s", names[k], helix_ctx_last_error(ctx));
        CHECK(hipDeviceSynchronize() == hipSuccess, "hipDeviceSynchronize");
        CHECK(hipMemcpy(y, d_y, nx * 4, hipMemcpyDeviceToHost) == hipSuccess &&
                  hipMemcpy(s1, d_s1, ns * 4, hipMemcpyDeviceToHost) == hipSuccess,
              "hipMemcpy to host");
        if (d_scr) (void)hipFree(d_scr);
        const double ey = excess(y, y_ref, nx, y_rel[k], y_abs[k]);
        const double es = excess(s1, s1_ref, ns, 5e-6, 5e-7);
        printf("gpu: %-20s %s: y excess %.3f, s1 excess %.3f (<= 1 passes)\n", names[k],
               helix_ctx_backend_desc(ctx, &d), ey, es);
        CHECK(ey <= 1.0, "%s: y outside the bound", names[k]);
        CHECK(es <= 1.0, "%s: s1 outside the fp32 bound", names[k]);
    }
    (void)hipFree(d_s0); (void)hipFree(d_x); (void)hipFree(d_dt); (void)hipFree(d_A);
    (void)hipFree(d_B); (void)hipFree(d_C); (void)hipFree(d_y); (void)hipFree(d_s1);
    free(s0); free(x); free(dt); free(A); free(B); free(C); free(y_ref); free(s1_ref); free(y); free(s1);
    helix_ctx_free(ctx);
    return 1;
}

int main(int argc, char** argv) {
    const int require_gpu = argc > 1 && strcmp(argv[1], "--require-gpu") == 0;
    const int host_only = argc > 1 && strcmp(argv[1], "--host-only") == 0;
    host_checks();
    const int ran = host_only ? 0 : device_checks();
    if (!ran) {
        printf("gpu: no device, device checks skipped\n");
        if (require_gpu) ++failures;
    }
    printf(failures ? "test_helix_c: %d failure(s)\n" : "test_helix_c: passed\n", failures);
    return failures ? 1 : 0;
}
