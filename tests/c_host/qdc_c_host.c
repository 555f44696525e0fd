/*
 * qdc_c_host.c -- a plain C99 host of libqdc_hip.so.
 *
 * Device buffers come from hipMalloc, the library's entry points are called
 * with raw pointers, element strides and dtype codes exactly as include/qdc_hip.h
 * declares them, and every result is checked against a reference loop in double
 * precision.  It stands for any caller that is not Python: the Julia binding
 * calls the same symbols with the same arguments through ccall.
 *
 *   qdc_c_host              every check (needs a GPU)
 *   qdc_c_host --host-only  only the checks that launch nothing: version,
 *                           status strings and argument errors found on the host
 *
 * Exit status 0 when every check passes.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qdc_hip.h"

static int failures = 0;

#define HIP_OK(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess) {                                                   \
            printf("FAIL %s:%d %s -> %s\n", __FILE__, __LINE__, #call,            \
                   hipGetErrorString(e_));                                        \
            exit(2);                                                              \
        }                                                                         \
    } while (0)

static void expect(int ok, const char *what, double value, double bar) {
    printf("%s %-52s %.3e (bar %.0e)\n", ok ? "ok  " : "FAIL", what, value, bar);
    if (!ok) ++failures;
}

static void expect_status(int32_t got, int32_t want, const char *what) {
    const int ok = got == want;
    printf("%s %-52s status %d (%s)\n", ok ? "ok  " : "FAIL", what, got, qdc_status_string(got));
    if (!ok) ++failures;
}

/* ----------------------------------------------------------- helpers ---- */
static uint64_t lcg = 0x9e3779b97f4a7c15ull;
static float uniform(void) { /* [-1, 1) */
    lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
    return (float)((double)(lcg >> 40) / (double)(1ull << 24) * 2.0 - 1.0);
}
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
/* round to nearest even (src/safetensors.jl:37-42), finite values */
static uint16_t to_bf16(float f) {
    const uint32_t b = f2u(f);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
static float from_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }

static double normwise(const double *got, const double *exp, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; ++i) {
        num += (got[i] - exp[i]) * (got[i] - exp[i]);
        den += exp[i] * exp[i];
    }
    return sqrt(num) / (sqrt(den) > 0 ? sqrt(den) : 1.0);
}

/* zero-centred RMSNorm of one row in double: (x * s) * (1 + w) */
static void rms_row(const double *x, const double *w, int width, double eps, double *out) {
    double ss = 0.0;
    for (int i = 0; i < width; ++i) ss += x[i] * x[i];
    const double s = 1.0 / sqrt(ss / width + eps);
    for (int i = 0; i < width; ++i) out[i] = (x[i] * s) * (1.0 + w[i]);
}

static void *dev_alloc(size_t bytes) {
    void *p = NULL;
    HIP_OK(hipMalloc(&p, bytes));
    return p;
}

/* ------------------------------------------------------ host-only checks -- */
static void host_checks(void) {
    const char *v = qdc_version();
    expect(v != NULL && strncmp(v, "qdc_hip ", 8) == 0, "qdc_version", 0.0, 0.0);
    for (int32_t s = 0; s >= -5; --s)
        expect(qdc_status_string(s) != NULL, "qdc_status_string", (double)s, 0.0);
    void *fake = (void *)(uintptr_t)0x10000; /* validation never dereferences it */
    expect_status(qdc_rmsnorm(fake, (char *)fake + 65536, (char *)fake + 131072, 4, 8, 8, 8,
                              1e-6f, 1, 7, QDC_F32, 0),
                  QDC_ERR_DTYPE, "qdc_rmsnorm: unknown dtype");
    expect_status(qdc_rmsnorm(NULL, fake, fake, 4, 8, 8, 8, 1e-6f, 1, QDC_F32, QDC_F32, 0),
                  QDC_ERR_NULL, "qdc_rmsnorm: NULL output");
    expect_status(qdc_swiglu(fake, (char *)fake + 65536, (char *)fake + 131072, 4, 6, 6, 6, 6,
                             QDC_F32, QDC_BF16X2, 0),
                  QDC_ERR_SHAPE, "qdc_swiglu: split output of width 6");
    const int64_t ids[3] = {0, 5, 4096};
    expect_status(qdc_check_ids(ids, 3, 4096), QDC_ERR_RANGE, "qdc_check_ids: id 4096 of 4096");
    expect_status(qdc_check_ids(ids, 2, 4096), QDC_OK, "qdc_check_ids: ids in range");
}

/* ----------------------------------------------------------- GPU checks -- */
static void gpu_checks(void) {
    enum { R = 37, W = 1024, I = 3584, T = 19, V = 512 };
    const double eps = 1e-6;
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));

    float *x = malloc(sizeof(float) * R * W), *wf = malloc(sizeof(float) * W);
    uint16_t *mb = malloc(2 * R * W), *wb = malloc(2 * W);
    double *xd = malloc(sizeof(double) * R * W);
    double *wd = malloc(sizeof(double) * W), *ref = malloc(sizeof(double) * R * W);
    double *got = malloc(sizeof(double) * R * W);
    for (int i = 0; i < R * W; ++i) {
        x[i] = uniform() * 2.0f;
        mb[i] = to_bf16(uniform());
        xd[i] = x[i];
    }
    for (int i = 0; i < W; ++i) {
        wb[i] = to_bf16(uniform() * 0.02f);
        wf[i] = from_bf16(wb[i]);
        wd[i] = wf[i];
    }
    void *dx = dev_alloc(4 * R * W), *dm = dev_alloc(2 * R * W), *dwf = dev_alloc(4 * W);
    void *dwb = dev_alloc(2 * W), *dres = dev_alloc(4 * R * W), *dout = dev_alloc(4 * R * W);
    HIP_OK(hipMemcpy(dx, x, 4 * R * W, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dm, mb, 2 * R * W, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dwf, wf, 4 * W, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dwb, wb, 2 * W, hipMemcpyHostToDevice));

    /* 1. zero-centred RMSNorm, fp32 rows */
    expect_status(qdc_rmsnorm(dout, dx, dwf, R, W, W, W, (float)eps, 1, QDC_F32, QDC_F32, stream),
                  QDC_OK, "qdc_rmsnorm fp32 launch");
    float *of = malloc(4 * R * W);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipMemcpy(of, dout, 4 * R * W, hipMemcpyDeviceToHost));
    for (int r = 0; r < R; ++r) rms_row(xd + r * W, wd, W, eps, ref + r * W);
    for (int i = 0; i < R * W; ++i) got[i] = of[i];
    double err = normwise(got, ref, R * W);
    expect(err <= 1e-5, "qdc_rmsnorm fp32 [37, 1024] vs double", err, 1e-5);

    /* 2. residual + norm: fp32 stream, bf16 addend, bf16 output */
    expect_status(qdc_residual_rmsnorm(dres, dout, dx, dm, dwb, R, W, (float)eps, QDC_F32, QDC_BF16,
                                       QDC_BF16, stream),
                  QDC_OK, "qdc_residual_rmsnorm launch");
    HIP_OK(hipStreamSynchronize(stream));
    float *res = malloc(4 * R * W);
    uint16_t *ob = malloc(2 * R * W);
    HIP_OK(hipMemcpy(res, dres, 4 * R * W, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(ob, dout, 2 * R * W, hipMemcpyDeviceToHost));
    int exact = 1;
    for (int i = 0; i < R * W; ++i) exact &= f2u(res[i]) == f2u(x[i] + from_bf16(mb[i]));
    expect(exact, "qdc_residual_rmsnorm residual = x + mixed, bit-exact", 0.0, 0.0);
    double *sum = malloc(sizeof(double) * R * W);
    for (int i = 0; i < R * W; ++i) sum[i] = res[i];
    for (int r = 0; r < R; ++r) rms_row(sum + r * W, wd, W, eps, ref + r * W);
    for (int i = 0; i < R * W; ++i) got[i] = from_bf16(ob[i]);
    err = normwise(got, ref, R * W);
    expect(err <= 1e-2, "qdc_residual_rmsnorm bf16 output vs double", err, 1e-2);

    /* 3. the same norm written as two bf16 terms per element (fp32 addend) */
    void *dm32 = dev_alloc(4 * R * W);
    float *m32 = malloc(4 * R * W);
    for (int i = 0; i < R * W; ++i) m32[i] = from_bf16(mb[i]);
    HIP_OK(hipMemcpy(dm32, m32, 4 * R * W, hipMemcpyHostToDevice));
    expect_status(qdc_residual_rmsnorm(dres, dx, dx, dm32, dwb, R, W, (float)eps, QDC_F32,
                                       QDC_F32, QDC_BF16X2, stream),
                  QDC_ERR_ALIAS, "qdc_residual_rmsnorm split output over x (refused)");
    expect_status(qdc_residual_rmsnorm(dres, dout, dx, dm32, dwb, R, W, (float)eps, QDC_F32,
                                       QDC_F32, QDC_BF16X2, stream),
                  QDC_OK, "qdc_residual_rmsnorm split launch");
    HIP_OK(hipStreamSynchronize(stream));
    uint16_t *split = malloc(4 * R * W);
    HIP_OK(hipMemcpy(split, dout, 4 * R * W, hipMemcpyDeviceToHost));
    for (int e = 0; e < R * W; ++e) { /* piece of 4 elements: [4 hi | 4 lo] */
        const int g = e / 4, j = e % 4;
        got[e] = (double)from_bf16(split[8 * g + j]) + (double)from_bf16(split[8 * g + 4 + j]);
    }
    err = normwise(got, ref, R * W);
    expect(err <= 1e-5, "qdc_residual_rmsnorm split output (hi + lo) vs double", err, 1e-5);

    /* 4. SwiGLU on the packed fp32 gate||up rows */
    float *gu = malloc(sizeof(float) * T * 2 * I);
    for (int i = 0; i < T * 2 * I; ++i) gu[i] = uniform() * 4.0f;
    void *dgu = dev_alloc(4 * T * 2 * I), *dact = dev_alloc(4 * T * I);
    HIP_OK(hipMemcpy(dgu, gu, 4 * T * 2 * I, hipMemcpyHostToDevice));
    expect_status(qdc_swiglu(dact, dgu, (char *)dgu + 4 * I, T, I, 2 * I, 2 * I, I, QDC_F32,
                             QDC_F32, stream),
                  QDC_OK, "qdc_swiglu launch");
    HIP_OK(hipStreamSynchronize(stream));
    float *act = malloc(4 * T * I);
    double *ga = malloc(sizeof(double) * T * I), *ea = malloc(sizeof(double) * T * I);
    HIP_OK(hipMemcpy(act, dact, 4 * T * I, hipMemcpyDeviceToHost));
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < I; ++i) {
            const double g = gu[t * 2 * I + i], u = gu[t * 2 * I + I + i];
            ea[t * I + i] = g / (1.0 + exp(-g)) * u;
            ga[t * I + i] = act[t * I + i];
        }
    err = normwise(ga, ea, T * I);
    expect(err <= 1e-5, "qdc_swiglu fp32 [19, 3584] vs double", err, 1e-5);

    /* 5. embedding gather: bf16 table rows widened to fp32, bit-exact */
    uint16_t *table = malloc(2 * V * W);
    for (int i = 0; i < V * W; ++i) table[i] = to_bf16(uniform() * 0.02f);
    int32_t ids[T];
    for (int t = 0; t < T; ++t) ids[t] = (int32_t)((t * 97 + 13) % V);
    void *dtab = dev_alloc(2 * V * W), *dids = dev_alloc(4 * T), *dg = dev_alloc(4 * T * W);
    HIP_OK(hipMemcpy(dtab, table, 2 * V * W, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dids, ids, 4 * T, hipMemcpyHostToDevice));
    expect_status(qdc_embedding_gather(dg, QDC_F32, dtab, QDC_BF16, dids, T, V, W, NULL, stream),
                  QDC_OK, "qdc_embedding_gather launch");
    HIP_OK(hipStreamSynchronize(stream));
    float *rows = malloc(4 * T * W);
    HIP_OK(hipMemcpy(rows, dg, 4 * T * W, hipMemcpyDeviceToHost));
    exact = 1;
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < W; ++i)
            exact &= f2u(rows[t * W + i]) == (uint32_t)table[ids[t] * W + i] << 16;
    expect(exact, "qdc_embedding_gather bf16 -> fp32 rows, bit-exact", 0.0, 0.0);

    HIP_OK(hipStreamDestroy(stream));
    void *bufs[] = {dx, dm, dwf, dwb, dres, dout, dm32, dgu, dact, dtab, dids, dg};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i) HIP_OK(hipFree(bufs[i]));
    free(x); free(wf); free(mb); free(wb); free(xd); free(wd); free(ref); free(got);
    free(of); free(res); free(ob); free(sum); free(m32); free(split); free(gu); free(act);
    free(ga); free(ea); free(table); free(rows);
}

int main(int argc, char **argv) {
    host_checks();
    if (!(argc > 1 && strcmp(argv[1], "--host-only") == 0)) gpu_checks();
    if (failures) {
        printf("%d check(s) failed\n", failures);
        return 1;
    }
    printf("all checks passed\n");
    return 0;
}
