/* A plain-C consumer of libingot_rocm through include/ingot_rocm.h only: the
 * calls a cgo binding makes (session, one-time weight upload, enqueue, sync,
 * copies, error text), checked against double-precision references computed
 * here. Exit status 0 when every check passes.
 *
 *  1. The reference's own CPU-runnable Gemm case: Y = ReLU(A·Bᵀ + bias),
 *     A [128, 256] ~U(-1, 1), B [512, 256] ~U(-1, 1) (transB = 1),
 *     bias [512] ~U(-0.1, 0.1), f32 weights and f32 math, within
 *     1e-3·sqrt(K)·max|A|·max|B| (and ReLU exact at zero).
 *  2. MatMulInteger, u8 A [33, 200] with zero point 128 against s8 B [200, 70]:
 *     int32 results equal to Σ (a − 128)·b exactly.
 *  3. The decode GEMV entry point, ingot_rocm_gemv_bf16, at M = 1 and M = 9
 *     (x [M, 2048] ~U(-1, 1) against a weight [512, 2048] ~U(-0.05, 0.05)
 *     packed as bf16 by the library): within 1e-3·sqrt(K)·max|x|·max|w| of
 *     the double-precision product with the bf16-rounded weight.
 *  4. An error: a K that does not match the weight returns INGOT_EINVAL and
 *     sets ingot_rocm_last_error. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ingot_rocm.h"

static int failures = 0;

#define CHECK(call)                                                                        \
    do {                                                                                   \
        int rc_ = (call);                                                                  \
        if (rc_ != INGOT_OK) {                                                             \
            fprintf(stderr, "%s:%d: %s -> %d (%s)\n", __FILE__, __LINE__, #call, rc_,     \
                    ingot_rocm_last_error());                                              \
            exit(1);                                                                       \
        }                                                                                  \
    } while (0)

/* splitmix64: a fixed, seedable stream (the same on every host) */
static uint64_t rng_state = 0x243F6A8885A308D3ull;
static uint64_t next_u64(void) {
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static float uniform(float lo, float hi) { return lo + (hi - lo) * (float)((next_u64() >> 40) * (1.0 / 16777216.0)); }

static void* to_device(ingot_rocm_session* s, const void* h, size_t bytes) {
    void* d = NULL;
    CHECK(ingot_rocm_device_alloc(s, bytes, &d));
    CHECK(ingot_rocm_memcpy_h2d(s, d, h, bytes));
    return d;
}

static void gemm_relu_case(ingot_rocm_session* s) {
    enum { M = 128, K = 256, N = 512 };
    float* a = malloc(sizeof(float) * M * K);
    float* b = malloc(sizeof(float) * N * K);
    float* bias = malloc(sizeof(float) * N);
    float* y = malloc(sizeof(float) * M * N);
    for (int i = 0; i < M * K; ++i) a[i] = uniform(-1.f, 1.f);
    for (int i = 0; i < N * K; ++i) b[i] = uniform(-1.f, 1.f);
    for (int i = 0; i < N; ++i) bias[i] = uniform(-0.1f, 0.1f);

    ingot_rocm_weight* w = NULL;
    CHECK(ingot_rocm_weight_upload(s, INGOT_DT_F32, INGOT_DT_F32, N, K, K, 1, b, &w));
    void* d_a = to_device(s, a, sizeof(float) * M * K);
    void* d_bias = to_device(s, bias, sizeof(float) * N);
    void* d_y = NULL;
    CHECK(ingot_rocm_device_alloc(s, sizeof(float) * M * N, &d_y));

    ingot_rocm_gemm_args g;
    memset(&g, 0, sizeof g);
    g.M = M;
    g.N = N;
    g.K = K;
    g.d_a = d_a;
    g.a_dtype = INGOT_DT_F32;
    g.lda = K;
    g.w = w;
    g.alpha = 1.f;
    g.beta = 1.f;
    g.d_c = (const float*)d_bias;
    g.c_mode = INGOT_C_ROW;
    g.math = INGOT_MATH_F32;
    g.act = INGOT_ACT_RELU;
    g.d_y = (float*)d_y;
    g.ldy = N;
    g.batch = 1;
    CHECK(ingot_rocm_gemm(s, &g));
    CHECK(ingot_rocm_sync(s));
    CHECK(ingot_rocm_memcpy_d2h(s, y, d_y, sizeof(float) * M * N));

    const double tol = 1e-3 * sqrt((double)K);  /* max|A| and max|B| are <= 1 */
    double worst = 0.0;
    int relu_bad = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = bias[n];
            for (int k = 0; k < K; ++k) acc += (double)a[m * K + k] * (double)b[n * K + k];
            const double want = acc > 0.0 ? acc : 0.0;
            const double err = fabs((double)y[m * N + n] - want);
            if (err > worst) worst = err;
            if (want == 0.0 && y[m * N + n] != 0.f) ++relu_bad;
        }
    if (worst > tol || relu_bad) {
        fprintf(stderr, "gemm+relu: max-abs error %.3e (tol %.3e), %d non-zero outputs where ReLU gives 0\n", worst,
                tol, relu_bad);
        ++failures;
    } else {
        printf("gemm+relu 128x256->512: max-abs error %.3e (tol %.3e)\n", worst, tol);
    }
    CHECK(ingot_rocm_weight_free(s, w));
    CHECK(ingot_rocm_device_free(s, d_a));
    CHECK(ingot_rocm_device_free(s, d_bias));
    CHECK(ingot_rocm_device_free(s, d_y));
    free(a), free(b), free(bias), free(y);
}

static void matmul_integer_case(ingot_rocm_session* s) {
    enum { M = 33, K = 200, N = 70 };
    const int32_t za = 128;
    uint8_t* a = malloc(M * K);
    int8_t* b = malloc(K * N);
    int32_t* y = malloc(sizeof(int32_t) * M * N);
    for (int i = 0; i < M * K; ++i) a[i] = (uint8_t)(next_u64() >> 56);
    for (int i = 0; i < K * N; ++i) b[i] = (int8_t)((int)(next_u64() % 255) - 127);

    ingot_rocm_weight* w = NULL;
    CHECK(ingot_rocm_weight_upload(s, INGOT_DT_I8, INGOT_DT_I8, K, N, N, 0, b, &w));
    void* d_a = to_device(s, a, M * K);
    void* d_y = NULL;
    CHECK(ingot_rocm_device_alloc(s, sizeof(int32_t) * M * N, &d_y));
    CHECK(ingot_rocm_matmul_integer(s, M, N, K, d_a, INGOT_DT_U8, K, za, w, (int32_t*)d_y, NULL, 1, 0, NULL));
    CHECK(ingot_rocm_sync(s));
    CHECK(ingot_rocm_memcpy_d2h(s, y, d_y, sizeof(int32_t) * M * N));
    int bad = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            int64_t acc = 0;
            for (int k = 0; k < K; ++k) acc += (int64_t)((int32_t)a[m * K + k] - za) * (int64_t)b[k * N + n];
            if ((int64_t)y[m * N + n] != acc) ++bad;
        }
    if (bad) {
        fprintf(stderr, "matmul_integer: %d of %d outputs differ from the exact sums\n", bad, M * N);
        ++failures;
    } else {
        printf("matmul_integer u8 33x200x70: bit-exact\n");
    }
    CHECK(ingot_rocm_weight_free(s, w));
    CHECK(ingot_rocm_device_free(s, d_a));
    CHECK(ingot_rocm_device_free(s, d_y));
    free(a), free(b), free(y);
}

/* float32 → bfloat16 → float32, round to nearest even (finite inputs) */
static double bf16_round(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    b = ((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16) << 16;
    memcpy(&f, &b, 4);
    return (double)f;
}

static void gemv_case(ingot_rocm_session* s, int m_rows) {
    enum { K = 2048, N = 512 };
    float* x = malloc(sizeof(float) * m_rows * K);
    float* w = malloc(sizeof(float) * N * K);
    float* y = malloc(sizeof(float) * m_rows * N);
    for (int i = 0; i < m_rows * K; ++i) x[i] = uniform(-1.f, 1.f);
    for (int i = 0; i < N * K; ++i) w[i] = uniform(-0.05f, 0.05f);

    ingot_rocm_weight* wh = NULL;
    CHECK(ingot_rocm_weight_upload(s, INGOT_DT_F32, INGOT_DT_BF16, N, K, K, 1, w, &wh));
    void* d_x = to_device(s, x, sizeof(float) * m_rows * K);
    void* d_y = NULL;
    CHECK(ingot_rocm_device_alloc(s, sizeof(float) * m_rows * N, &d_y));
    ingot_rocm_gemm_args g;
    memset(&g, 0, sizeof g);
    g.M = m_rows;
    g.N = N;
    g.K = K;
    g.d_a = d_x;
    g.a_dtype = INGOT_DT_F32;
    g.lda = K;
    g.w = wh;
    g.alpha = 1.f;
    g.d_y = (float*)d_y;
    g.ldy = N;
    g.batch = 1;
    CHECK(ingot_rocm_gemv_bf16(s, &g));
    CHECK(ingot_rocm_sync(s));
    CHECK(ingot_rocm_memcpy_d2h(s, y, d_y, sizeof(float) * m_rows * N));

    const double tol = 1e-3 * sqrt((double)K) * 0.05;  /* max|x| <= 1, max|w| <= 0.05 */
    double worst = 0.0;
    for (int m = 0; m < m_rows; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)x[m * K + k] * bf16_round(w[n * K + k]);
            const double err = fabs((double)y[m * N + n] - acc);
            if (err > worst) worst = err;
        }
    if (worst > tol) {
        fprintf(stderr, "gemv_bf16 M=%d: max-abs error %.3e (tol %.3e)\n", m_rows, worst, tol);
        ++failures;
    } else {
        printf("gemv_bf16 M=%d 2048->512: max-abs error %.3e (tol %.3e)\n", m_rows, worst, tol);
    }
    CHECK(ingot_rocm_weight_free(s, wh));
    CHECK(ingot_rocm_device_free(s, d_x));
    CHECK(ingot_rocm_device_free(s, d_y));
    free(x), free(w), free(y);
}

static void error_case(ingot_rocm_session* s) {
    float b[4 * 3] = {0};
    ingot_rocm_weight* w = NULL;
    CHECK(ingot_rocm_weight_upload(s, INGOT_DT_F32, INGOT_DT_F32, 4, 3, 3, 1, b, &w));
    void* d = NULL;
    CHECK(ingot_rocm_device_alloc(s, 64, &d));
    ingot_rocm_gemm_args g;
    memset(&g, 0, sizeof g);
    g.M = 1;
    g.N = 4;
    g.K = 5; /* the weight has K = 3 */
    g.d_a = d;
    g.a_dtype = INGOT_DT_F32;
    g.lda = 5;
    g.w = w;
    g.alpha = 1.f;
    g.d_y = (float*)d;
    g.ldy = 4;
    g.batch = 1;
    const int rc = ingot_rocm_gemm(s, &g);
    const char* msg = ingot_rocm_last_error();
    if (rc != INGOT_EINVAL || !msg || !*msg) {
        fprintf(stderr, "mismatched K: status %d, message '%s' (want INGOT_EINVAL and a message)\n", rc,
                msg ? msg : "(null)");
        ++failures;
    } else {
        printf("mismatched K: INGOT_EINVAL, \"%s\"\n", msg);
    }
    CHECK(ingot_rocm_weight_free(s, w));
    CHECK(ingot_rocm_device_free(s, d));
}

int main(void) {
    ingot_rocm_session* s = NULL;
    CHECK(ingot_rocm_open(0, &s));
    gemm_relu_case(s);
    matmul_integer_case(s);
    gemv_case(s, 1);
    gemv_case(s, 9);
    error_case(s);
    CHECK(ingot_rocm_close(s));
    if (failures) {
        fprintf(stderr, "c-abi consumer: %d check(s) failed\n", failures);
        return 1;
    }
    printf("c-abi consumer ok\n");
    return 0;
}
