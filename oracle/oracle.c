/*
 * oracle.c — CPU restatement of ingot's dense-contraction hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the GPU kernels,
 * never part of the product.
 *
 * Pinning (tests/test_oracle.py): the reference's known-answer tests
 * (TestGemmTransB ops/compute_optest_test.go:232-252, TestMatMulBatched
 * :254-274, TestDequantizeLinear ops/quant_optest_test.go:60-73,
 * TestQLinearMatMulAndMatMulInteger :194-223), closed forms (RNE bit
 * patterns of F32ToBF16, erf/tanh identities, exact small-integer products)
 * and independent implementations (numpy float64 matmul, brute-force int64).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* F32ToBF16 (kernels/gemm/bgemm.go:20-26): RNE, NaN kept quiet. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

/* BF16ToF32 (kernels/gemm/bgemm.go:28-29). */
float orc_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

void orc_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_bf16(x[i]);
}

/* expScalar's clamp (kernels/vek/scalar.go:7-13). */
static double exp_clamped(double x) {
    const double lo = -87.33654, hi = 88.37626;
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return exp(x);
}

static double clamp01(double x) { return x < 0 ? 0 : (x > 1 ? 1 : x); }

/* Activations of the epilogue set: ops/epilogue.go:48-73 with the generics
 * of kernels/vek/vek_generic.go:48-76 (relu, hardswish, hardsigmoid, clip,
 * leakyrelu), :121-125 (sigmoid), :150-155 (silu), :165-170 (gelu erf) and
 * geluTanh (ops/elementwise.go:411-414). */
double orc_act(double x, int act, double a, double b) {
    switch (act) {
        case ORC_ACT_RELU: return x > 0 ? x : 0;
        case ORC_ACT_GELU_ERF: return 0.5 * x * (1 + erf(x / sqrt(2.0)));
        case ORC_ACT_GELU_TANH: return 0.5 * x * (1 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
        case ORC_ACT_SIGMOID: return 1 / (1 + exp_clamped(-x));
        case ORC_ACT_SILU: return x / (1 + exp_clamped(-x));
        case ORC_ACT_HARDSWISH: return x * clamp01(x / 6 + 0.5);
        case ORC_ACT_HARDSIGMOID: return clamp01(a * x + b);
        case ORC_ACT_CLIP: return x < a ? a : (x > b ? b : x);
        case ORC_ACT_LEAKYRELU: return x < 0 ? x * a : x;
        default: return x;
    }
}

/* Ref (kernels/gemm/ref.go:4-18): f32 accumulation in k order. */
void orc_gemm_ref_f32(int64_t m, int64_t n, int64_t k, float alpha, const float* a, int64_t lda, const float* b,
                      int64_t ldb, float beta, float* c, int64_t ldc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float acc = 0;
            for (int64_t p = 0; p < k; ++p) acc += a[i * lda + p] * b[p * ldb + j];
            if (beta == 0) c[i * ldc + j] = alpha * acc;
            else c[i * ldc + j] = alpha * acc + beta * c[i * ldc + j];
        }
}

/* The Gemm op (ops/matmul.go:27-139) in float64: Y = post_scale·act(
 * alpha·op(A)·op(B) + beta·C) + post_shift, C broadcast by the rules of
 * ops/matmul.go:50-76, B f32 or bf16 bits (widened exactly). The float64
 * accumulation is the oracle form of kernels/gemm/gemm_test.go:19-31. */
int orc_gemm(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, int transA, const void* B, int b_dtype,
             int64_t ldb, int transB, float alpha, float beta, const float* C, int c_mode, int64_t ldc, int act,
             float act_alpha, float act_beta, int post, float post_scale, float post_shift, double* Y) {
    if (b_dtype != ORC_F32 && b_dtype != ORC_BF16) return 1;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double acc = 0;
            for (int64_t p = 0; p < K; ++p) {
                const double av = transA ? A[p * lda + i] : A[i * lda + p];
                const int64_t bi = transB ? j * ldb + p : p * ldb + j;
                const double bv = b_dtype == ORC_F32 ? ((const float*)B)[bi] : orc_bf16_to_f32(((const uint16_t*)B)[bi]);
                acc += av * bv;
            }
            double v = (double)alpha * acc;
            if (C && beta != 0) {
                double c = 0;
                switch (c_mode) {
                    case ORC_C_FULL: c = C[i * ldc + j]; break;
                    case ORC_C_ROW: c = C[j]; break;
                    case ORC_C_COL: c = C[i]; break;
                    case ORC_C_SCALAR: c = C[0]; break;
                    default: break;
                }
                v += (double)beta * c;
            }
            v = orc_act(v, act, act_alpha, act_beta);
            if (post) v = v * post_scale + post_shift;
            Y[i * N + j] = v;
        }
    return 0;
}

/* vek.DotBF16 generic form (kernels/vek/vek_generic.go:183-190): sequential f32. */
float orc_dot_bf16(const float* a, const uint16_t* b, int64_t n) {
    float s = 0;
    for (int64_t i = 0; i < n; ++i) s += a[i] * orc_bf16_to_f32(b[i]);
    return s;
}

/* GemvBF16 (kernels/gemm/bgemm.go:201-206): y[j] = DotBF16(x, W[j]). */
void orc_gemv_bf16(int64_t n, int64_t k, const float* x, const uint16_t* w, int64_t ldw, float* y) {
    for (int64_t j = 0; j < n; ++j) y[j] = orc_dot_bf16(x, w + j * ldw, k);
}

/* QgemmRef (kernels/gemm/qgemm.go:173-183): u8 × s8 → exact int32. */
void orc_qgemm_ref(int64_t m, int64_t n, int64_t k, const uint8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                   int32_t* c, int64_t ldc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            uint32_t s = 0;
            for (int64_t p = 0; p < k; ++p) s += (uint32_t)((int32_t)a[i * lda + p] * (int32_t)b[p * ldb + j]);
            c[i * ldc + j] = (int32_t)s;
        }
}

static int32_t a_at(const void* A, int a_dtype, int64_t i) {
    return a_dtype == ORC_U8 ? (int32_t)((const uint8_t*)A)[i] : (int32_t)((const int8_t*)A)[i];
}

/* MatMulInteger semantics, closed form: Y[i,j] = Σ_p (A[i,p] − za)·B[p,j]
 * (the expectation of TestQLinearMatMulAndMatMulInteger,
 * ops/quant_optest_test.go:202-211), int32 wrap-around. */
void orc_matmul_integer(int64_t M, int64_t N, int64_t K, const void* A, int a_dtype, int32_t za, const int8_t* B,
                        int32_t* Y) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            uint32_t s = 0;
            for (int64_t p = 0; p < K; ++p)
                s += (uint32_t)(a_at(A, a_dtype, i * K + p) - za) * (uint32_t)(int32_t)B[p * N + j];
            Y[i * N + j] = (int32_t)s;
        }
}

/* The reference's route (ops/quant.go:308-321, 803-829, 868-900): u8 → s8
 * by ^0x80 with za′ = za − 128, the s8 product, then + (−za′)·colSum[j]. */
void orc_matmul_integer_shifted(int64_t M, int64_t N, int64_t K, const void* A, int a_dtype, int32_t za,
                                const int8_t* B, int32_t* Y) {
    const int u8 = a_dtype == ORC_U8;
    const int32_t zs = u8 ? za - 128 : za;
    for (int64_t j = 0; j < N; ++j) {
        uint32_t cs = 0;
        for (int64_t p = 0; p < K; ++p) cs += (uint32_t)(int32_t)B[p * N + j];
        const uint32_t corr = (uint32_t)(-zs) * cs;
        for (int64_t i = 0; i < M; ++i) {
            uint32_t s = 0;
            for (int64_t p = 0; p < K; ++p) {
                int32_t av = u8 ? (int32_t)(int8_t)(((const uint8_t*)A)[i * K + p] ^ 0x80) : a_at(A, a_dtype, i * K + p);
                s += (uint32_t)(av * (int32_t)B[p * N + j]);
            }
            Y[i * N + j] = (int32_t)(s + corr);
        }
    }
}

/* satU8 / satI8 (ops/quant.go:26-46) after the requant expression of
 * qmatmulOp.Run (ops/quant.go:911-925). volatile keeps the product and the
 * sum separately rounded to f32 whatever the contraction settings. */
float orc_qlinear_mult(float sa, float sb, float sy) {
    volatile float ab = sa * sb;
    volatile float m = ab / sy;
    return m;
}

void orc_qlinear_requant(int64_t n, const int32_t* v, float mult, int32_t zy, int u8, void* y) {
    const float fz = (float)zy;
    for (int64_t i = 0; i < n; ++i) {
        volatile float t = (float)v[i] * mult;
        volatile float u = t + fz;
        const double r = nearbyint((double)u); /* default rounding mode: half to even */
        if (u8) {
            ((uint8_t*)y)[i] = r <= 0 ? 0 : (r >= 255 ? 255 : (uint8_t)r);
        } else {
            ((int8_t*)y)[i] = r <= -128 ? -128 : (r >= 127 ? 127 : (int8_t)r);
        }
    }
}

void orc_quantize_i8g(int64_t n, int64_t k, const float* w, int64_t ldw, int8_t* q, float* s) {
    const int64_t gk = k / 64;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t g = 0; g < gk; ++g) {
            float amax = 0.f;
            for (int64_t c = g * 64; c < (g + 1) * 64; ++c) amax = fmaxf(amax, fabsf(w[r * ldw + c]));
            volatile float sc = amax / 127.f;
            s[r * gk + g] = sc;
            for (int64_t c = g * 64; c < (g + 1) * 64; ++c) {
                int v = 0;
                if (sc != 0.f) {
                    volatile float d = w[r * ldw + c] / sc;
                    const double rr = nearbyint((double)d);
                    v = rr < -127 ? -127 : (rr > 127 ? 127 : (int)rr);
                }
                q[r * k + c] = (int8_t)v;
            }
        }
}

void orc_quantize_x16(int64_t k, const float* x, int8_t* xh, int8_t* xl, float* sx) {
    const float x16max = 127.f * 128.f;
    for (int64_t g = 0; g < k / 64; ++g) {
        float amax = 0.f;
        for (int64_t i = g * 64; i < (g + 1) * 64; ++i) amax = fmaxf(amax, fabsf(x[i]));
        volatile float sc = amax / x16max;
        sx[g] = sc;
        if (sc == 0.f) {
            memset(xh + g * 64, 0, 64);
            memset(xl + g * 64, 0, 64);
            continue;
        }
        volatile float inv = 1.f / sc;
        for (int64_t i = g * 64; i < (g + 1) * 64; ++i) {
            volatile float prod = x[i] * inv;
            double rr = nearbyint((double)prod);
            int32_t qv = rr < -16256 ? -16256 : (rr > 16256 ? 16256 : (int32_t)rr);
            const int32_t h = (qv + 64) >> 7;
            xh[i] = (int8_t)h;
            xl[i] = (int8_t)(qv - h * 128);
        }
    }
}

float orc_dot_q8(int64_t k, const int8_t* w, const int8_t* xh, const int8_t* xl, const float* sx, const float* sw) {
    volatile float acc = 0.f;
    for (int64_t g = 0; g < k / 64; ++g) {
        int32_t p = 0;
        for (int64_t i = g * 64; i < (g + 1) * 64; ++i) p += (int32_t)w[i] * (128 * (int32_t)xh[i] + (int32_t)xl[i]);
        volatile float st = sx[g] * sw[g];
        volatile float t = st * (float)p;
        acc = acc + t;
    }
    return acc;
}

void orc_gemv_i8g(int64_t M, int64_t N, int64_t K, const float* x, int64_t ldx, const int8_t* q, const float* s,
                  float alpha, float beta, const float* c, float* y) {
    const int64_t gk = K / 64;
    int8_t* xh = (int8_t*)malloc((size_t)K);
    int8_t* xl = (int8_t*)malloc((size_t)K);
    float* sx = (float*)malloc(sizeof(float) * (size_t)(gk ? gk : 1));
    for (int64_t m = 0; m < M; ++m) {
        orc_quantize_x16(K, x + m * ldx, xh, xl, sx);
        for (int64_t j = 0; j < N; ++j) {
            volatile float v = alpha * orc_dot_q8(K, q + j * K, xh, xl, sx, s + j * gk);
            if (beta != 0.f && c) {
                volatile float bc = beta * c[m * N + j];
                v = v + bc;
            }
            y[m * N + j] = v;
        }
    }
    free(xh);
    free(xl);
    free(sx);
}

static int32_t int_at(const void* p, int dt, int64_t i) {
    switch (dt) {
        case ORC_U8: return ((const uint8_t*)p)[i];
        case ORC_I8: return ((const int8_t*)p)[i];
        case ORC_I32: return ((const int32_t*)p)[i];
    }
    return 0;
}

/* DequantizeLinear (ops/quant.go:173-229): y = float32(x − z)·scale[c],
 * c = (i / inner) % n_scale; per-tensor uses zp[0]. Two f32 roundings, so
 * this is bit-exact to the reference. */
void orc_dequantize_linear(const void* x, int x_dtype, int64_t n, const float* scale, int64_t n_scale, int64_t inner,
                           const void* zp, int zp_dtype, int64_t n_zp, float* y) {
    for (int64_t i = 0; i < n; ++i) {
        const int64_t c = n_scale == 1 ? 0 : (i / inner) % n_scale;
        int32_t z = 0;
        if (zp) z = int_at(zp, zp_dtype, n_zp > 1 ? c : 0);
        const int32_t d = (int32_t)((uint32_t)int_at(x, x_dtype, i) - (uint32_t)z);
        y[i] = (float)d * scale[c];
    }
}

/* convOut (ops/conv.go:110-113). */
static int64_t conv_out(int64_t in, int64_t k, int64_t stride, int64_t dil, int64_t pa, int64_t pb) {
    const int64_t eff = dil * (k - 1) + 1;
    return (in + pa + pb - eff) / stride + 1;
}

int64_t orc_qlinear_conv(const int64_t* geom, const void* x, int x_dtype, int32_t zx, const int8_t* w,
                         const int32_t* bias, const float* mult, int32_t zy, int y_u8, void* y) {
    const int64_t N = geom[0], C = geom[1], H = geom[2], W = geom[3], M = geom[4], KH = geom[5], KW = geom[6];
    const int64_t G = geom[7], sh = geom[8], sw = geom[9], dh = geom[10], dw = geom[11];
    const int64_t pt = geom[12], pl = geom[13], pb = geom[14], pr = geom[15];
    if (G < 1 || C % G != 0 || M % G != 0 || sh < 1 || sw < 1 || dh < 1 || dw < 1) return -1;
    const int64_t OH = conv_out(H, KH, sh, dh, pt, pb), OW = conv_out(W, KW, sw, dw, pl, pr);
    if (OH < 0 || OW < 0) return -1;
    const int64_t Cg = C / G, Mg = M / G, K = Cg * KH * KW, P = OH * OW;
    /* shiftToS8: u8 x -> x ^ 0x80 (= x - 128), zx' = zx - 128 */
    const int u8 = x_dtype == ORC_U8;
    const int32_t zs = u8 ? zx - 128 : zx;
    const int8_t pv = (int8_t)zs;
    int8_t* col = (int8_t*)malloc((size_t)(K > 0 ? K : 1));
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(P > 0 ? P : 1) * (size_t)(Mg > 0 ? Mg : 1));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < G; ++g) {
            for (int64_t i = 0; i < P * Mg; ++i) acc[i] = 0;
            for (int64_t p = 0; p < P; ++p) {
                const int64_t oh = p / OW, ow = p % OW;
                /* qim2colRows: k = (c, kh, kw), c-major within the group */
                for (int64_t k = 0; k < K; ++k) {
                    const int64_t c = g * Cg + k / (KH * KW), kh = (k / KW) % KH, kw = k % KW;
                    const int64_t ih = oh * sh + kh * dh - pt, iw = ow * sw + kw * dw - pl;
                    int8_t v = pv;
                    if (ih >= 0 && ih < H && iw >= 0 && iw < W) {
                        const int64_t xi = ((n * C + c) * H + ih) * W + iw;
                        v = u8 ? (int8_t)(((const uint8_t*)x)[xi] ^ 0x80) : ((const int8_t*)x)[xi];
                    }
                    col[k] = v;
                }
                for (int64_t mi = 0; mi < Mg; ++mi) {
                    uint32_t s = 0;
                    const int8_t* wr = w + (g * Mg + mi) * K;
                    for (int64_t k = 0; k < K; ++k) s += (uint32_t)((int32_t)wr[k] * (int32_t)col[k]);
                    acc[mi * P + p] = (int32_t)s;
                }
            }
            for (int64_t mi = 0; mi < Mg; ++mi) {
                const int64_t m = g * Mg + mi;
                uint32_t sumw = 0;
                for (int64_t k = 0; k < K; ++k) sumw += (uint32_t)(int32_t)w[m * K + k];
                uint32_t corr = (uint32_t)(-zs) * sumw;
                if (bias) corr += (uint32_t)bias[m];
                int32_t* v = acc + mi * P;
                for (int64_t p = 0; p < P; ++p) v[p] = (int32_t)((uint32_t)v[p] + corr);
                void* dst = (char*)y + (n * M + m) * P;
                orc_qlinear_requant(P, v, mult[m], zy, y_u8, dst);
            }
        }
    free(col);
    free(acc);
    return P;
}
