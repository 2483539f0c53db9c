/*
 * oracle.h — CPU restatement of ingot's dense-contraction hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker. The
 * product (libingot_rocm.so) never links or calls it.
 *
 * The reference (github.com/giraffesyo/ingot, Go 1.27.3) cannot be built in
 * this image (no Go toolchain), so these functions restate its algorithms in
 * C from the Go sources; each cites the file:line it follows. Floating-point
 * functions accumulate in double (the float64 oracle form of the reference's
 * own tests, kernels/gemm/gemm_test.go:19-31) unless they restate an f32
 * routine bit for bit (orc_gemm_ref_f32, orc_dot_bf16, orc_dequantize_linear,
 * orc_f32_to_bf16); integer functions are exact with int32 wrap-around.
 */
#ifndef INGOT_ORACLE_H
#define INGOT_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: tensor/dtype.go:12-23 */
#define ORC_F32 1
#define ORC_BF16 3
#define ORC_I8 4
#define ORC_U8 5
#define ORC_I32 7

/* activation codes (same values as INGOT_ACT_* in include/ingot_rocm.h) */
#define ORC_ACT_NONE 0
#define ORC_ACT_RELU 1
#define ORC_ACT_GELU_ERF 2
#define ORC_ACT_GELU_TANH 3
#define ORC_ACT_SIGMOID 4
#define ORC_ACT_SILU 5
#define ORC_ACT_HARDSWISH 6
#define ORC_ACT_HARDSIGMOID 7
#define ORC_ACT_CLIP 8
#define ORC_ACT_LEAKYRELU 9

/* C broadcast modes (INGOT_C_*) */
#define ORC_C_NONE 0
#define ORC_C_FULL 1
#define ORC_C_ROW 2
#define ORC_C_COL 3
#define ORC_C_SCALAR 4

uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n);

double orc_act(double x, int act, double a, double b);

void orc_gemm_ref_f32(int64_t m, int64_t n, int64_t k, float alpha, const float* a, int64_t lda, const float* b,
                      int64_t ldb, float beta, float* c, int64_t ldc);

int orc_gemm(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, int transA, const void* B, int b_dtype,
             int64_t ldb, int transB, float alpha, float beta, const float* C, int c_mode, int64_t ldc, int act,
             float act_alpha, float act_beta, int post, float post_scale, float post_shift, double* Y);

float orc_dot_bf16(const float* a, const uint16_t* b, int64_t n);
void orc_gemv_bf16(int64_t n, int64_t k, const float* x, const uint16_t* w, int64_t ldw, float* y);

void orc_qgemm_ref(int64_t m, int64_t n, int64_t k, const uint8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                   int32_t* c, int64_t ldc);
void orc_matmul_integer(int64_t M, int64_t N, int64_t K, const void* A, int a_dtype, int32_t za, const int8_t* B,
                        int32_t* Y);
void orc_matmul_integer_shifted(int64_t M, int64_t N, int64_t K, const void* A, int a_dtype, int32_t za,
                                const int8_t* B, int32_t* Y);

/* QLinearMatMul requantisation (ops/quant.go:902-928): for each int32
 * product v (already zero-point corrected),
 *   y = sat(RoundToEven(fl32(fl32(float32(v)·mult) + zy))),
 * mult = fl32(fl32(sa·sb)/sy) (orc_qlinear_mult), sat to [0,255] (u8 = 1) or
 * [-128,127]. The multiply and the add are rounded separately (the
 * reference's float32 expression as compiled for amd64). Bit-exact. */
float orc_qlinear_mult(float sa, float sb, float sy);
void orc_qlinear_requant(int64_t n, const int32_t* v, float mult, int32_t zy, int u8, void* y);
/* Grouped int8 decode GEMV (ingot_weight_quant="int8"), group = 64 k:
 * orc_quantize_i8g : quantizeI8G (kernels/gemm/i8g.go:33-56) of an [n][k]
 *   f32 weight: s = max|w|/127 per row-group, q = clamp(RoundToEven(w/s), ±127).
 * orc_quantize_x16 : vek.QuantizeX16 (kernels/vek/scalar.go:38-60):
 *   s = max|x|/16256, q = clamp(RoundToEven(x·(1/s)), ±16256),
 *   xh = (q + 64) >> 7, xl = q − 128·xh.
 * orc_dot_q8       : dotQ8Ref (kernels/vek/scalar.go:20-32): exact int32
 *   group sums, acc += (sx·sw)·float32(p) in group order.
 * orc_gemv_i8g     : GemvI8G (kernels/gemm/i8g.go:70-86) per row of x:
 *   y = alpha·dot (+ beta·c when beta != 0), c = the broadcast C [M][N].
 * Each f32 operation is rounded on its own (no contraction). Bit-exact. */
void orc_quantize_i8g(int64_t n, int64_t k, const float* w, int64_t ldw, int8_t* q, float* s);
void orc_quantize_x16(int64_t k, const float* x, int8_t* xh, int8_t* xl, float* sx);
float orc_dot_q8(int64_t k, const int8_t* w, const int8_t* xh, const int8_t* xl, const float* sx, const float* sw);
void orc_gemv_i8g(int64_t M, int64_t N, int64_t K, const float* x, int64_t ldx, const int8_t* q, const float* s,
                  float alpha, float beta, const float* c, float* y);
void orc_dequantize_linear(const void* x, int x_dtype, int64_t n, const float* scale, int64_t n_scale, int64_t inner,
                           const void* zp, int zp_dtype, int64_t n_zp, float* y);
/* QLinearConv (ops/quant.go:343-420, qconvRun.corr/requant :441-468, the
 * im2col path :642-706) along the reference's own route: x shifted to s8
 * (u8: x ^ 0x80, zx' = zx - 128, shiftToS8 :308-321), taps outside the image
 * read pv = int8(zx') (:657, :676-690), acc = sum_k w[m][k]·col[k][p] with
 * int32 wrap-around, corr(m) = -zx'·sumW[m] + bias[m] (:441-447), then
 *   y = sat(RoundToEven(fl32(fl32(float32(acc + corr)·mult[m]) + zy)))
 * (vek.RequantU8/I8, kernels/vek/quant_amd64.go:52-70). geom holds
 * N, C, H, W, M, KH, KW, group, stride_h, stride_w, dil_h, dil_w and the
 * resolved pads top, left, bottom, right; w is [M][C/group][KH][KW], bias may
 * be NULL, y is [N][M][OH][OW] with OH/OW from convOut (ops/conv.go:110-113).
 * Returns OH·OW, or -1 for an invalid geometry. Bit-exact. */
int64_t orc_qlinear_conv(const int64_t* geom, const void* x, int x_dtype, int32_t zx, const int8_t* w,
                         const int32_t* bias, const float* mult, int32_t zy, int y_u8, void* y);

#ifdef __cplusplus
}
#endif
#endif
