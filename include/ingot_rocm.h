/*
 * ingot_rocm.h — C ABI of libingot_rocm.so, the MI355X (gfx950) backend for
 * ingot's dense-contraction hot path: ONNX Gemm / MatMul with fused
 * bias+activation epilogues, bf16-weight GEMM and decode GEMV, and int8
 * MatMulInteger + DequantizeLinear.
 *
 * Two layers are exported.
 *
 *  1. Kernel layer (ingot_rocm_gemm, ingot_rocm_gemm_dynamic_b, ingot_rocm_gemv_bf16,
 *     ingot_rocm_matmul_integer, ingot_rocm_dequantize_linear, ...). Plain
 *     device pointers and sizes. This is what a Go `rocm` backend binds with
 *     cgo, one call per gpuOp.prepare encoding
 *     (reference: graph/gpuops_darwin_arm64.go:14-22, the Metal encoder calls
 *     e.Gemm / e.GemmEp / gemv_bf16 at graph/gpuops_darwin_arm64.go:509-576,
 *     kernels/metal/gemm.go:78, kernels/metal/gemmep.go:68,
 *     kernels/metal/decode.go:65).
 *
 *  2. Operator layer (ingot_rocm_op_create / ingot_rocm_op_run). ONNX-semantics
 *     ops over device tensors with the reference's op.Op contract: validate,
 *     allocate outputs from the session pool, dispatch
 *     (reference: ops/op.go:106-111 Op.Run, ops/op.go:143 Lookup,
 *     ops/matmul.go:454-472, ops/quant.go:941-949).
 *
 * Conventions (reference ownership rules: ops/op.go:50-60, graph/session.go:14-22):
 *  - Every function returns INGOT_OK (0) or a non-zero status; the message of
 *    the last failure on the calling thread is ingot_rocm_last_error(). The
 *    Go side wraps it with NodeInfo.Errorf (ops/op.go:179-181).
 *  - INGOT_EDECLINED is the gpuOp.prepare "ok=false" answer: the inputs are
 *    valid for the op but this backend does not run them; the caller runs the
 *    CPU op (graph/gpu_darwin_arm64.go:474-498). Nothing was allocated.
 *  - Pointers named d_* are device pointers (from ingot_rocm_device_alloc or
 *    any hipMalloc'd memory of the session's device). Compute calls are
 *    enqueued on the session's single HIP stream and return without waiting;
 *    ingot_rocm_sync waits. Calls on one session must be serialized by the
 *    caller (GPUSession.runMu, graph/gpu_darwin_arm64.go:308).
 *  - Matrices are dense row-major with an element leading dimension (ld*),
 *    the tensor.Tensor layout (tensor/tensor.go:12).
 */
#ifndef INGOT_ROCM_H
#define INGOT_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define INGOT_OK 0
#define INGOT_EINVAL 1       /* invalid argument, shape or dtype (the CPU op errors too) */
#define INGOT_EDECLINED 2    /* valid, but not run by this backend: use the CPU op */
#define INGOT_EDEVICE 3      /* HIP runtime failure */
#define INGOT_ENOMEM 4       /* device or pinned allocation failed */

/* ---- element types: the numbering of tensor.DType (tensor/dtype.go:12-23) ---- */
#define INGOT_DT_F32 1
#define INGOT_DT_F16 2
#define INGOT_DT_BF16 3
#define INGOT_DT_I8 4
#define INGOT_DT_U8 5
#define INGOT_DT_I16 6
#define INGOT_DT_I32 7
#define INGOT_DT_I64 8
#define INGOT_DT_BOOL 9

/* ---- epilogue activations ----
 * y = post_scale · act(alpha·acc + beta·C) + post_shift.
 * relu..leakyrelu: ops/epilogue.go:22-73 and the kernels/vek generics
 * (kernels/vek/vek_generic.go:48-76,121-125,150-170); gelu_erf: ingot.Gelu /
 * Gelu (ops/elementwise.go:533-539); gelu_tanh: geluTanh
 * (ops/elementwise.go:411-414); the GPU act set (kernels/metal/cnn.go:15-37). */
#define INGOT_ACT_NONE 0
#define INGOT_ACT_RELU 1
#define INGOT_ACT_GELU_ERF 2
#define INGOT_ACT_GELU_TANH 3
#define INGOT_ACT_SIGMOID 4
#define INGOT_ACT_SILU 5
#define INGOT_ACT_HARDSWISH 6
#define INGOT_ACT_HARDSIGMOID 7 /* clamp01(act_alpha·x + act_beta) */
#define INGOT_ACT_CLIP 8        /* min(max(x, act_alpha), act_beta) */
#define INGOT_ACT_LEAKYRELU 9   /* x < 0 ? act_alpha·x : x */

/* ---- Gemm C operand broadcast (ops/matmul.go:50-76) ---- */
#define INGOT_C_NONE 0   /* no C, or beta == 0 */
#define INGOT_C_FULL 1   /* [M,N] (or [N] with M == 1), leading dim ldc */
#define INGOT_C_ROW 2    /* numel N: [N] or [1,N], broadcast over rows (the Linear bias) */
#define INGOT_C_COL 3    /* [M,1]: broadcast over columns */
#define INGOT_C_SCALAR 4 /* numel 1 */

/* ---- math type of a GEMM ---- */
/* Pack type of ingot_rocm_weight_upload beyond the tensor dtypes: int8
 * weights with one f32 scale per 64 consecutive k of a row, for decode GEMV
 * (ingot_weight_quant="int8": gemm.I8GWeights, kernels/gemm/i8g.go:12-56). */
#define INGOT_PACK_I8G 100

#define INGOT_MATH_AUTO 0 /* the weight's packed type: f32 weights → f32 MFMA, bf16 → bf16 MFMA */
#define INGOT_MATH_F32 1
#define INGOT_MATH_BF16 2

typedef struct ingot_rocm_session ingot_rocm_session;
typedef struct ingot_rocm_weight ingot_rocm_weight;
typedef struct ingot_rocm_op ingot_rocm_op;

/* ================= session lifecycle and memory ================= */

/* Opens a session on HIP device `device` with its own stream, device pool and
 * weight table. The ROCm counterpart of CompileGPU's metal.Open + pool set-up
 * (graph/gpu_darwin_arm64.go:96-148). */
int ingot_rocm_open(int device, ingot_rocm_session** out);
/* Waits for queued work, frees every weight, pooled buffer and the stream
 * (GPUSession.Close, graph/gpu_other.go:33). */
int ingot_rocm_close(ingot_rocm_session* s);
/* Message of the calling thread's last failure ("" if none). */
const char* ingot_rocm_last_error(void);
/* Library version string. */
const char* ingot_rocm_version(void);
/* Waits until all work queued on the session's stream has finished; reports
 * any kernel fault (GPU errors surface at Flush: graph/gpu_darwin_arm64.go:319-323). */
int ingot_rocm_sync(ingot_rocm_session* s);
/* The session's hipStream_t, for callers that record their own events. */
int ingot_rocm_stream(ingot_rocm_session* s, void** stream);

int ingot_rocm_device_alloc(ingot_rocm_session* s, size_t bytes, void** d_out);
int ingot_rocm_device_free(ingot_rocm_session* s, void* d_ptr);
/* Pinned host memory, the backing of a tensor.NewPoolAlloc pool
 * (tensor/pool.go:22; Metal's pageMem, graph/gpu_darwin_arm64.go:114-117). */
int ingot_rocm_host_alloc(ingot_rocm_session* s, size_t bytes, void** h_out);
int ingot_rocm_host_free(ingot_rocm_session* s, void* h_ptr);
/* Synchronous copies (return when the data has arrived). */
int ingot_rocm_memcpy_h2d(ingot_rocm_session* s, void* d_dst, const void* h_src, size_t bytes);
int ingot_rocm_memcpy_d2h(ingot_rocm_session* s, void* h_dst, const void* d_src, size_t bytes);
int ingot_rocm_memcpy_d2d(ingot_rocm_session* s, void* d_dst, const void* d_src, size_t bytes);
/* Enqueues a fill of `bytes` bytes with `value` (a kernel, not hipMemset). */
int ingot_rocm_memset(ingot_rocm_session* s, void* d_dst, int value, size_t bytes);

/* GPU timing on the session stream (GPUSession.GPUTime / Profile,
 * graph/gpu_other.go:13-22): timer_start records an event, timer_stop records
 * a second one, waits for it and returns the elapsed milliseconds. */
int ingot_rocm_timer_start(ingot_rocm_session* s);
int ingot_rocm_timer_stop(ingot_rocm_session* s, float* ms);

/* ================= constant weights (pack once) ================= */

/* Uploads a constant weight B and packs it once into the layout the kernels
 * read: [Np][Kp] row-major, K-contiguous (the "NT" / Linear form), zero
 * padded, in `pack_dtype`. Mirrors the reference's one-time packs: bCache
 * (ops/matmul.go:200-236), packedBF16 (ops/matmul.go:270-280), bWeights with
 * column sums (ops/quant.go:803-829) and the GPU's bf16Const
 * (graph/gpuops_darwin_arm64.go:612-629).
 *   src_dtype  : INGOT_DT_F32, INGOT_DT_BF16 (bit patterns) or INGOT_DT_I8.
 *   pack_dtype : INGOT_DT_F32 (from f32), INGOT_DT_BF16 (from f32 by RNE
 *                F32ToBF16, kernels/gemm/bgemm.go:20-26, or from bf16) or
 *                INGOT_DT_I8 (from i8; column sums computed) or
 *                INGOT_PACK_I8G (from f32 or bf16, K a multiple of 64:
 *                quantizeI8G, kernels/gemm/i8g.go:33-56).
 *   trans = 1  : the source is [N,K] (Gemm transB=1, nn.Linear); rows = N, cols = K.
 *   trans = 0  : the source is [K,N] (MatMul, Gemm transB=0); rows = K, cols = N.
 *   ld         : source leading dimension in elements (>= cols).
 * `h_src` is host memory; ingot_rocm_weight_pack_device takes device memory
 * (the per-call pack of a non-constant B). */
int ingot_rocm_weight_upload(ingot_rocm_session* s, int src_dtype, int pack_dtype, int64_t rows, int64_t cols,
                             int64_t ld, int trans, const void* h_src, ingot_rocm_weight** out);
int ingot_rocm_weight_pack_device(ingot_rocm_session* s, int src_dtype, int pack_dtype, int64_t rows, int64_t cols,
                                  int64_t ld, int trans, const void* d_src, ingot_rocm_weight** out);
int ingot_rocm_weight_free(ingot_rocm_session* s, ingot_rocm_weight* w);
/* Logical N, K and the packed dtype of a weight. */
int ingot_rocm_weight_info(const ingot_rocm_weight* w, int64_t* n, int64_t* k, int* pack_dtype);

/* ================= kernel layer ================= */

/* Y[M,N] = post_scale · act(alpha · op(A)·Bᵀ + beta · C) + post_shift
 * The ONNX Gemm (ops/matmul.go:27-139) with the fused epilogue of
 * SgemmPackedBEpi (kernels/gemm/gemm.go:521-597) and the GPU GemmEp
 * (kernels/metal/gemmep.go:68). B is a packed weight (logical [N,K]).
 *   a_dtype : INGOT_DT_F32 or INGOT_DT_BF16 (bf16-resident activations).
 *   trans_a : A is stored [K,M] (Gemm transA=1).
 *   math    : INGOT_MATH_AUTO follows the weight's packed dtype. f32 A with
 *             bf16 weights then runs as two bf16 planes (hi = bf16(a),
 *             lo = bf16(a − hi)), keeping the reference's f32-activation
 *             accuracy (~2⁻¹⁷ relative); ±Inf and NaN in A propagate as in
 *             the f32 dot, and finite A never overflows to Inf in the split.
 *             INGOT_MATH_BF16 rounds A to bf16
 *             once (RNE), the GPUBF16 semantics of graph/device.go:20-30, at
 *             half the MFMA work. The accumulation is always f32.
 *   C       : d_c with c_mode INGOT_C_* and ldc (INGOT_C_FULL only).
 * Routing of bf16 weights with f32 A (no transA, batch 1): M <= 4 runs the
 * decode GEMV of ingot_rocm_gemv_bf16, and so does M = 5..16 when N < 4096;
 * M = 5..16 with N >= 4096 runs the GEMM (four-stage 32x32 tiles), which is
 * faster there. ingot_rocm_gemv_bf16 always runs the GEMV (M <= 16).
 * A row of Y does not depend on M (kernels/gemm/minvariance_test.go:21): every
 * GEMM tile of one weight/math kind sums K in the same order, so rows are
 * bit-identical across M for f32 weights, and for bf16 weights at every M the
 * GEMM serves (above); the GEMV sums in its own order, as the reference's M = 1
 * GEMV does. int8 results are exact. */
typedef struct ingot_rocm_gemm_args {
    int64_t M, N, K;
    const void* d_a;
    int32_t a_dtype;
    int32_t trans_a;
    int64_t lda;
    const ingot_rocm_weight* w;
    float alpha, beta;
    const float* d_c;
    int32_t c_mode;
    int32_t math;
    int64_t ldc;
    int32_t act;
    float act_alpha, act_beta;
    int32_t post; /* apply post_scale/post_shift (ops/epilogue.go:37-41) */
    float post_scale, post_shift;
    float* d_y;
    int64_t ldy;
    int64_t batch;    /* >= 1: strided batch of independent products sharing w */
    int64_t stride_a; /* elements between batch items of A */
    int64_t stride_y; /* elements between batch items of Y */
    int32_t y_dtype;  /* Y element type: INGOT_DT_F32 (or 0) or INGOT_DT_BF16 (RNE store: a
                         bf16-resident activation for the next product, GPUBF16
                         graph/device.go:20-30) */
} ingot_rocm_gemm_args;

int ingot_rocm_gemm(ingot_rocm_session* s, const ingot_rocm_gemm_args* args);

/* ingot_rocm_gemm without any allocation: the same validation, routing and
 * kernels, with the per-call scratch (packed activations, the decode GEMV's x
 * planes, the int8 GEMV's quantised x) in a fixed device array of
 * INGOT_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, instead
 * of the session's growable workspace. No hipMalloc, hipFree or allocating
 * library routine runs in the call. A product needing more scratch fails with
 * INGOT_EINVAL and a message naming the size. No counterpart in the
 * reference: it is for callers that cannot allocate (HIP graph capture, tight
 * serving loops, harnesses that forbid it). The array is shared by every call
 * on that GPU, from any session, and keeps the last call's contents (each call
 * writes every scratch byte it reads). The library orders the calls: a call
 * from one session makes its stream wait for the last no-alloc call another
 * session made on that GPU, so they run in the order the host issued them
 * (calls made at the same moment from several host threads still run one
 * after another, in an order the library picks). A stream under graph capture
 * gets no such wait: the captured graph's replays race on the array with its
 * other users unless the caller orders them. */
#define INGOT_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int ingot_rocm_gemm_noalloc(ingot_rocm_session* s, const ingot_rocm_gemm_args* args);

/* Bytes of device memory the session's growable workspace holds now (0 until
 * a call needs scratch: packed activations, GEMV x planes, int8 A, im2col).
 * No counterpart in the reference: a diagnostic, e.g. to show that
 * ingot_rocm_gemm_noalloc leaves the workspace unused. */
int ingot_rocm_session_workspace(const ingot_rocm_session* s, size_t* bytes);

/* Batched GEMM whose B is an activation: each batch item i multiplies its A
 * (stride_a) by its own B at d_b + i·stride_b elements (stride_b 0: one B for
 * every item), packed on the device per call. B items are [N,K] with row
 * pitch ldb when trans_b (attention Q·Kᵀ), else [K,N] (P·V); b_dtype f32 or
 * bf16. args->w must be NULL; every other field is as for ingot_rocm_gemm
 * (f32 B runs f32 math unless math = INGOT_MATH_BF16). Replaces the
 * per-batch-item loop of matmulOp for a batched right operand
 * (ops/matmul.go:375-403). */
int ingot_rocm_gemm_dynamic_b(ingot_rocm_session* s, const ingot_rocm_gemm_args* args, const void* d_b,
                              int32_t b_dtype, int32_t trans_b, int64_t ldb, int64_t stride_b);

/* Decode GEMV: y[m,n] = alpha·Σ_k x[m,k]·W[n,k] + beta·C (+act) for M <= 16
 * rows of f32 x against a bf16 weight; K is split across the lanes of a wave
 * (M <= 4) or the waves of a workgroup (M > 4) and the partial sums are added
 * in a fixed order, so results are run-to-run identical (reference: gemvBF16 ops/matmul.go:177-190, GemvBF16
 * kernels/gemm/bgemm.go:201-206, Metal gemv_bf16 kernels/metal/decode.go:65).
 * Uses the same argument block as ingot_rocm_gemm (a_dtype f32, trans_a 0,
 * batch 1); fails with INGOT_EINVAL for M > 16 or a non-bf16 weight. */
int ingot_rocm_gemv_bf16(ingot_rocm_session* s, const ingot_rocm_gemm_args* args);

/* MatMulInteger (+ fused DequantizeLinear):
 *   Y_i32[m,n] = Σ_k (A[m,k] − za) · B[k,n]       (exact, int32 wrap-around)
 *   Y_f32[m,n] = float32(Y_i32[m,n] − dq_zp) · dq_scale[n or 0]
 * A is u8 (a_dtype INGOT_DT_U8) or s8 (INGOT_DT_I8), [M,K] with lda; za the
 * per-tensor zero point; B a weight packed as INGOT_DT_I8 (weight zero point
 * 0, s8Weights ops/quant.go:285-302). Reference: qmatmulOp.Run
 * ops/quant.go:831-900 (u8 → s8 by ^0x80 with za−128 and the −za′·colSum
 * correction, :308-321, :890-900), DequantizeLinear ops/quant.go:173-229.
 * Either output may be NULL (not both). n_scale is 1 (per-tensor) or N. */
int ingot_rocm_matmul_integer(ingot_rocm_session* s, int64_t M, int64_t N, int64_t K, const void* d_a,
                              int32_t a_dtype, int64_t lda, int32_t za, const ingot_rocm_weight* w, int32_t* d_y_i32,
                              const float* d_dq_scale, int64_t n_scale, int32_t dq_zp, float* d_y_f32);

/* QLinearMatMul (ops/quant.go:791-928, requant branch): the product of
 * ingot_rocm_matmul_integer requantised on the device,
 *   Y[m,n] = sat(RoundToEven(fl32(fl32(float32(Y_i32[m,n])·mult) + zy))),
 * saturated to [0,255] (y_dtype INGOT_DT_U8, satU8 ops/quant.go:26-35) or
 * [-128,127] (INGOT_DT_I8, satI8 :37-46). mult = fl32(fl32(a_scale·b_scale)
 * / y_scale) is computed by the caller as the reference does (per-tensor
 * scales, :911). The multiply and the add are rounded separately. */
int ingot_rocm_qlinear_matmul(ingot_rocm_session* s, int64_t M, int64_t N, int64_t K, const void* d_a,
                              int32_t a_dtype, int64_t lda, int32_t za, const ingot_rocm_weight* w, float mult,
                              int32_t zy, int32_t y_dtype, void* d_y);

/* QLinearConv, 2-D NCHW (qlinearConvOp.Run, ops/quant.go:343-420; requant
 * qconvRun.corr/requant :441-468):
 *   v[n,m,oh,ow] = Σ_{cg,kh,kw} W[m,cg,kh,kw]·(x[n, g·Cg+cg, ih, iw] − zx) + bias[m]
 *     (ih = oh·stride_h + kh·dilation_h − pad_top, iw likewise; taps outside
 *      the image contribute 0: the reference pads with the zero point)
 *   Y[n,m,oh,ow] = sat(RoundToEven(fl32(fl32(float32(v)·mult[m]) + zy)))
 * int32 wrap-around as the reference's accumulators. W is packed as
 * INGOT_DT_I8 from its [M, C/group·KH·KW] view (rows = M, trans = 1), weight
 * zero point 0 (s8Weights :285-302). x is u8 or s8 with zero point zx in the
 * range of its dtype (else INGOT_EDECLINED); d_mult[m] = fl32(fl32(x_scale·
 * w_scale[m]) / y_scale) (:380-390) is computed by the caller; d_bias may be
 * NULL. Pads are resolved (auto_pad applied, ops/conv.go:115-136); OH and OW
 * follow convOut (ops/conv.go:110-113). Y is [N, M, OH, OW] of y_dtype
 * (INGOT_DT_U8 or INGOT_DT_I8). Large groups run an im2col + int8 MFMA GEMM
 * (the reference's pointwise / im2colTiled paths, :612-673); depthwise and
 * narrow groups a direct kernel (:472-598). */
typedef struct ingot_rocm_qconv_args {
    int64_t n, c, h, w;   /* x [N, C, H, W] */
    int64_t m, kh, kw;    /* weight [M, C/group, KH, KW] */
    int64_t group;
    int64_t stride_h, stride_w, dilation_h, dilation_w;
    int64_t pad_top, pad_left, pad_bottom, pad_right;
    const void* d_x;
    int32_t x_dtype;
    int32_t zx;
    const float* d_mult;    /* [M] */
    const int32_t* d_bias;  /* [M] or NULL */
    int32_t zy;
    int32_t y_dtype;
    void* d_y;
} ingot_rocm_qconv_args;

int ingot_rocm_qlinear_conv(ingot_rocm_session* s, const ingot_rocm_qconv_args* args, const ingot_rocm_weight* w);

/* DequantizeLinear over a dense tensor of n elements (ops/quant.go:173-229):
 *   y[i] = float32(x[i] − zp[c]) · scale[c],  c = (i / inner) % n_scale
 * x_dtype U8, I8 or I32; n_scale 1 = per-tensor (then inner is ignored);
 * d_zp may be NULL (zero), else zp_dtype U8, I8 or I32 with n_zp 1 or n_scale. */
int ingot_rocm_dequantize_linear(ingot_rocm_session* s, const void* d_x, int32_t x_dtype, int64_t n,
                                 const float* d_scale, int64_t n_scale, int64_t inner, const void* d_zp,
                                 int32_t zp_dtype, int64_t n_zp, float* d_y);

/* Elementwise activation / epilogue pass y = post_scale·act(x + bias[j]) + post_shift
 * over rows of width `cols` (bias may be NULL): the standalone Relu / Gelu /
 * ingot.Gelu nodes (ops/elementwise.go:492,533-539) and the MatMul bias /
 * ingot_act tail when no GEMM epilogue absorbed them (ops/matmul.go:417-425). */
int ingot_rocm_activation(ingot_rocm_session* s, const float* d_x, float* d_y, int64_t rows, int64_t cols,
                          const float* d_bias, int32_t act, float act_alpha, float act_beta, int32_t post,
                          float post_scale, float post_shift);

/* f32 → bf16 (RNE, NaN kept quiet: F32ToBF16, kernels/gemm/bgemm.go:20-26)
 * over n elements; the GPU CastBF16 (graph/gpuops_darwin_arm64.go:588). */
int ingot_rocm_cast_bf16(ingot_rocm_session* s, const float* d_x, uint16_t* d_y, int64_t n);

/* ================= operator layer (op.Op mirror) ================= */

/* A tensor handed across the boundary: dense row-major, data on the device. */
typedef struct ingot_rocm_tensor {
    int32_t dtype;
    int32_t rank;
    int64_t dims[8];
    void* data;
} ingot_rocm_tensor;

/* Builds an op like ops.Lookup(domain, op_type, opset)(NodeInfo)
 * (ops/op.go:143-181). `attrs` is "name=value" pairs separated by ';', each
 * name prefixed by its kind: "i:transB=1;f:alpha=0.5;s:ingot_act=gelu".
 * Supported: Gemm@7 (ops/matmul.go:455), MatMul@1 (:465), MatMulInteger@10
 * (ops/quant.go:943), DequantizeLinear@10 (:947), Relu@6, Gelu@20, ingot.Gelu@1
 * (ops/elementwise.go:492,533,539). Unknown ops fail loudly (INGOT_EINVAL). */
int ingot_rocm_op_create(ingot_rocm_session* s, const char* domain, const char* op_type, int opset,
                         const char* attrs, ingot_rocm_op** out);
/* Op.Run: inputs (NULL data = omitted optional input) → outputs allocated
 * from the session pool (ctx.NewUninit). `*n_out` receives the count. */
int ingot_rocm_op_run(ingot_rocm_op* op, int n_in, const ingot_rocm_tensor* in, int max_out, ingot_rocm_tensor* out,
                      int* n_out);
/* Declares input `input` of the op constant (is_const = 1): its device storage
 * holds the same values on every run, as a graph initializer does. Such a
 * weight operand is packed once and the pack reused; every undeclared operand
 * is packed per call, since a pooled device buffer is handed back at the same
 * address with new contents. The reference's GPU session caches only graph
 * constants, by value id (bf16Const, graph/gpuops_darwin_arm64.go:610-629);
 * the CPU bCache keys on storage (ops/matmul.go:200-236). The graph session
 * marks its bound constants itself. */
int ingot_rocm_op_set_const(ingot_rocm_op* op, int input, int is_const);
int ingot_rocm_op_free(ingot_rocm_op* op);
/* Returns an op output's storage to the session pool (Session.Release). */
int ingot_rocm_tensor_release(ingot_rocm_session* s, ingot_rocm_tensor* t);

/* ---- Graph session ----
 * An ONNX node list over the operator layer, compiled with the reference's
 * GPU-session planning for this path and run on the session stream
 * (reference: graph.CompileGPU / GPUSession.Run, graph/gpu_other.go:13-37,
 * graph/gpu_darwin_arm64.go:96-576). Text form, one statement per line:
 *   input  <name> <dtype> [<d0,d1,...> | ?]
 *   const  <name> <dtype> <d0,d1,...>      (device data: ingot_rocm_graph_bind)
 *   node   [<domain>.]<op>[@<opset>] <in,...|_> -> <out,...> [<attrs>]
 *   output <name>
 * dtype: f32 bf16 f16 i8 u8 i16 i32 i64 bool; attrs as for ingot_rocm_op_create.
 * With s = NULL a graph can be created, bound, compiled and described but
 * not run (planning on a host without a GPU). */
typedef struct ingot_rocm_graph ingot_rocm_graph;
#define INGOT_GRAPH_FUSE_BIAS 1 /* fuseMatMulBias (graph/fuse_matmul_bias.go:12-63) */
#define INGOT_GRAPH_FUSE_ACT 2  /* a product's sole activation consumer in its store (planHalf,
                                   graph/gpuhalf_darwin_arm64.go:53-73) */
#define INGOT_GRAPH_HALF 4      /* GPUBF16 (graph/device.go:20-30): bf16 products against constant
                                   weights, bf16-resident values read only by them */
int ingot_rocm_graph_create(ingot_rocm_session* s, const char* text, ingot_rocm_graph** out);
/* Binds a declared constant to device data (same dtype and shape). */
int ingot_rocm_graph_bind(ingot_rocm_graph* g, const char* name, const ingot_rocm_tensor* t);
int ingot_rocm_graph_compile(ingot_rocm_graph* g, int flags);
/* Feeds inputs by name; outputs come back in declaration order as session
 * pool tensors (release each with ingot_rocm_tensor_release). */
int ingot_rocm_graph_run(ingot_rocm_graph* g, int n_in, const char* const* names, const ingot_rocm_tensor* in,
                         int max_out, ingot_rocm_tensor* out, int* n_out);
/* what = 0: pass statistics ("fuse-act=2;fuse-matmul-bias=2;half-out=1;steps=3;");
 * what = 1: the compiled steps, one line each. */
int ingot_rocm_graph_describe(const ingot_rocm_graph* g, int what, char* buf, size_t n);
int ingot_rocm_graph_free(ingot_rocm_graph* g);

#ifdef __cplusplus
}
#endif
#endif /* INGOT_ROCM_H */
