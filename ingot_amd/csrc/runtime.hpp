// Session and weight objects shared by runtime.cpp and ops.cpp.
#pragma once

#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "kernels.hpp"

struct ingot_rocm_weight {
    int pack_dtype;          // INGOT_DT_F32 / BF16 / I8
    ingot::GemmKind kind;
    int64_t n, k;            // logical [n][k]
    int64_t np, kp;          // packed [np][kp], zero padded to multiples of 256
    int64_t ldk;             // row pitch in elements (>= kp)
    void* data;
    int32_t* colsum;         // int8 weights: Σ_k W[n][k]
    float* gscale;           // KIND_I8G: one scale per 64 k of a row, [np][kp / 64]
};

struct ingot_rocm_session {
    int device = 0;
    int num_cus = 256;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    void* scratch = nullptr;  // this device's fixed scratch array (ingot_rocm_gemm_noalloc)
    void* ws = nullptr;  // workspace: packed activations (bf16 A planes, GEMV x planes, int8 A, im2col)
    size_t ws_bytes = 0;
    // Test and bisection hooks, read once when the session opens (a launch
    // must not pay for getenv): INGOT_GEMM_CFG forces a GEMM tile
    // configuration, INGOT_GEMV_CFG a GEMV launch configuration,
    // INGOT_I8G_ROWS the int8 GEMV rows per wave, INGOT_NO_GEMV sends decode
    // rows to the GEMM, INGOT_QCONV_PATH forces QLinearConv's route (1 direct,
    // 2 GEMM). -1 / 0 / false: not set.
    int force_gemm_cfg = -1;
    int force_gemv_cfg = 0;
    int i8g_rows = 0;
    bool no_gemv = false;
    int qconv_path = 0;
    std::vector<ingot_rocm_weight*> weights;
    std::map<size_t, std::vector<void*>> free_bufs;    // pool: size class → free buffers
    std::unordered_map<void*, size_t> buf_class;       // pool: buffer → size class
};

namespace ingot {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
int session_enter(ingot_rocm_session* s);
int ws_reserve(ingot_rocm_session* s, size_t bytes, void** out);
// Applies a graph plan to an op of the operator layer (ops.cpp).
int op_plan(ingot_rocm_op* op, int fused_act, bool half, bool out_bf16);
void* pool_get(ingot_rocm_session* s, size_t bytes);
void pool_put(ingot_rocm_session* s, void* p);

}  // namespace ingot
