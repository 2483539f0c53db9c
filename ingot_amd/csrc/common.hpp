// Shared device/host definitions for the gfx950 kernels of libingot_rocm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ingot_rocm.h"

namespace ingot {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// float32 → bfloat16 bits, round to nearest even, NaN kept quiet.
// Restates F32ToBF16 (kernels/gemm/bgemm.go:20-26) bit for bit.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t b;
    __builtin_memcpy(&b, &f, 4);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    __builtin_memcpy(&f, &b, 4);
    return f;
}

// A raw buffer resource over [base, base + bytes): loads at offsets past
// `bytes` return zero (and LDS-DMA loads write zeros), so kernels bound their
// reads by the resource instead of by branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// An LDS address as the LDS-DMA builtins take it.
#define LDS_AS(ptr) ((__attribute__((address_space(3))) void*)(ptr))

// The 32 bits lane ^ off holds (off = 32, 16, ..., 1: a butterfly partner),
// moved by VALU lane permutes instead of the LDS crossbar (ds_bpermute):
// off = 32 and 16 by the permlane swaps, which trade the upper half (of the
// wave, or of each pair of 16-lane rows) of one copy of u with the lower half
// of another, so lane l finds its partner in the copy whose half it is not in;
// 8 by a rotation of each row by 8 lanes; 4 by two row shifts, each written to
// the 4-lane banks that take from that direction; 2 and 1 by quad
// permutations. All 64 lanes must be active.
__device__ __forceinline__ int xor_partner_bits(int u, int off, int lane) {
    switch (off) {
        case 32: {
            const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            return (int)((lane & 32) ? s[0] : s[1]);
        }
        case 16: {
            const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            return (int)((lane & 16) ? s[0] : s[1]);
        }
        case 8: return __builtin_amdgcn_update_dpp(0, u, 0x128, 0xF, 0xF, false);  // row_ror:8
        case 4: {
            const int t = __builtin_amdgcn_update_dpp(0, u, 0x104, 0xF, 0x5, false);  // row_shl:4, banks 0, 2
            return __builtin_amdgcn_update_dpp(t, u, 0x114, 0xF, 0xA, false);         // row_shr:4, banks 1, 3
        }
        case 2: return __builtin_amdgcn_update_dpp(0, u, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
        default: return __builtin_amdgcn_update_dpp(0, u, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
    }
}
__device__ __forceinline__ float xor_partner(float x, int off, int lane) {
    return __int_as_float(xor_partner_bits(__float_as_int(x), off, lane));
}

// f32 x as two bf16 terms, hi + lo = x to within 2⁻¹⁷|x|, so that hi·w + lo·w
// over a bf16 w keeps f32-activation accuracy: hi = bf16(x) (RNE), lo =
// bf16(x − hi). Two cases keep the products IEEE-faithful: a finite x whose
// rounding overflows (|x| >= 0x1.ffp127) takes hi = ±0x7F7F, the largest
// finite bf16, so lo stays finite; a non-finite x (±Inf, NaN) is carried by
// hi alone with lo = +0, so ±Inf·w is ±Inf (not Inf − Inf = NaN) as in the
// f32 dot.
__host__ __device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    uint32_t b;
    __builtin_memcpy(&b, &x, 4);
    uint16_t h = f32_to_bf16(x);
    if ((b & 0x7FFFFFFFu) >= 0x7F800000u) {
        hi = h;
        lo = 0;
        return;
    }
    if ((h & 0x7FFFu) == 0x7F80u) h = (uint16_t)((h & 0x8000u) | 0x7F7Fu);
    hi = h;
    lo = f32_to_bf16(x - bf16_to_f32(h));
}

// Float epilogue: y = post_scale·act(alpha·acc + beta·C) + post_shift.
// The C operand follows the Gemm broadcast rules of ops/matmul.go:50-76.
struct Epi {
    float alpha, beta;
    const float* c;
    int64_t ldc;
    int c_mode;
    int act;
    float act_alpha, act_beta;
    int post;
    float post_scale, post_shift;
    int y_bf16;  // Y stored as bf16 (RNE) instead of f32
};

// One output element, f32 or bf16 (RNE) per the epilogue.
__device__ __forceinline__ void store_y(void* y, int64_t i, float v, const Epi& e) {
    if (e.y_bf16)
        ((uint16_t*)y)[i] = f32_to_bf16(v);
    else
        ((float*)y)[i] = v;
}

// The clamps compare, as Go's min and max do: a NaN passes through (fminf and
// fmaxf would return the bound instead).
__device__ __forceinline__ float clamp_to(float x, float lo, float hi) {
    x = x < lo ? lo : x;
    return x > hi ? hi : x;
}

// exp with the argument clamp of expScalar (kernels/vek/scalar.go:7-13).
__device__ __forceinline__ float exp_clamped(float x) { return __expf(clamp_to(x, -87.33654f, 88.37626f)); }

__device__ __forceinline__ float clamp01(float x) { return clamp_to(x, 0.f, 1.f); }

// erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the approximation
// the reference's amd64 GELU kernel evaluates (kernels/vek/genamd64/main.go:62-99):
//   erf(|z|) = 1 − t·(a1 + t·(a2 + t·(a3 + t·(a4 + t·a5))))·e^(−z²),
//   t = 1 / (1 + p·|z|), odd in z.
// The reciprocal and the exponential are the hardware ones (v_rcp_f32,
// v_exp_f32, about 1 ulp), far inside the formula's own error.
__device__ __forceinline__ float erf_as(float z) {
    const float az = fabsf(z);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, az, 1.f));
    float poly = fmaf(1.061405429f, t, -1.453152027f);
    poly = fmaf(poly, t, 1.421413741f);
    poly = fmaf(poly, t, -0.284496736f);
    poly = fmaf(poly, t, 0.254829592f);
    const float r = 1.f - poly * t * __expf(-az * az);
    return copysignf(r, z);
}

// Activation set of ops/epilogue.go:48-73 plus the GELU forms of
// ops/elementwise.go:411-414 (tanh) and kernels/vek/vek_amd64.go:346-353 (erf).
__device__ __forceinline__ float apply_act(float x, int act, float a, float b) {
    switch (act) {
        case INGOT_ACT_RELU: return fmaxf(x, 0.f);
        case INGOT_ACT_GELU_ERF: return 0.5f * x * (1.f + erf_as(x * 0.70710678118654752f));
        case INGOT_ACT_GELU_TANH: {
            // 1 + tanh(v) from u = e^(−2|v|) ∈ [0, 1]: 2/(1 + u) for v >= 0 and
            // 2u/(1 + u) for v < 0. Nothing cancels in the negative tail (x below
            // about −3, where 1 + tanh(v) is tiny), so the result stays accurate
            // relative to its value, and nothing overflows. The reference rounds
            // tanh(v) to float32 before adding 1, an absolute error of up to
            // 2^−25·|x| in that tail, which this stays within.
            const float v = 0.7978845608028654f * (x + 0.044715f * x * x * x);
            const float u = __expf(-2.f * fabsf(v));
            const float g = (v < 0.f ? 2.f * u : 2.f) * __builtin_amdgcn_rcpf(1.f + u);
            return 0.5f * x * g;
        }
        // IEEE quotients: past x = −87.3 the clamped 1 + e^(−x) exceeds 2^126, and
        // the hardware reciprocal would flush 1/(1 + e^(−x)) to zero where the
        // reference's quotient is subnormal (or, times a huge x, finite)
        case INGOT_ACT_SIGMOID: return 1.f / (1.f + exp_clamped(-x));
        case INGOT_ACT_SILU: return x / (1.f + exp_clamped(-x));
        case INGOT_ACT_HARDSWISH: return x * clamp01(x * (1.f / 6.f) + 0.5f);
        case INGOT_ACT_HARDSIGMOID: return clamp01(a * x + b);
        case INGOT_ACT_CLIP: return clamp_to(x, a, b);
        case INGOT_ACT_LEAKYRELU: return x < 0.f ? x * a : x;
        default: return x;
    }
}

__device__ __forceinline__ float epi_apply(const Epi& e, float acc, int64_t m, int64_t n) {
    float v = e.alpha * acc;
    switch (e.c_mode) {
        case INGOT_C_FULL: v += e.beta * e.c[m * e.ldc + n]; break;
        case INGOT_C_ROW: v += e.beta * e.c[n]; break;
        case INGOT_C_COL: v += e.beta * e.c[m]; break;
        case INGOT_C_SCALAR: v += e.beta * e.c[0]; break;
        default: break;
    }
    if (e.act != INGOT_ACT_NONE) v = apply_act(v, e.act, e.act_alpha, e.act_beta);
    if (e.post) v = v * e.post_scale + e.post_shift;
    return v;
}

// Integer epilogue of MatMulInteger + DequantizeLinear:
//   yi = acc + corr[n]                      (corr[n] = −za′·colSum[n], int32 wrap)
//   yf = float32(yi − dq_zp) · scale[n or 0]
struct QEpi {
    const int32_t* colsum;
    int32_t neg_za;  // −za′ (za′ = za − 128 for u8 activations shifted to s8)
    int32_t* yi;
    float* yf;
    const float* scale;
    int64_t n_scale;
    int32_t dq_zp;
    // QLinearMatMul (ops/quant.go:902-928): yq = sat(rne(fl32(fl32(float(yi))·rq_mult) + rq_zy))
    void* yq;
    int yq_u8;  // 1: u8 [0,255]; 0: s8 [-128,127]
    float rq_mult, rq_zy;
    // QLinearConv (ops/quant.go:441-468): an int32 bias added to the
    // correction and one multiplier per output column (NULL: none / rq_mult),
    // both at index col_batch·blockIdx.y + n, like colsum.
    const int32_t* bias;
    const float* rq_mults;
    int32_t col_batch;
    // conv_p > 0: row m is pixel m % conv_p of image m / conv_p and column n
    // its channel plane, stored at (m / conv_p)·conv_img + n·conv_p + m % conv_p
    // (NCHW); yq only.
    int32_t conv_p;
    int64_t conv_img;
};

__device__ __forceinline__ int32_t wrap_mul(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a * (uint32_t)b);
}
__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

}  // namespace ingot
