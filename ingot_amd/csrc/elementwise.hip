// Memory-bound helper kernels: weight and activation packing, DequantizeLinear,
// the standalone activation / bias pass, the f32 → bf16 cast and fills.

#include <algorithm>

#include "kernels.hpp"

namespace ingot {

namespace {

__device__ __forceinline__ float load_f(const void* p, int dt, int64_t i) {
    switch (dt) {
        case INGOT_DT_F32: return ((const float*)p)[i];
        case INGOT_DT_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
        default: return 0.f;
    }
}

__device__ __forceinline__ int32_t load_i(const void* p, int dt, int64_t i) {
    switch (dt) {
        case INGOT_DT_U8: return (int32_t)((const uint8_t*)p)[i];
        case INGOT_DT_I8: return (int32_t)((const int8_t*)p)[i];
        case INGOT_DT_I32: return ((const int32_t*)p)[i];
        default: return 0;
    }
}

inline unsigned grid_for(int64_t work, int per_block) {
    int64_t b = (work + per_block - 1) / per_block;
    if (b > (1 << 20)) b = 1 << 20;
    if (b < 1) b = 1;
    return (unsigned)b;
}

// dst[j][k] (np × kp, dst_kind) = src element (j, k) of the logical [n][k]
// weight, zero outside n × k. One thread per destination element.
__global__ void pack_weight_kernel(const void* src, int src_dt, int64_t ld, int trans, int64_t n, int64_t k,
                                   void* dst, int dst_kind, int64_t np, int64_t kp, int64_t ldk, int64_t src_item,
                                   int64_t dst_item) {
    // blockIdx.y: matrix item (src_item / dst_item elements apart)
    const int dsz = dst_kind == KIND_I8 ? 1 : (dst_kind == KIND_BF16 ? 2 : 4);
    const int ssz = src_dt == INGOT_DT_F32 ? 4 : (src_dt == INGOT_DT_BF16 ? 2 : 1);
    src = (const char*)src + blockIdx.y * src_item * ssz;
    dst = (char*)dst + blockIdx.y * dst_item * dsz;
    const int64_t total = np * kp;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t j = t / kp, kk = t - j * kp;
        const int64_t i = j * ldk + kk;
        const bool in = j < n && kk < k;
        const int64_t si = trans ? j * ld + kk : kk * ld + j;
        if (dst_kind == KIND_I8) {
            ((int8_t*)dst)[i] = in ? ((const int8_t*)src)[si] : (int8_t)0;
        } else {
            const float v = in ? load_f(src, src_dt, si) : 0.f;
            if (dst_kind == KIND_BF16) {
                ((uint16_t*)dst)[i] = (in && src_dt == INGOT_DT_BF16) ? ((const uint16_t*)src)[si] : f32_to_bf16(v);
            } else {
                ((float*)dst)[i] = v;
            }
        }
    }
}

// One wave per row: colsum[j] = Σ_k packed[j][k] (int32 wrap-around).
__global__ void colsum_kernel(const int8_t* packed, int64_t kp, int64_t ldk, int64_t n, int32_t* colsum) {
    const int64_t j = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (j >= n) return;
    uint32_t s = 0;
    for (int64_t k = lane; k < kp; k += 64) s += (uint32_t)(int32_t)packed[j * ldk + k];
    for (int off = 32; off > 0; off >>= 1) s += (uint32_t)__shfl_xor((int)s, off);
    if (lane == 0) colsum[j] = (int32_t)s;
}

// Packs activations into [m][kl] rows of dst_kind, zero padded beyond k.
// Each thread produces one 16-byte chunk of a destination row. KIND_BF16X2
// writes two planes, hi at dst and lo at dst + plane (split_bf16).
__device__ __forceinline__ float load_a(const char* sb, int src_dt, int trans, int64_t lda, int64_t row, int64_t kk) {
    const int64_t si = trans ? kk * lda + row : row * lda + kk;
    return load_f(sb, src_dt, si);
}

template <int KD>
__global__ void pack_a_kernel(const void* src, int src_dt, int64_t lda, int trans, int64_t m, int64_t k,
                              int64_t src_stride, void* dst, int64_t kl, int64_t dst_stride, int64_t plane) {
    // grid: x over the 16-byte chunks of a row, y over rows (strided), z over batch items
    constexpr int EPC = KD == KIND_F32 ? 4 : (KD == KIND_I8 ? 16 : 8);  // elements per chunk
    const int64_t chunks_per_row = kl / EPC;
    const int64_t cc = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (cc >= chunks_per_row) return;
    const int b = blockIdx.z;
    const char* sb = (const char*)src;
    const int esz = src_dt == INGOT_DT_F32 ? 4 : (src_dt == INGOT_DT_BF16 ? 2 : 1);
    sb += (int64_t)b * src_stride * esz;
    const int esz_d = KD == KIND_F32 ? 4 : (KD == KIND_I8 ? 1 : 2);
    const int64_t k0 = cc * EPC;
    for (int64_t row = blockIdx.y; row < m; row += gridDim.y) {
        char* db = (char*)dst + ((int64_t)b * dst_stride + row * kl + k0) * esz_d;
        if (KD == KIND_I8) {
            uint8_t v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t kk = k0 + e;
                uint8_t x = 0;
                if (kk < k) {
                    const int64_t si = trans ? kk * lda + row : row * lda + kk;
                    x = ((const uint8_t*)sb)[si];
                    if (src_dt == INGOT_DT_U8) x ^= 0x80;
                }
                v[e] = x;
            }
            i32x4_t out;
            __builtin_memcpy(&out, v, 16);
            *(i32x4_t*)db = out;
        } else if (KD == KIND_F32) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = k0 + e < k ? load_a(sb, src_dt, trans, lda, row, k0 + e) : 0.f;
            i32x4_t out;
            __builtin_memcpy(&out, v, 16);
            *(i32x4_t*)db = out;
        } else {
            float v[8];
            if (!trans && src_dt == INGOT_DT_F32 && k0 + 8 <= k && ((row * lda + k0) & 3) == 0 &&
                (((uintptr_t)sb) & 15) == 0) {
                const f32x4_t* s4 = (const f32x4_t*)((const float*)sb + row * lda + k0);
                const f32x4_t lo = s4[0], hi = s4[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = lo[e];
                    v[e + 4] = hi[e];
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = k0 + e < k ? load_a(sb, src_dt, trans, lda, row, k0 + e) : 0.f;
            }
            uint16_t h[8], l[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (KD == KIND_BF16X2)
                    split_bf16(v[e], h[e], l[e]);
                else
                    h[e] = f32_to_bf16(v[e]);
            }
            i32x4_t out;
            __builtin_memcpy(&out, h, 16);
            *(i32x4_t*)db = out;
            if (KD == KIND_BF16X2) {
                __builtin_memcpy(&out, l, 16);
                *(i32x4_t*)(db + plane * esz_d) = out;
            }
        }
    }
}

// The common activation pack — f32 rows already dense in whole k-tiles (lda = k = kl, one batch
// item), to bf16 (or the hi/lo planes) — as a flat stream: each thread converts U groups of 8
// elements per step, all U loads issued before any conversion, over a grid of a few workgroups
// per CU (grid-stride), so that the copy runs at streaming rate instead of one small workgroup
// per 2048 elements.
template <int KD, int U>
__global__ __launch_bounds__(256) void pack_a_flat_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                          int64_t groups, int64_t plane) {
    const int64_t stride = (int64_t)gridDim.x * 256 * U;
    for (int64_t g0 = (int64_t)blockIdx.x * 256 * U + threadIdx.x; g0 < groups; g0 += stride) {
        f32x4_t v[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = g0 + (int64_t)u * 256;
            if (g < groups) {
                v[u][0] = __builtin_nontemporal_load((const f32x4_t*)(src + g * 8));
                v[u][1] = __builtin_nontemporal_load((const f32x4_t*)(src + g * 8 + 4));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = g0 + (int64_t)u * 256;
            if (g >= groups) continue;
            uint16_t h[8], l[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = v[u][e >> 2][e & 3];
                if (KD == KIND_BF16X2)
                    split_bf16(x, h[e], l[e]);
                else
                    h[e] = f32_to_bf16(x);
            }
            i32x4_t out;
            __builtin_memcpy(&out, h, 16);
            *(i32x4_t*)(dst + g * 8) = out;
            if (KD == KIND_BF16X2) {
                __builtin_memcpy(&out, l, 16);
                *(i32x4_t*)(dst + plane + g * 8) = out;
            }
        }
    }
}

__global__ void dequant_kernel(const void* x, int x_dt, int64_t n, const float* scale, int64_t n_scale, int64_t inner,
                               const void* zp, int zp_dt, int64_t n_zp, float* y) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t c = n_scale == 1 ? 0 : (i / inner) % n_scale;
        int32_t z = 0;
        if (zp) z = load_i(zp, zp_dt, n_zp > 1 ? c : 0);
        y[i] = (float)wrap_add(load_i(x, x_dt, i), -z) * scale[c];
    }
}

__global__ void activation_kernel(const float* x, float* y, int64_t rows, int64_t cols, const float* bias, int act,
                                  float a, float b, int post, float ps, float pb) {
    const int64_t total = rows * cols;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        float v = x[i];
        if (bias) v += bias[i % cols];
        if (act != INGOT_ACT_NONE) v = apply_act(v, act, a, b);
        if (post) v = v * ps + pb;
        y[i] = v;
    }
}

__global__ void cast_bf16_kernel(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = f32_to_bf16(x[i]);
}

__global__ void fill_kernel(uint8_t* d, uint8_t v, size_t bytes) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < bytes; i += (size_t)gridDim.x * blockDim.x)
        d[i] = v;
}

}  // namespace

hipError_t launch_pack_weight(const void* src, int src_dtype, int64_t ld, int trans, int64_t n, int64_t k, void* dst,
                              GemmKind dst_kind, int64_t np, int64_t kp, int64_t ldk, hipStream_t st, int items,
                              int64_t src_item, int64_t dst_item) {
    hipLaunchKernelGGL(pack_weight_kernel, dim3(grid_for(np * kp, 256), items), dim3(256), 0, st, src, src_dtype, ld,
                       trans, n, k, dst, (int)dst_kind, np, kp, ldk, src_item, dst_item);
    return hipGetLastError();
}

hipError_t launch_colsum_i8(const int8_t* packed, int64_t kp, int64_t ldk, int64_t n, int32_t* colsum,
                            hipStream_t st) {
    hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, packed, kp, ldk, n, colsum);
    return hipGetLastError();
}

hipError_t launch_pack_a(const void* src, int src_dtype, int64_t lda, int trans, int64_t m, int64_t k,
                         int64_t src_stride, void* dst, GemmKind dst_kind, int64_t kl, int64_t dst_stride, int batch,
                         hipStream_t st) {
    const int epc = dst_kind == KIND_F32 ? 4 : (dst_kind == KIND_I8 ? 16 : 8);
    // (large activations only: at decode sizes the per-row grid below spreads the few rows over more CUs;
    // M = 16, K = 2048 took 5.4 us flat against 3.7)
    if ((dst_kind == KIND_BF16 || dst_kind == KIND_BF16X2) && src_dtype == INGOT_DT_F32 && !trans && batch == 1 &&
        lda == k && kl == k && k % 8 == 0 && m * k >= ((int64_t)1 << 22) && (((uintptr_t)src) & 15) == 0 &&
        (((uintptr_t)dst) & 15) == 0) {
        const int64_t groups = m * k / 8;
        const int64_t need = (groups + 256 * 4 - 1) / (256 * 4);
        const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(need, 2048));
        if (dst_kind == KIND_BF16)
            hipLaunchKernelGGL((pack_a_flat_kernel<KIND_BF16, 4>), dim3(grid), dim3(256), 0, st, (const float*)src,
                               (uint16_t*)dst, groups, m * kl);
        else
            hipLaunchKernelGGL((pack_a_flat_kernel<KIND_BF16X2, 4>), dim3(grid), dim3(256), 0, st, (const float*)src,
                               (uint16_t*)dst, groups, m * kl);
        return hipGetLastError();
    }
    const int64_t chunks = kl / epc;
    dim3 grid((unsigned)((chunks + 255) / 256), (unsigned)(m < 65535 ? (m > 0 ? m : 1) : 65535), batch);
    const int64_t plane = m * kl;
    switch (dst_kind) {
        case KIND_BF16:
            hipLaunchKernelGGL(pack_a_kernel<KIND_BF16>, grid, dim3(256), 0, st, src, src_dtype, lda, trans, m, k,
                               src_stride, dst, kl, dst_stride, plane);
            break;
        case KIND_BF16X2:
            hipLaunchKernelGGL(pack_a_kernel<KIND_BF16X2>, grid, dim3(256), 0, st, src, src_dtype, lda, trans, m, k,
                               src_stride, dst, kl, dst_stride, plane);
            break;
        case KIND_F32:
            hipLaunchKernelGGL(pack_a_kernel<KIND_F32>, grid, dim3(256), 0, st, src, src_dtype, lda, trans, m, k,
                               src_stride, dst, kl, dst_stride, plane);
            break;
        case KIND_I8:
            hipLaunchKernelGGL(pack_a_kernel<KIND_I8>, grid, dim3(256), 0, st, src, src_dtype, lda, trans, m, k,
                               src_stride, dst, kl, dst_stride, plane);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_dequant(const void* x, int x_dtype, int64_t n, const float* scale, int64_t n_scale, int64_t inner,
                          const void* zp, int zp_dtype, int64_t n_zp, float* y, hipStream_t st) {
    hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, x, x_dtype, n, scale, n_scale,
                       inner < 1 ? 1 : inner, zp, zp_dtype, n_zp, y);
    return hipGetLastError();
}

hipError_t launch_activation(const float* x, float* y, int64_t rows, int64_t cols, const float* bias, int act, float a,
                             float b, int post, float ps, float pb, hipStream_t st) {
    hipLaunchKernelGGL(activation_kernel, dim3(grid_for(rows * cols, 256)), dim3(256), 0, st, x, y, rows, cols, bias,
                       act, a, b, post, ps, pb);
    return hipGetLastError();
}

hipError_t launch_cast_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL(cast_bf16_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, x, y, n);
    return hipGetLastError();
}

hipError_t launch_fill(void* dst, int value, size_t bytes, hipStream_t st) {
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for((int64_t)bytes, 256)), dim3(256), 0, st, (uint8_t*)dst,
                       (uint8_t)value, bytes);
    return hipGetLastError();
}

}  // namespace ingot
