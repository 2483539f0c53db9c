// Grouped-int8 decode GEMV for gfx950 (ingot_weight_quant="int8"):
// weights quantised once to int8 with one f32 scale per 64 consecutive k of
// a row, activations split per call into ~14-bit fixed point per 64-group,
// products as exact int32 group sums scaled in f32. Half the weight bytes of
// bf16 on an HBM-bound path.
//
// Reference: gemm.I8GWeights / quantizeI8G (kernels/gemm/i8g.go:12-56),
// vek.QuantizeX16 (kernels/vek/scalar.go:38-60), dotQ8Ref
// (kernels/vek/scalar.go:20-32) and GemvI8G (kernels/gemm/i8g.go:70-86).
// Every step is the reference's arithmetic: the quantisations use IEEE f32
// division/multiplication and round half to even; group sums are exact; the
// group terms (sx·sw)·float32(p) are added in group order by one lane, each
// operation rounded separately (no contraction in this file), so outputs
// match dotQ8Ref bit for bit.

#include "kernels.hpp"

#pragma clang fp contract(off)

namespace ingot {

namespace {

constexpr int G = 64;             // I8Group
constexpr float X16_MAX = 16256;  // 127·128

__device__ __forceinline__ float wave_max(float v, int lane) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, xor_partner(v, off, lane));
    return v;
}

__device__ __forceinline__ float load_w(const void* src, int dt, int64_t i) {
    if (dt == INGOT_DT_BF16) return __uint_as_float((uint32_t)((const uint16_t*)src)[i] << 16);
    return ((const float*)src)[i];
}

// One wave per (row j, group g): lane l takes k = 64g + l. s = max|w| / 127,
// q = clamp(RoundToEven(w / s), ±127); s = 0 leaves the group zero.
__global__ void quantize_w_kernel(const void* src, int src_dt, int64_t ld, int trans, int64_t n, int64_t k,
                                  int64_t np, int64_t gk, int8_t* q, float* sc, int64_t ldk) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= np * gk) return;
    const int lane = threadIdx.x & 63;
    const int64_t j = wid / gk, g = wid - j * gk;
    const int64_t kk = g * G + lane;
    const bool in = j < n && kk < k;
    const float v = in ? load_w(src, src_dt, trans ? j * ld + kk : kk * ld + j) : 0.f;
    const float s = wave_max(fabsf(v), lane) / 127.f;
    int qi = 0;
    if (s != 0.f) qi = (int)fminf(127.f, fmaxf(-127.f, rintf(v / s)));
    q[j * ldk + kk] = (int8_t)qi;
    if (lane == 0) sc[j * gk + g] = s;
}

// One wave per (row m, group g) of x: s = max|x| / 16256, inv = 1 / s,
// q = clamp(RoundToEven(x·inv), ±16256), xh = (q + 64) >> 7, xl = q − 128·xh.
__global__ void quantize_x_kernel(const float* x, int64_t ldx, int M, int64_t K, int64_t kp, int8_t* xh, int8_t* xl,
                                  float* sx) {
    const int64_t gk = kp / G;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= (int64_t)M * gk) return;
    const int lane = threadIdx.x & 63;
    const int64_t m = wid / gk, g = wid - m * gk;
    const int64_t kk = g * G + lane;
    const float v = kk < K ? x[m * ldx + kk] : 0.f;
    const float s = wave_max(fabsf(v), lane) / X16_MAX;
    int h = 0, l = 0;
    if (s != 0.f) {
        const float inv = 1.f / s;
        const int qi = (int)fminf(X16_MAX, fmaxf(-X16_MAX, rintf(v * inv)));
        h = (qi + 64) >> 7;
        l = qi - (h << 7);
    }
    xh[m * kp + kk] = (int8_t)h;
    xl[m * kp + kk] = (int8_t)l;
    if (lane == 0) sx[m * gk + g] = s;
}

// y[m][j] = epilogue(Σ_g (sx[m][g]·sw[j][g])·float32(p_g)): one wave per R
// weight rows, MM <= 4 activation rows. Lane l reads 16 int8 at
// k = 1024c + 16l of each row (1 KiB contiguous per load instruction) and of
// both x planes (shared by the R rows); p = 128·Σ w·xh + Σ w·xl by v_dot4
// (exact int32), summed over the 4 lanes of each 64-group; the group's lane
// writes its f32 term to the wave's LDS slice, and lane r·MM + m then adds
// (row r, activation row m)'s terms in group order. LDS operations of one
// wave complete in order, so the slice needs no workgroup barrier.
template <int R, int MM>
__global__ __launch_bounds__(256) void gemv_i8g_kernel(I8gArgs p) {
    extern __shared__ float terms[];  // [4 waves][R][MM][gk]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * R;
    if (row0 >= p.N) return;
    const int64_t gk = p.kp / G;
    float* t = terms + (int64_t)wave * R * MM * gk;
    const int chunks = (int)((p.kp + 1023) / 1024);
    // CH chunks per step, all loads issued before any dot product
    constexpr int CH = R * MM <= 2 ? 4 : 2;
    for (int c0 = 0; c0 < chunks; c0 += CH) {
        i32x4_t w[CH][R], h[CH][MM], l[CH][MM];
        float sw[CH][R], sx[CH][MM];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            if (c0 + c >= chunks) break;  // wave-uniform: no loads past the last chunk
            const int64_t k0 = (int64_t)(c0 + c) * 1024 + lane * 16;
            const int64_t kk = k0 < p.kp ? k0 : 0;
            const int64_t g = kk / G;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t j = min(row0 + r, (int64_t)p.N - 1);
                w[c][r] = *(const i32x4_t*)(p.q + j * p.ldk + kk);
                sw[c][r] = p.sw[j * gk + g];
            }
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const int mm = min(m, p.M - 1);
                h[c][m] = *(const i32x4_t*)(p.xh + mm * p.kp + kk);
                l[c][m] = *(const i32x4_t*)(p.xl + mm * p.kp + kk);
                sx[c][m] = p.sx[mm * gk + g];
            }
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            if (c0 + c >= chunks) break;
            const int64_t k0 = (int64_t)(c0 + c) * 1024 + lane * 16;
            // whole 4-lane groups are in or out together (kp % 64 == 0)
            const bool store = k0 < p.kp;
            const int64_t g = k0 / G;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m >= p.M) break;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    int ph = 0, pl = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ph = __builtin_amdgcn_sdot4(w[c][r][e], h[c][m][e], ph, false);
                        pl = __builtin_amdgcn_sdot4(w[c][r][e], l[c][m][e], pl, false);
                    }
                    int part = 128 * ph + pl;
                    part += xor_partner_bits(part, 1, lane);
                    part += xor_partner_bits(part, 2, lane);
                    if (store && (lane & 3) == 0) {
                        const float st = sx[c][m] * sw[c][r];
                        t[(r * MM + m) * gk + g] = st * (float)part;
                    }
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int r = lane / MM, m = lane % MM;
    const int64_t j = row0 + r;
    if (r >= R || m >= p.M || j >= p.N) return;
    // the adds stay in group order; the reads run ahead 8 terms at a time
    // (gk is a multiple of 4, so each row's slice is 16-byte aligned)
    const f32x4_t* tm = (const f32x4_t*)(t + (r * MM + m) * gk);
    float acc = 0.f;
    int64_t gi = 0;
    for (; gi + 8 <= gk; gi += 8) {
        const f32x4_t u0 = tm[gi / 4], u1 = tm[gi / 4 + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + u0[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + u1[e];
    }
    for (; gi < gk; gi += 4) {
        const f32x4_t u0 = tm[gi / 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + u0[e];
    }
    // GemvI8G's store (kernels/gemm/i8g.go:79-84): alpha·dot, then + beta·C
    const Epi& e = p.epi;
    float v = e.alpha * acc;
    switch (e.c_mode) {
        case INGOT_C_FULL: v = v + e.beta * e.c[m * e.ldc + j]; break;
        case INGOT_C_ROW: v = v + e.beta * e.c[j]; break;
        case INGOT_C_COL: v = v + e.beta * e.c[m]; break;
        case INGOT_C_SCALAR: v = v + e.beta * e.c[0]; break;
        default: break;
    }
    if (e.act != INGOT_ACT_NONE) v = apply_act(v, e.act, e.act_alpha, e.act_beta);
    if (e.post) v = v * e.post_scale + e.post_shift;
    store_y(p.y, (int64_t)m * p.ldy + j, v, e);
}

template <int R, int MM>
hipError_t launch_i8g(const I8gArgs& a, hipStream_t st) {
    const size_t lds = (size_t)4 * R * MM * (a.kp / G) * sizeof(float);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const int64_t waves = (a.N + R - 1) / R;
    hipLaunchKernelGGL((gemv_i8g_kernel<R, MM>), dim3((unsigned)((waves + 3) / 4)), dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int MM>
hipError_t launch_i8g_rows(const I8gArgs& a, int cfg, hipStream_t st) {
    // rows per wave: as many as keep >= 4096 waves in flight (16 per CU) and
    // fit the wave's LDS slice (4 waves · R · MM · kp/64 floats <= 64 KiB)
    int r = cfg ? cfg : (a.N >= 4 * 4096 ? 4 : (a.N >= 2 * 4096 ? 2 : 1));
    while (r > 1 && (size_t)4 * r * MM * (a.kp / G) * sizeof(float) > 64 * 1024) r /= 2;
    if (r == 4) return launch_i8g<4, MM>(a, st);
    if (r == 2) return launch_i8g<2, MM>(a, st);
    return launch_i8g<1, MM>(a, st);
}

}  // namespace

hipError_t launch_quantize_i8g(const void* src, int src_dtype, int64_t ld, int trans, int64_t n, int64_t k, int8_t* q,
                               float* scales, int64_t np, int64_t kp, int64_t ldk, hipStream_t st) {
    const int64_t waves = np * (kp / G);
    hipLaunchKernelGGL(quantize_w_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, src, src_dtype, ld,
                       trans, n, k, np, kp / G, q, scales, ldk);
    return hipGetLastError();
}

hipError_t launch_quantize_x16(const float* x, int64_t ldx, int M, int64_t K, int64_t kp, int8_t* xh, int8_t* xl,
                               float* sx, hipStream_t st) {
    const int64_t waves = (int64_t)M * (kp / G);
    hipLaunchKernelGGL(quantize_x_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, x, ldx, M, K, kp, xh,
                       xl, sx);
    return hipGetLastError();
}

hipError_t launch_gemv_i8g(const I8gArgs& a, int cfg, hipStream_t st) {
    if (a.M < 1 || a.M > 4 || a.kp % 256) return hipErrorInvalidValue;
    if (a.M == 1) return launch_i8g_rows<1>(a, cfg, st);
    if (a.M == 2) return launch_i8g_rows<2>(a, cfg, st);
    return launch_i8g_rows<4>(a, cfg, st);
}

}  // namespace ingot
