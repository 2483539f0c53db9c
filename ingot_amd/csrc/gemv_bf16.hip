// Decode GEMV for gfx950: y[m,n] = epilogue(Σ_k x[m,k]·W[n,k]) for M <= 16
// rows of f32 activations against a packed bf16 weight [Np][Kp]. Two kernels:
// M <= 4 streams weight rows whole with VALU FMAs (gemv_rows_kernel, below);
// M = 5..16 runs the MFMA kernel described here.
//
// HBM-bound: the weight is streamed exactly once with 16-byte loads, and all
// of a wave's loads for a round are issued before any MFMA waits on them.
// The products run on v_mfma_f32_16x16x32_bf16 with the weight as the first
// operand (16 weight rows) and the activations as the second (up to 16 rows,
// zero beyond M). To keep f32 activation accuracy, each x is split into bf16
// hi + lo parts (hi = bf16(x), lo = bf16(x − hi); |x − hi − lo| <= 2⁻¹⁷|x|)
// and both are multiplied: bf16×bf16 products are exact in f32, so the only
// roundings are the f32 accumulations, as in the reference's f32 dot
// (kernels/vek/vek_generic.go:183-190). Under INGOT_MATH_BF16 (split = 0)
// only the hi part is used: x rounded to bf16 once.
//
// Work split: one workgroup per 16 weight rows; its NW waves split K
// (wavefront split-K) by 256-wide rounds, round t going to wave t % NW. In a
// round, lane (r, g) loads, for u = 0..7, the 16 bytes of row r at
// k = t·256 + (u·4 + g)·8: every load instruction reads 64 contiguous bytes
// of each of the 16 rows. Lanes r < M read the same k of activation row r
// (f32, L2-resident) and split it in registers. The NW partial tiles are
// added in wave order through LDS — deterministic, no cross-workgroup
// traffic, no fences — and the epilogue runs on the sum.
//
// Reference counterparts: gemvBF16 / gemm.GemvBF16 (ops/matmul.go:177-190,
// kernels/gemm/bgemm.go:201-206) and the Metal gemv_bf16 kernel
// (kernels/metal/decode.go:9-64).

#include "kernels.hpp"

namespace ingot {

namespace {

constexpr int KR = 256;  // k granularity of the packed weight

__device__ __forceinline__ void split8(const float* v, i32x4_t& hi, i32x4_t& lo, bool split) {
    uint16_t h[8], l[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        h[e] = f32_to_bf16(v[e]);
        l[e] = split ? f32_to_bf16(v[e] - bf16_to_f32(h[e])) : (uint16_t)0;
    }
    __builtin_memcpy(&hi, h, 16);
    __builtin_memcpy(&lo, l, 16);
}

// U: 16-byte weight chunks per lane per round (a round covers 32·U of k).
template <int NW, int U>
__global__ __launch_bounds__(64 * NW) void gemv_bf16_kernel(GemvArgs p) {
    constexpr int RK = 32 * U;  // k per round
    __shared__ f32x4_t red[NW][64];
    const int rb = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int rounds = (int)(p.kp / RK);

    const uint16_t* wrow = p.w + (int64_t)(rb * 16 + r) * p.ldw + g * 8;
    const bool xrow = r < p.M;
    const float* xr = p.x + (int64_t)(xrow ? r : 0) * p.ldx + g * 8;

    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int t = wave; t < rounds; t += NW) {
        i32x4_t w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) w[u] = *(const i32x4_t*)(wrow + t * RK + u * 32);
        float xv[U][8];
        if (xrow) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k0 = t * RK + u * 32 + g * 8;
                const float* src = xr + t * RK + u * 32;
                if (p.x_vec && k0 + 8 <= p.K) {
                    const f32x4_t a = *(const f32x4_t*)src, b = *(const f32x4_t*)(src + 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        xv[u][e] = a[e];
                        xv[u][e + 4] = b[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xv[u][e] = k0 + e < p.K ? src[e] : 0.f;
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[u][e] = 0.f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            i32x4_t hi, lo;
            split8(xv[u], hi, lo, p.split);
            const bf16x8_t wv = __builtin_bit_cast(bf16x8_t, w[u]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, __builtin_bit_cast(bf16x8_t, hi), acc, 0, 0, 0);
            if (p.split) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, __builtin_bit_cast(bf16x8_t, lo), acc, 0, 0, 0);
        }
    }

    // lane (r, g) holds y[m = r][n = rb·16 + 4g + q], q = 0..3
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0 || !xrow) return;
    f32x4_t sum = red[0][lane];
#pragma unroll
    for (int v = 1; v < NW; ++v) sum += red[v][lane];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = rb * 16 + 4 * g + q;
        if (n < p.N) p.y[(int64_t)r * p.ldy + n] = epi_apply(p.epi, sum[q], r, n);
    }
}

}  // namespace

// ---- M <= 4: rows streamed whole by VALU FMAs ----
// A wave owns R weight rows and walks K in 512-wide chunks: lane l reads the
// 16 bytes at k = c·512 + 8l of each row (1 KiB contiguous per row per load
// instruction) and the matching 8 f32 activations of each of the MM rows, and
// accumulates in f32. The 64 lane partials of each output are then added by a
// fixed butterfly (deterministic). x stays f32 (the reference's f32 dot),
// except under INGOT_MATH_BF16 (split = 0), where it is rounded to bf16 once.
template <int R, int MM>
__global__ __launch_bounds__(256) void gemv_rows_kernel(GemvArgs p) {
    constexpr int CH = MM >= 4 ? 2 : 4;  // chunks in flight per step
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * 4 + wave) * R;
    if (row0 >= p.N) return;
    const int chunks = (int)((p.kp + 511) / 512);
    float acc[R][MM];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;

    for (int c0 = 0; c0 < chunks; c0 += CH) {
        i32x4_t w[CH][R];
        float xv[CH][MM][8];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int k0 = (c0 + c) * 512 + lane * 8;
            const bool win = c0 + c < chunks && k0 < p.kp;
#pragma unroll
            for (int r = 0; r < R; ++r)
                w[c][r] = win ? *(const i32x4_t*)(p.w + (int64_t)(row0 + r) * p.ldw + k0) : i32x4_t{0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const float* src = p.x + (int64_t)m * p.ldx + k0;
                if (m < p.M && win && p.x_vec && k0 + 8 <= p.K) {
                    const f32x4_t a = *(const f32x4_t*)src, b = *(const f32x4_t*)(src + 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        xv[c][m][e] = a[e];
                        xv[c][m][e + 4] = b[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xv[c][m][e] = (m < p.M && win && k0 + e < p.K) ? src[e] : 0.f;
                }
            }
        }
        if (!p.split) {
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int m = 0; m < MM; ++m)
#pragma unroll
                    for (int e = 0; e < 8; ++e) xv[c][m][e] = bf16_to_f32(f32_to_bf16(xv[c][m][e]));
        }
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t* wb = (const uint32_t*)&w[c][r];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = __uint_as_float(wb[e] << 16);
                    const float hi = __uint_as_float(wb[e] & 0xFFFF0000u);
#pragma unroll
                    for (int m = 0; m < MM; ++m) {
                        acc[r][m] = fmaf(xv[c][m][2 * e], lo, acc[r][m]);
                        acc[r][m] = fmaf(xv[c][m][2 * e + 1], hi, acc[r][m]);
                    }
                }
            }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            float v = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            acc[r][m] = v;
        }
    if (lane != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = row0 + r;
        if (n >= p.N) continue;
#pragma unroll
        for (int m = 0; m < MM; ++m)
            if (m < p.M) p.y[(int64_t)m * p.ldy + n] = epi_apply(p.epi, acc[r][m], m, n);
    }
}

template <int R, int MM>
hipError_t launch_rows(const GemvArgs& a, hipStream_t st) {
    const int waves = (a.N + R - 1) / R;
    hipLaunchKernelGGL((gemv_rows_kernel<R, MM>), dim3((waves + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int NW, int U>
hipError_t launch_cfg(const GemvArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((gemv_bf16_kernel<NW, U>), dim3((a.N + 15) / 16), dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_gemv_bf16(const GemvArgs& a, int cfg, hipStream_t st) {
    if (a.kp % KR != 0 || a.M < 1 || a.M > 16) return hipErrorInvalidValue;
    if (cfg == 0) {  // default: rows kernel for M <= 4, MFMA kernel above
        if (a.M == 1) return launch_rows<1, 1>(a, st);
        if (a.M == 2) return launch_rows<1, 2>(a, st);
        if (a.M <= 4) return launch_rows<1, 4>(a, st);
        return launch_cfg<8, 2>(a, st);
    }
    switch (cfg) {
        case 10: return launch_rows<1, 1>(a, st);
        case 11: return launch_rows<2, 1>(a, st);
        case 12: return launch_rows<4, 1>(a, st);
        case 13: return launch_rows<1, 4>(a, st);
        case 14: return launch_rows<2, 4>(a, st);
        case 15: return launch_rows<1, 2>(a, st);
        case 20: return launch_cfg<8, 8>(a, st);
        case 1: return launch_cfg<4, 8>(a, st);
        case 2: return launch_cfg<8, 4>(a, st);
        case 3: return launch_cfg<4, 4>(a, st);
        case 4: return launch_cfg<2, 8>(a, st);
        case 5: return launch_cfg<4, 2>(a, st);
        case 6: return launch_cfg<16, 4>(a, st);
        case 7: return launch_cfg<8, 2>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace ingot
