// Decode GEMV for gfx950: y[m,n] = epilogue(Σ_k x[m,k]·W[n,k]) for M <= 16
// rows of f32 activations against a packed bf16 weight [Np][Kp].
//
// HBM-bound: the weight is streamed exactly once with 16-byte loads, and all
// of a wave's loads for a round are issued before any MFMA waits on them.
// The products run on v_mfma_f32_16x16x32_bf16 with the weight as the first
// operand (16 weight rows per wave) and the activations as the second
// (up to 16 rows, zero beyond M). To keep f32 activation accuracy, each x is
// split into bf16 hi + lo parts (hi = bf16(x), lo = bf16(x − hi); |x − hi −
// lo| <= 2⁻¹⁷|x|) and both are multiplied: bf16×bf16 products are exact in
// f32, so the only roundings are the f32 accumulations, as in the reference's
// f32 dot (kernels/vek/vek_generic.go:183-190). Under INGOT_MATH_BF16
// (split = 0) only the hi part is used: x rounded to bf16 once.
//
// Work split: a workgroup (4 waves) owns 64 weight rows and one K slice of
// KS elements; the grid's y dimension splits K (wavefront split-K). Lane
// (r, g) of a wave loads, per round, 8 consecutive 16-byte chunks of row r:
// k = k0 + t·256 + g·64 + u·8 + [0, 8). The activation slice is staged once
// per workgroup in LDS (hi and lo planes, padded rows) and read with the same
// k mapping. With S > 1 the partial sums go to a scratch buffer and the last
// workgroup of each row block (arrival counter) adds the S partials in fixed
// order — deterministic, one launch — applies the epilogue and re-arms the
// counter.
//
// Reference counterparts: gemvBF16 / gemm.GemvBF16 (ops/matmul.go:177-190,
// kernels/gemm/bgemm.go:201-206) and the Metal gemv_bf16 kernel
// (kernels/metal/decode.go:9-64).

#include "kernels.hpp"

namespace ingot {

namespace {

constexpr int U = 8;        // 16-byte weight chunks per lane per round
constexpr int KR = 32 * U;  // k per round per wave

__global__ __launch_bounds__(256) void gemv_bf16_kernel(GemvArgs p) {
    extern __shared__ __attribute__((aligned(16))) char xs_raw[];
    __shared__ int s_last;
    const int M = p.M;
    const int KS = p.KS;
    const int XP = KS + 8;  // padded LDS row (elements)
    uint16_t* xhi = (uint16_t*)xs_raw;
    uint16_t* xlo = xhi + M * XP;

    const int rb = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int k0 = s * KS;

    const uint16_t* wp = p.w + (int64_t)(rb * 64 + wave * 16 + r) * p.ldw + k0 + g * (8 * U);
    i32x4_t w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = *(const i32x4_t*)(wp + u * 8);

    // stage x[0..M)[k0 .. k0+KS) as bf16 hi/lo planes
    for (int idx = tid; idx < M * KS; idx += 256) {
        const int m = idx / KS;
        const int kk = idx - m * KS;
        const int k = k0 + kk;
        const float v = k < p.K ? p.x[(int64_t)m * p.ldx + k] : 0.f;
        const uint16_t h = f32_to_bf16(v);
        xhi[m * XP + kk] = h;
        xlo[m * XP + kk] = p.split ? f32_to_bf16(v - bf16_to_f32(h)) : (uint16_t)0;
    }
    __syncthreads();

    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    const bool xrow = r < M;
    const uint16_t* xh = xhi + (xrow ? r : 0) * XP + g * (8 * U);
    const uint16_t* xl = xlo + (xrow ? r : 0) * XP + g * (8 * U);
    const i32x4_t zero = {0, 0, 0, 0};
    const int rounds = KS / KR;
    for (int t = 0; t < rounds; ++t) {
        const bool more = t + 1 < rounds;
        i32x4_t wn[U];
        if (more) {
#pragma unroll
            for (int u = 0; u < U; ++u) wn[u] = *(const i32x4_t*)(wp + (t + 1) * KR + u * 8);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const i32x4_t h = xrow ? *(const i32x4_t*)(xh + t * KR + u * 8) : zero;
            const i32x4_t l = xrow ? *(const i32x4_t*)(xl + t * KR + u * 8) : zero;
            const bf16x8_t wv = __builtin_bit_cast(bf16x8_t, w[u]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, __builtin_bit_cast(bf16x8_t, h), acc, 0, 0, 0);
            if (p.split) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, __builtin_bit_cast(bf16x8_t, l), acc, 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int u = 0; u < U; ++u) w[u] = wn[u];
        }
    }

    // lane (r, g) holds y[m = r][n = nb + q], q = 0..3
    const int nloc = wave * 16 + 4 * g;
    if (p.S == 1) {
        if (xrow) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = rb * 64 + nloc + q;
                if (n < p.N) p.y[(int64_t)r * p.ldy + n] = epi_apply(p.epi, acc[q], r, n);
            }
        }
        return;
    }

    float* part = p.part + (int64_t)(rb * p.S + s) * M * 64;
    if (xrow) *(f32x4_t*)(part + r * 64 + nloc) = acc;
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&p.cnt[rb], 1u) == (unsigned)(p.S - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float* pb = p.part + (int64_t)rb * p.S * M * 64;
    for (int idx = tid; idx < M * 64; idx += 256) {
        const int m = idx >> 6;
        const int n = rb * 64 + (idx & 63);
        float sum = 0.f;
        for (int s2 = 0; s2 < p.S; ++s2)
            sum += __hip_atomic_load(pb + (s2 * M + m) * 64 + (idx & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (n < p.N) p.y[(int64_t)m * p.ldy + n] = epi_apply(p.epi, sum, m, n);
    }
    if (tid == 0) __hip_atomic_store(&p.cnt[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_gemv_bf16(const GemvArgs& a, hipStream_t st) {
    if (a.KS % KR != 0 || a.M < 1 || a.M > 16) return hipErrorInvalidValue;
    dim3 grid((a.N + 63) / 64, a.S);
    const size_t lds = (size_t)a.M * (a.KS + 8) * 2 * sizeof(uint16_t);
    hipLaunchKernelGGL(gemv_bf16_kernel, grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

}  // namespace ingot
