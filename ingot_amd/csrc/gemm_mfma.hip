// MFMA GEMM for gfx950: Y[M,N] = epilogue(A[M,K] · B[N,K]ᵀ).
//
// One template serves the three math types of the hot path. In every case a
// lane feeds 16 bytes of K into each MFMA step:
//   bf16: v_mfma_f32_16x16x32_bf16 (8 bf16 per lane)
//   f32 : 4 × v_mfma_f32_16x16x4_f32 (one float per lane each)
//   int8: v_mfma_i32_16x16x64_i8 (16 int8 per lane)
// so one LDS layout (rows of 128-byte k-tiles, 16-byte pad to keep the
// 16-lane ds_read_b128 phases conflict free) and one k-slot mapping serve
// all three. Within an MFMA, lane group g = lane/16 supplies the 16-byte
// chunk g of the current 64-byte half of the k-tile for both operands, so
// the reduction pairs the same k on both sides.
//
// The weight is the first MFMA operand (rows n) and A the second (rows m):
// D[n][m] lands in lane (m%16, n/4) as 4 consecutive n, stored as one float4
// (or int4) per lane.
//
// Workgroup: 256 threads = 4 waves in a 2×2 grid, each wave a
// (BM/2)×(BN/2) sub-tile of 16×16 MFMA blocks. A and B k-tiles are staged
// global → registers → LDS with two LDS buffers (one barrier per k-tile);
// the next k-tile's global loads are in flight while the current one is
// multiplied. Tile order is XCD-aware (consecutive tiles of the grouped
// order run on one XCD's L2) and grouped by GROUP_M tile rows.
//
// Reference counterparts: the packed-B sweep + micro-kernel of
// kernels/gemm/gemm.go:280-334,431-490 (f32), PackBBF16/widenPanel
// kernels/gemm/gemm.go:920-962 (bf16 weights), QgemmPackedS8 + VNNI kernel
// kernels/gemm/qgemm.go:246-320 (int8), and the bias/act store epilogue of
// SgemmPackedBEpi kernels/gemm/gemm.go:521-597.

#include "kernels.hpp"

namespace ingot {

namespace {

constexpr int PITCH = KTILE_BYTES + 16;  // LDS row pitch in bytes
constexpr int GROUP_M = 4;

template <int KD> struct AccOf { typedef f32x4_t type; };
template <> struct AccOf<KIND_I8> { typedef i32x4_t type; };

template <int KD>
__device__ __forceinline__ void mma16(typename AccOf<KD>::type& acc, const i32x4_t& x, const i32x4_t& y);

template <>
__device__ __forceinline__ void mma16<KIND_BF16>(f32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, x), __builtin_bit_cast(bf16x8_t, y),
                                                   acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mma16<KIND_BF16X2>(f32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    mma16<KIND_BF16>(acc, x, y);
}

template <>
__device__ __forceinline__ void mma16<KIND_F32>(f32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    const f32x4_t xf = __builtin_bit_cast(f32x4_t, x);
    const f32x4_t yf = __builtin_bit_cast(f32x4_t, y);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[0], yf[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[1], yf[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[2], yf[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[3], yf[3], acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mma16<KIND_I8>(i32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, y, acc, 0, 0, 0);
}

template <int KD, int BM, int BN>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs p) {
    constexpr bool SPLIT = KD == KIND_BF16X2;
    constexpr int AP = SPLIT ? 2 : 1;  // activation planes
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int LA = BM / 32, LB = BN / 32;  // 16-byte chunks per thread per k-tile
    constexpr int STAGE = (AP * BM + BN) * PITCH;
    static_assert(BM % 32 == 0 && BN % 32 == 0, "tile must be a multiple of 32");
    typedef typename AccOf<KD>::type Acc;

    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // ---- tile coordinates: XCD-contiguous, then grouped along M ----
    const int nt = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
    const int per_group = GROUP_M * p.tiles_n;
    const int grp = bid / per_group;
    const int first_m = grp * GROUP_M;
    const int gsz = min(p.tiles_m - first_m, GROUP_M);
    const int in_grp = bid - grp * per_group;
    const int m0 = (first_m + in_grp % gsz) * BM;
    const int n0 = (in_grp / gsz) * BN;

    // ---- global load addressing (rows clamped; garbage rows are never stored) ----
    const char* A = p.a + (int64_t)blockIdx.y * p.stride_a_bytes;
    const int lrow = tid >> 3;
    const int lcol = (tid & 7) * 16;
    const char* pa[LA];
    const char* pb[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int m = min(m0 + lrow + i * 32, p.M - 1);
        pa[i] = A + (int64_t)m * p.lda_bytes + lcol;
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
        const int n = min(n0 + lrow + i * 32, p.b_rows - 1);
        pb[i] = p.b + (int64_t)n * p.ldb_bytes + lcol;
    }
    i32x4_t ra[AP][LA], rb[LB];
    const int axor = p.a_xor ? (int)0x80808080u : 0;

    auto gload = [&](int kt) {
        const int64_t off = (int64_t)kt * KTILE_BYTES;
#pragma unroll
        for (int pl = 0; pl < AP; ++pl)
#pragma unroll
            for (int i = 0; i < LA; ++i) ra[pl][i] = *(const i32x4_t*)(pa[i] + pl * p.a_plane_bytes + off);
#pragma unroll
        for (int i = 0; i < LB; ++i) rb[i] = *(const i32x4_t*)(pb[i] + off);
    };
    auto lstore = [&](int buf) {
        char* sa = smem + buf * STAGE;
        char* sb = sa + AP * BM * PITCH;
#pragma unroll
        for (int pl = 0; pl < AP; ++pl)
#pragma unroll
            for (int i = 0; i < LA; ++i) {
                i32x4_t v = ra[pl][i];
                if (KD == KIND_I8) v ^= axor;
                *(i32x4_t*)(sa + (pl * BM + lrow + i * 32) * PITCH + lcol) = v;
            }
#pragma unroll
        for (int i = 0; i < LB; ++i) *(i32x4_t*)(sb + (lrow + i * 32) * PITCH + lcol) = rb[i];
    };

    Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Acc{0, 0, 0, 0};

    // fragment read offsets: lane row (lane % 16), 16-byte chunk (lane / 16)
    const int frag_off = (lane & 15) * PITCH + (lane >> 4) * 16;
    const int a_off = (wm * WM) * PITCH + frag_off;
    const int b_off = AP * BM * PITCH + (wn * WN) * PITCH + frag_off;

    gload(0);
    lstore(0);
    __syncthreads();

    for (int kt = 0; kt < p.kt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < p.kt;
        if (more) gload(kt + 1);
        const char* st = smem + cur * STAGE;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            i32x4_t fa[AP][TM], fb[TN];
#pragma unroll
            for (int pl = 0; pl < AP; ++pl)
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    fa[pl][i] = *(const i32x4_t*)(st + a_off + (pl * BM + i * 16) * PITCH + s * 64);
#pragma unroll
            for (int j = 0; j < TN; ++j) fb[j] = *(const i32x4_t*)(st + b_off + j * 16 * PITCH + s * 64);
#pragma unroll
            for (int pl = 0; pl < AP; ++pl)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) mma16<KD>(acc[i][j], fb[j], fa[pl][i]);
        }
        if (more) lstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
    // Each wave stages half of its sub-tile at a time through its own LDS
    // region (the k-loop's buffers are free now): lanes write their 4-wide
    // column strips, then the wave walks the staged rows with row-contiguous
    // 16-byte stores. Accumulators are only indexed statically.
    constexpr int HR = WM / 2;          // rows per pass
    constexpr int SP = WN + 4;          // staging pitch (elements)
    static_assert(4 * HR * SP * 4 <= 2 * STAGE, "staging must fit in LDS");
    static_assert(WN % 4 == 0, "row width must be whole float4s");
    char* stage = smem + wave * (HR * SP * 4);
    const int r = lane & 15;
    const int g4 = (lane >> 4) * 4;
    const int row0 = m0 + wm * WM;
    const int col0 = n0 + wn * WN;
    const int64_t ybatch = (int64_t)blockIdx.y * p.stride_y;
    // 16-byte stores need an aligned row start (n is always a multiple of 4 here)
    uintptr_t ybase;
    if (KD == KIND_I8)
        ybase = (uintptr_t)(p.qepi.yi ? p.qepi.yi + ybatch : nullptr) | (uintptr_t)(p.qepi.yf ? p.qepi.yf + ybatch : nullptr);
    else
        ybase = (uintptr_t)((float*)p.y + ybatch);
    const bool vec_ok = (ybase & 15) == 0 && (p.ldy & 3) == 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < TM / 2; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                *(Acc*)(stage + ((i * 16 + r) * SP + j * 16 + g4) * 4) = acc[h * (TM / 2) + i][j];
        __syncthreads();
        constexpr int Q = WN / 4;  // float4 per staged row
        for (int idx = lane; idx < HR * Q; idx += 64) {
            const int rr = idx / Q;
            const int cc = (idx - rr * Q) * 4;
            const int m = row0 + h * HR + rr;
            const int n = col0 + cc;
            if (m >= p.M || n >= p.N) continue;
            const Acc a4 = *(const Acc*)(stage + (rr * SP + cc) * 4);
            const int64_t o = ybatch + (int64_t)m * p.ldy + n;
            const bool full = n + 3 < p.N;
            if (KD == KIND_I8) {
                const QEpi& q = p.qepi;
                const i32x4_t ai = __builtin_bit_cast(i32x4_t, a4);
                int32_t v[4];
                float f[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int nn = min(n + e, p.N - 1);
                    v[e] = wrap_add(ai[e], wrap_mul(q.colsum[nn], q.neg_za));
                    f[e] = q.yf ? (float)wrap_add(v[e], -q.dq_zp) * q.scale[q.n_scale == 1 ? 0 : nn] : 0.f;
                }
                if (full && vec_ok) {
                    if (q.yi) *(i32x4_t*)(q.yi + o) = i32x4_t{v[0], v[1], v[2], v[3]};
                    if (q.yf) *(f32x4_t*)(q.yf + o) = f32x4_t{f[0], f[1], f[2], f[3]};
                } else {
                    for (int e = 0; e < 4 && n + e < p.N; ++e) {
                        if (q.yi) q.yi[o + e] = v[e];
                        if (q.yf) q.yf[o + e] = f[e];
                    }
                }
            } else {
                float* y = (float*)p.y;
                const f32x4_t af = __builtin_bit_cast(f32x4_t, a4);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = epi_apply(p.epi, af[e], m, min(n + e, p.N - 1));
                if (full && vec_ok) {
                    *(f32x4_t*)(y + o) = f32x4_t{v[0], v[1], v[2], v[3]};
                } else {
                    for (int e = 0; e < 4 && n + e < p.N; ++e) y[o + e] = v[e];
                }
            }
        }
        __syncthreads();
    }
}

// Tile configurations per kind. occupancy: workgroups per CU the LDS and
// register footprint allow; eff: relative throughput per CU slot.
const GemmConfig kBF16Cfgs[] = {{256, 192, 1, 1.00f}, {128, 128, 2, 0.80f}, {128, 64, 2, 0.65f}, {64, 64, 4, 0.45f}};
const GemmConfig kF32Cfgs[] = {{128, 128, 2, 1.00f}, {128, 64, 2, 0.95f}, {64, 64, 4, 0.85f}};
const GemmConfig kBF16X2Cfgs[] = {{128, 128, 1, 1.00f}, {128, 64, 1, 0.85f}, {64, 64, 2, 0.60f}};
const GemmConfig kI8Cfgs[] = {{256, 192, 1, 1.00f}, {128, 128, 2, 0.80f}, {128, 64, 2, 0.65f}, {64, 64, 4, 0.45f}};

template <int KD, int BM, int BN>
hipError_t launch_one(const GemmArgs& a, int batch, hipStream_t st) {
    dim3 grid(a.tiles_m * a.tiles_n, batch);
    hipLaunchKernelGGL((gemm_kernel<KD, BM, BN>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace

int gemm_configs(GemmKind kind, const GemmConfig** out) {
    switch (kind) {
        case KIND_BF16: *out = kBF16Cfgs; return (int)(sizeof(kBF16Cfgs) / sizeof(kBF16Cfgs[0]));
        case KIND_F32: *out = kF32Cfgs; return (int)(sizeof(kF32Cfgs) / sizeof(kF32Cfgs[0]));
        case KIND_I8: *out = kI8Cfgs; return (int)(sizeof(kI8Cfgs) / sizeof(kI8Cfgs[0]));
        case KIND_BF16X2: *out = kBF16X2Cfgs; return (int)(sizeof(kBF16X2Cfgs) / sizeof(kBF16X2Cfgs[0]));
    }
    return 0;
}

hipError_t launch_gemm(GemmKind kind, int cfg, const GemmArgs& a, int batch, hipStream_t st) {
    switch (kind) {
        case KIND_BF16:
            switch (cfg) {
                case 0: return launch_one<KIND_BF16, 256, 192>(a, batch, st);
                case 1: return launch_one<KIND_BF16, 128, 128>(a, batch, st);
                case 2: return launch_one<KIND_BF16, 128, 64>(a, batch, st);
                case 3: return launch_one<KIND_BF16, 64, 64>(a, batch, st);
            }
            break;
        case KIND_F32:
            switch (cfg) {
                case 0: return launch_one<KIND_F32, 128, 128>(a, batch, st);
                case 1: return launch_one<KIND_F32, 128, 64>(a, batch, st);
                case 2: return launch_one<KIND_F32, 64, 64>(a, batch, st);
            }
            break;
        case KIND_BF16X2:
            switch (cfg) {
                case 0: return launch_one<KIND_BF16X2, 128, 128>(a, batch, st);
                case 1: return launch_one<KIND_BF16X2, 128, 64>(a, batch, st);
                case 2: return launch_one<KIND_BF16X2, 64, 64>(a, batch, st);
            }
            break;
        case KIND_I8:
            switch (cfg) {
                case 0: return launch_one<KIND_I8, 256, 192>(a, batch, st);
                case 1: return launch_one<KIND_I8, 128, 128>(a, batch, st);
                case 2: return launch_one<KIND_I8, 128, 64>(a, batch, st);
                case 3: return launch_one<KIND_I8, 64, 64>(a, batch, st);
            }
            break;
    }
    return hipErrorInvalidValue;
}

}  // namespace ingot
