// Decode GEMV for gfx950: y[m,n] = epilogue(Σ_k x[m,k]·W[n,k]) for M <= 16
// rows of f32 activations against a packed bf16 weight [Np][Kp]. M <= 8
// streams weight rows with VALU FMAs — straight into registers at M = 1
// (gemv_rows_kernel, below), through LDS at M = 2..4 and at M = 5..8 with
// K <= 2048 (gemv_dma_kernel) — and the other M <= 16 products run the MFMA
// kernel described here.
//
// HBM-bound: the weight is streamed exactly once with 16-byte loads, and all
// of a wave's loads for a round are issued before any MFMA waits on them.
// The products run on v_mfma_f32_16x16x32_bf16 with the weight as the first
// operand (RB weight rows, the rest of the 16 zero) and the activations as
// the second (16 rows, zero beyond M). To keep f32 activation accuracy, x is
// split once per call, before this kernel, into bf16 hi + lo planes
// (split_bf16: hi = bf16(x), lo = bf16(x − hi); |x − hi − lo| <= 2⁻¹⁷|x|;
// non-finite x in hi alone) and both are
// multiplied: bf16×bf16 products are exact in f32, so the only roundings are
// the f32 accumulations, as in the reference's f32 dot
// (kernels/vek/vek_generic.go:183-190). Under INGOT_MATH_BF16 (split = 0)
// only the hi plane is used: x rounded to bf16 once. The planes are
// written by pack_x_kernel in MFMA fragment order — for each 32-wide k step
// the 16 rows × 32 k form 1 KiB in lane order (lane 16g + r: row r, k =
// 32s + 8g .. +7; rows >= M zero) — so each x load instruction of this
// kernel reads 1 KiB contiguous. Every workgroup reads all of x (twice the
// weight bytes it streams, with both planes): converting it per workgroup
// cost about five VALU operations per weight byte, and reading it with the
// weight's 16-rows × 64-byte pattern bound the kernel on address traffic.
//
// Work split: one workgroup per RB weight rows (RB = 8 keeps 256 workgroups
// busy at N = 2048); its NW waves split K by rounds of 32·U, round t going
// to wave t % NW. In a round, lane (r, g) loads, for u = 0..U-1, the 16
// bytes of weight row r (r < RB) at k = t·32U + 32u + 8g and its own 16
// bytes of x step t·U + u in both planes. The NW partial tiles are added in wave order through LDS —
// deterministic, no cross-workgroup traffic, no fences — and the epilogue
// runs on the sum.
//
// Reference counterparts: gemvBF16 / gemm.GemvBF16 (ops/matmul.go:177-190,
// kernels/gemm/bgemm.go:201-206) and the Metal gemv_bf16 kernel
// (kernels/metal/decode.go:9-64).

#include "kernels.hpp"

namespace ingot {

namespace {

constexpr int KR = 256;  // k granularity of the packed weight

// x (f32 [M][ldx]) → bf16 planes in MFMA fragment order: 16-byte chunk c is
// step s = c / 64, lane l = c % 64 (row r = l % 16, k = 32s + 8(l / 16));
// rows >= M and k >= K are zero. split: hi, lo = split_bf16(x); else hi = bf16(x) RNE.
__global__ void pack_x_kernel(const float* x, int64_t ldx, int M, int K, int64_t chunks, int split, uint16_t* dst,
                              int64_t plane) {
    const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const int l = (int)(c & 63);
    const int r = l & 15;
    const int64_t k0 = (c >> 6) * 32 + (l >> 4) * 8;
    uint16_t h[8], lo[8];
    float v[8];
    const float* src = x + (int64_t)r * ldx + k0;
    if (r < M && k0 + 8 <= K && (((uintptr_t)src) & 15) == 0) {  // two 16-byte loads
        const f32x4_t a = *(const f32x4_t*)src, b = *(const f32x4_t*)(src + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = a[e];
            v[e + 4] = b[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (r < M && k0 + e < K) ? src[e] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (split)
            split_bf16(v[e], h[e], lo[e]);
        else
            h[e] = f32_to_bf16(v[e]);
    }
    i32x4_t o;
    __builtin_memcpy(&o, h, 16);
    *(i32x4_t*)(dst + c * 8) = o;
    if (split) {
        __builtin_memcpy(&o, lo, 16);
        *(i32x4_t*)(dst + plane + c * 8) = o;
    }
}

template <int NW, int U, int RB>
__global__ __launch_bounds__(64 * NW) void gemv_mfma_kernel(GemvArgs p) {
    static_assert(RB == 8 || RB == 16, "8 or 16 weight rows per workgroup");
    constexpr int RK = 32 * U;  // k per round
    __shared__ f32x4_t red[NW][64];
    const int rb = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int rounds = (int)(p.kp / RK);

    const bool wrow = r < RB;
    const uint16_t* wrp = p.w + (int64_t)(rb * RB + (wrow ? r : 0)) * p.ldw + g * 8;
    const i32x4_t* xh_p = (const i32x4_t*)p.xb + lane;
    const i32x4_t* xl_p = (const i32x4_t*)(p.xb + p.xb_plane) + lane;

    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int t = wave; t < rounds; t += NW) {
        i32x4_t w[U], xh[U], xl[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            w[u] = wrow ? *(const i32x4_t*)(wrp + t * RK + u * 32) : i32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t step = (int64_t)(t * U + u) * 64;
            xh[u] = xh_p[step];
            xl[u] = p.split ? xl_p[step] : i32x4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bf16x8_t wv = __builtin_bit_cast(bf16x8_t, w[u]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, __builtin_bit_cast(bf16x8_t, xh[u]), acc, 0, 0, 0);
            if (p.split)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, __builtin_bit_cast(bf16x8_t, xl[u]), acc, 0, 0, 0);
        }
    }

    // lane (r, g) holds y[m = r][n = rb·RB + 4g + q], q = 0..3
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0 || r >= p.M || 4 * g >= RB) return;
    f32x4_t sum = red[0][lane];
#pragma unroll
    for (int v = 1; v < NW; ++v) sum += red[v][lane];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = rb * RB + 4 * g + q;
        if (n < p.N) store_y(p.y, (int64_t)r * p.ldy + n, epi_apply(p.epi, sum[q], r, n), p.epi);
    }
}

}  // namespace

// A wave's R·MM sums (acc[r][m]: row row0 + r of W times row m of x), each
// held as 64 lane partials, added by a butterfly over lane distances 32, 16,
// ..., 1 and stored through the epilogue. While more than one sum is left per
// lane, each step halves them: the lane keeps the upper half if its bit of the
// distance is set, else the lower half, and adds its partner's copy of the half
// it keeps (partner = lane ^ distance keeps the other). Every sum is formed by
// exactly the pairings of a full butterfly, own partial first, so the result
// is bit-identical to one, with V − 1 + log2(64 / V) exchanges instead of 6·V.
// Sum j (= r·MM + m) ends in the lanes whose bits 5, 4, ... (one per halving)
// spell j; the one with the other bits clear stores it.
template <int R, int MM, typename A>
__device__ __forceinline__ void reduce_store(float (&acc)[R][MM], int lane, int row0, const A& p) {
    constexpr int V = R * MM;
    static_assert((V & (V - 1)) == 0 && V <= 64, "R·MM must be a power of two");
    float v[V];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) v[r * MM + m] = acc[r][m];
    int j = 0;  // index of the first sum this lane still holds
#pragma unroll
    for (int c = V, off = 32; off > 0; off >>= 1) {
        if (c > 1) {
            const bool up = (lane & off) != 0;
            c >>= 1;
#pragma unroll
            for (int i = 0; i < c; ++i) {
                const float keep = up ? v[i + c] : v[i];
                const float give = up ? v[i] : v[i + c];
                v[i] = keep + xor_partner(give, off, lane);
            }
            j = 2 * j + (up ? 1 : 0);
        } else {
            v[0] += xor_partner(v[0], off, lane);
        }
    }
    constexpr int SPLITS = V == 1 ? 0 : (V == 2 ? 1 : (V == 4 ? 2 : (V == 8 ? 3 : (V == 16 ? 4 : (V == 32 ? 5 : 6)))));
    // the halving steps used lane bits 5 .. 6 − SPLITS; the store lane has the rest clear
    if ((lane & ((64 >> SPLITS) - 1)) != 0) return;
    const int r = j / MM, m = j % MM;
    const int n = row0 + r;
    if (n < p.N && m < p.M) store_y(p.y, (int64_t)m * p.ldy + n, epi_apply(p.epi, v[0], m, n), p.epi);
}

// ---- M <= 4: rows streamed whole by VALU FMAs ----
// A wave owns R weight rows and walks K in 512-wide chunks: lane l reads the
// 16 bytes at k = c·512 + 8l of each row (1 KiB contiguous per row per load
// instruction) and the matching 8 f32 activations of each of the MM rows, and
// accumulates in f32. The 64 lane partials of each output are then added by a
// fixed butterfly (deterministic). x stays f32 (the reference's f32 dot),
// except under INGOT_MATH_BF16 (split = 0), where it is rounded to bf16 once.
// CHX > 0 sets the chunks in flight per step (0: 4, or 2 for MM >= 4).
// A is GemvArgs, or PlainView (below) over the 40-byte GemvPlainArgs.
template <int R, int MM, int WPB, int CHX = 0, typename A = GemvArgs>
__global__ __launch_bounds__(64 * WPB) void gemv_rows_kernel(A p) {
    constexpr int CH = CHX ? CHX : (MM >= 4 ? 2 : 4);  // chunks in flight per step
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * WPB + wave) * R;
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
    reduce_store<R, MM>(acc, lane, row0, p);
}

template <int R, int MM, int WPB = 4, int CHX = 0, typename A = GemvArgs>
hipError_t launch_rows(const A& a, hipStream_t st) {
    const int waves = (a.N + R - 1) / R;
    hipLaunchKernelGGL((gemv_rows_kernel<R, MM, WPB, CHX, A>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0, st, a);
    return hipGetLastError();
}

// ---- M = 2..8: weight rows streamed through LDS by DMA ----
// The rows kernel holds every in-flight weight chunk, and the activations that
// go with it, in registers, which at M = 3..4 leaves one 512-k chunk per wave
// in flight. Here the weight moves global → LDS by DMA (buffer_load_dwordx4
// ... lds, no registers held while a load is in flight), D units ahead per
// wave, a unit being R weight rows × 512 k; x is staged in LDS once per
// workgroup. Each lane reads back exactly the 16 bytes it fetched, and its
// activations from the staged copy, so after the start no wave waits for
// another: it waits on its own DMA (vmcnt; loads complete in issue order).
// Persistent grid: wave g of G takes row groups g, g + G, ...; per row group
// the FMAs run in the rows kernel's order (chunk by chunk, the same sequence)
// and the same butterfly adds the lane partials, so y is bit-identical to it.
// wait_vm<V>: until at most V vector-memory operations of this wave are in
// flight (s_waitcnt vmcnt(V), the other counters unconstrained); wait_lgkm0:
// until its LDS operations have returned (lgkmcnt(0)).
template <int V>
__device__ __forceinline__ void wait_vm() {
    static_assert(V >= 0 && V < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | 0x70 | 0xF00);
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | 0x70); }

template <int R, int MM, int NW, int D, int XC>
__global__ __launch_bounds__(64 * NW) void gemv_dma_kernel(GemvArgs p) {
    constexpr int XBYTES = MM * XC * 2048;  // x: [MM][XC][2] blocks, lane l's 16 bytes at 16·l
    constexpr int UBYTES = R * 1024;         // one unit: R rows × 512 k of bf16
    static_assert(XBYTES + NW * D * UBYTES <= 160 * 1024, "LDS must fit in 160 KiB");
    static_assert(D * R < 64, "outstanding DMA must fit the 6-bit vmcnt");
    __shared__ __attribute__((aligned(1024))) char lds[XBYTES + NW * D * UBYTES];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int chunks = (int)((p.kp + 511) / 512);  // <= XC (the host checks)
    const int gw = blockIdx.x * NW + wave;
    const int GW = gridDim.x * NW;
    const int T = (p.N + R - 1) / R;  // row groups
    const int units = gw < T ? ((T - 1 - gw) / GW + 1) * chunks : 0;

    // x → LDS: block (m, c, h) holds x[m][512c + 8l + 4h .. +3] in lane l's 16 bytes
    // (zero for m >= M and past K: the host requires K % 4 == 0)
    const __amdgpu_buffer_rsrc_t rsx = make_rsrc(p.x, (uint32_t)(((int64_t)(p.M - 1) * p.ldx + p.K) * 4));
    for (int b = wave; b < MM * chunks * 2; b += NW) {
        const int h = b & 1, c = (b >> 1) % chunks, m = (b >> 1) / chunks;
        const int k = c * 512 + lane * 8 + h * 4;
        const uint32_t off = m < p.M && k + 4 <= p.K ? (uint32_t)(((int64_t)m * p.ldx + k) * 4) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsx, LDS_AS(lds + ((m * XC + c) * 2 + h) * 1024), 16, off, 0, 0, 0);
    }

    // weight units → this wave's ring of D slots; past the last unit (or past
    // kp, or row >= N) the offset is out of range and the slot fills with zeros,
    // so every unit issues exactly R loads
    const __amdgpu_buffer_rsrc_t rsw = make_rsrc(p.w, (uint32_t)((int64_t)p.N * p.ldw * 2));
    char* ring = lds + XBYTES + wave * (D * UBYTES);
    int iu = 0, it = 0, ic = 0, islot = 0;  // next unit to issue: index, row group (this wave's), chunk, slot
    auto issue = [&]() {
        const int k = ic * 512 + lane * 8;
        const bool live = iu < units && k < p.kp;
        const int row0 = (gw + it * GW) * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t off =
                live && row0 + r < p.N ? (uint32_t)(((int64_t)(row0 + r) * p.ldw + k) * 2) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, LDS_AS(ring + islot * UBYTES + r * 1024), 16, off, 0, 0, 0);
        }
        ++iu;
        if (++ic == chunks) {
            ic = 0;
            ++it;
        }
        islot = islot + 1 == D ? 0 : islot + 1;
    };
    static_assert(D >= 2, "one slot is refilled while the others are in flight");
#pragma unroll
    for (int s = 0; s < D - 1; ++s) issue();
    wait_vm<(D - 1) * R>();  // this wave's x blocks (issued before its units) have landed
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's x blocks have landed
    asm volatile("" ::: "memory");

    float acc[R][MM];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
    int ct = 0, cc = 0, cslot = 0;  // unit consumed next: row group, chunk, slot
    for (int u = 0; u < units; ++u) {
        // unit u has landed (D - 1 units in flight, in issue order), and the
        // previous unit's LDS reads have returned: its slot is refilled below
        wait_vm<(D - 2) * R>();
        wait_lgkm0();
        asm volatile("" ::: "memory");
        const char* slot = ring + cslot * UBYTES;
        i32x4_t w[R];
        f32x4_t xa[MM][2];
#pragma unroll
        for (int r = 0; r < R; ++r) w[r] = *(const i32x4_t*)(slot + r * 1024 + lane * 16);
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h) xa[m][h] = *(const f32x4_t*)(lds + ((m * XC + cc) * 2 + h) * 1024 + lane * 16);
        issue();  // unit u + D - 1 → the slot of unit u - 1
        float xv[MM][8];
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[m][e] = xa[m][e >> 2][e & 3];
        if (!p.split) {
#pragma unroll
            for (int m = 0; m < MM; ++m)
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[m][e] = bf16_to_f32(f32_to_bf16(xv[m][e]));
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t* wb = (const uint32_t*)&w[r];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = __uint_as_float(wb[e] << 16);
                const float hi = __uint_as_float(wb[e] & 0xFFFF0000u);
#pragma unroll
                for (int m = 0; m < MM; ++m) {
                    acc[r][m] = fmaf(xv[m][2 * e], lo, acc[r][m]);
                    acc[r][m] = fmaf(xv[m][2 * e + 1], hi, acc[r][m]);
                }
            }
        }
        if (++cc == chunks) {
            reduce_store<R, MM>(acc, lane, (gw + ct * GW) * R, p);
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
            cc = 0;
            ++ct;
        }
        cslot = cslot + 1 == D ? 0 : cslot + 1;
    }
    wait_vm<0>();  // the tail's zero-fill loads land before the workgroup's LDS is released
}

// What gemv_dma_kernel assumes: whole 16-byte x pieces (K % 4 == 0), rows of
// at most 12 chunks of 512 k (x staged whole in LDS), 32-bit buffer offsets,
// and the device's CU count for the persistent grid.
bool dma_ok(const GemvArgs& a) {
    return gemv_dma_fits(a.M, a.K, a.kp, a.N, a.ldw, a.ldx) && a.cus > 0;
}

template <int R, int MM, int NW, int D>
hipError_t launch_dma(const GemvArgs& a, hipStream_t st) {
    if (a.M > MM || !dma_ok(a)) return hipErrorInvalidValue;
    const int64_t chunks = (a.kp + 511) / 512;
    const int T = (a.N + R - 1) / R;
    auto go = [&](auto kern, int bytes) {
        const int occ = std::max(1, 160 * 1024 / bytes);
        const int grid = std::min((T + NW - 1) / NW, a.cus * occ);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * NW), 0, st, a);
        return hipGetLastError();
    };
    if (chunks <= 4) return go(gemv_dma_kernel<R, MM, NW, D, 4>, MM * 4 * 2048 + NW * D * R * 1024);
    // rows of 5..12 chunks: x for 8 activation rows would not fit (dma_ok sends M > 4 here only up to 4 chunks)
    if constexpr (MM * 12 * 2048 + NW * D * R * 1024 <= 160 * 1024)
        return go(gemv_dma_kernel<R, MM, NW, D, 12>, MM * 12 * 2048 + NW * D * R * 1024);
    return hipErrorInvalidValue;
}

// GemvPlainArgs seen through the members gemv_rows_kernel reads: the fixed
// parts of the plain case are compile-time constants, and its epilogue is the
// identity with an f32 store.
struct PlainEpi {};
__device__ __forceinline__ float epi_apply(const PlainEpi&, float acc, int64_t, int64_t) { return acc; }
__device__ __forceinline__ void store_y(void* y, int64_t i, float v, const PlainEpi&) { ((float*)y)[i] = v; }
struct PlainView : GemvPlainArgs {
    static constexpr int64_t ldx = 0, ldy = 0;
    static constexpr int M = 1, x_vec = 1, split = 1;
    PlainEpi epi;
};

bool gemv_plain_ok(const GemvArgs& a) {
    const Epi& e = a.epi;
    return a.M == 1 && a.x_vec && a.split && e.alpha == 1.f && e.c_mode == INGOT_C_NONE && e.act == INGOT_ACT_NONE &&
           !e.post && !e.y_bf16 && a.ldw <= INT32_MAX && a.kp <= INT32_MAX;
}

hipError_t launch_gemv_plain(const GemvArgs& a, hipStream_t st) {
    if (!gemv_plain_ok(a) || a.kp % KR != 0) return hipErrorInvalidValue;
    PlainView v = {};
    v.x = a.x;
    v.w = a.w;
    v.y = a.y;
    v.ldw = (int32_t)a.ldw;
    v.kp = (int32_t)a.kp;
    v.N = a.N;
    v.K = a.K;
    const int64_t chunks = (a.kp + 511) / 512;
    return chunks > 4 && chunks <= 12 ? launch_rows<1, 1, 4, 12, PlainView>(v, st) : launch_rows<1, 1, 4, 0, PlainView>(v, st);
}

hipError_t launch_pack_x(const float* x, int64_t ldx, int M, int K, int64_t kp, int split, uint16_t* dst,
                        hipStream_t st) {
    const int64_t chunks = kp / 32 * 64;  // 16 rows × kp / 8 elements per chunk
    hipLaunchKernelGGL(pack_x_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, x, ldx, M, K, chunks,
                       split, dst, kp * 16);
    return hipGetLastError();
}

template <int NW, int U, int RB>
hipError_t launch_mfma(const GemvArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((gemv_mfma_kernel<NW, U, RB>), dim3((a.N + RB - 1) / RB), dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

bool gemv_cfg_is_dma(int cfg) { return cfg >= 23 && cfg <= 30; }

bool gemv_dma_fits(int M, int64_t K, int64_t kp, int64_t N, int64_t ldw, int64_t ldx) {
    const int64_t chunks = (kp + 511) / 512;
    return M >= 1 && M <= 8 && K % 4 == 0 && chunks <= (M <= 4 ? 12 : 4) && N * ldw * 2 < (1ll << 31) &&
           ((int64_t)(M - 1) * ldx + K) * 4 < (1ll << 31);
}

hipError_t launch_gemv_bf16(const GemvArgs& a, int cfg, hipStream_t st) {
    if (a.kp % KR != 0 || a.M < 1 || a.M > 16) return hipErrorInvalidValue;
    // M = 5..8 with x for 8 rows staged whole (K <= 2048): no x pre-pass launch.
    // On MI355X at K = 2048, M = 8: N = 2048 6.3 instead of 9.8 µs (pre-pass
    // + MFMA kernel); N = 6144 12.2, N = 11264 20.0 µs (the runtime sends
    // N >= 4096 to the GEMM, 14.8 and 13.7 µs there, which keeps those rows
    // bit-identical to larger M).
    if (cfg == 0 && a.M >= 5 && a.M <= 8 && dma_ok(a)) return launch_dma<1, 8, 8, 4>(a, st);
    switch (cfg) {  // M <= 8, x read in place (no pre-pass)
        case 27: return launch_dma<1, 8, 8, 4>(a, st);
        case 28: return launch_dma<1, 8, 16, 3>(a, st);
        case 29: return launch_dma<1, 8, 16, 2>(a, st);
        case 30: return launch_dma<1, 8, 12, 3>(a, st);
    }
    if (a.M > 4 && !a.xb) return hipErrorInvalidValue;
    if (cfg == 0) {  // default: rows kernel for M <= 4, MFMA kernel above (measured on MI355X)
        // M = 1 with rows of 5..12 chunks of 512 k: a whole row in flight per
        // wave (one step, no dependent second round of loads); longer rows keep
        // 4 chunks per step, shorter ones fit in one step anyway. On MI355X the
        // 5632-long rows of the decode down projection took 6.1 µs instead of 6.5.
        const int64_t chunks = (a.kp + 511) / 512;
        if (a.M == 1) return chunks > 4 && chunks <= 12 ? launch_rows<1, 1, 4, 12>(a, st) : launch_rows<1, 1>(a, st);
        // M = 2..4: the weight streamed through LDS (gemv_dma_kernel). On MI355X
        // the decode step of the four GEMVs (QKV, O, gate+up, down) took
        // 33.8–35.6 instead of 43.1–43.4 µs at M = 4, 33.0–34.1 instead of 44.0
        // at M = 3 and 30.8–32.0 instead of 34.8–35.5 at M = 2 (at M = 1 it was
        // slower: 28.7 against 25.5–25.9 µs). The row kernels below remain for
        // shapes outside its preconditions.
        if (a.M <= 4 && dma_ok(a)) return a.M == 2 ? launch_dma<1, 2, 8, 4>(a, st) : launch_dma<1, 4, 8, 4>(a, st);
        if (a.M == 2) return launch_rows<1, 2>(a, st);
        // M = 3..4: one chunk in flight per step keeps these kernels at 46–54
        // VGPRs (8+ waves per SIMD: the 5632 waves of N = 11264 fit in one
        // round instead of 1.1 at 95 VGPRs); on MI355X the gate+up GEMV went from
        // 14.1 to 12.8 µs, QKV 10.1 to 9.4, the 5632-long down rows 11.0 to 10.4.
        // Short rows at N < 4096 keep two chunks per step (O: 5.7 µs, 5.9 with one).
        if (a.M <= 4)
            return a.N >= 4096 ? launch_rows<2, 4, 1, 1>(a, st)
                               : (a.kp > 4096 ? launch_rows<1, 4, 4, 1>(a, st) : launch_rows<1, 4>(a, st));
        // 16 rows per workgroup leave CUs idle below N = 4096 (N = 2048: 128
        // workgroups); 8 rows with 16 waves splitting K there (measured on MI355X)
        return a.N > 4096 ? launch_mfma<8, 4, 16>(a, st) : launch_mfma<16, 4, 8>(a, st);
    }
    if (a.M <= 4) {
        switch (cfg) {
            case 10: return launch_rows<1, 1>(a, st);
            case 11: return launch_rows<2, 1>(a, st);
            case 12: return launch_rows<4, 1>(a, st);
            case 13: return launch_rows<1, 4>(a, st);
            case 14: return launch_rows<2, 4>(a, st);
            case 15: return launch_rows<1, 2>(a, st);
            case 16: return launch_rows<4, 4, 1>(a, st);
            case 17: return launch_rows<2, 4, 1>(a, st);
            case 18: return launch_rows<4, 4, 2>(a, st);
            case 19: return launch_rows<2, 2, 1>(a, st);
            case 20: return launch_rows<1, 1, 4, 12>(a, st);
            case 21: return launch_rows<2, 4, 1, 1>(a, st);
            case 22: return launch_rows<1, 4, 4, 1>(a, st);
            case 23: return launch_dma<1, 4, 8, 4>(a, st);
            case 24: return launch_dma<1, 2, 8, 4>(a, st);
            case 25: return launch_dma<1, 1, 8, 4>(a, st);
            case 26: return launch_dma<2, 4, 8, 3>(a, st);
        }
        return hipErrorInvalidValue;
    }
    switch (cfg) {
        case 1: return launch_mfma<8, 8, 16>(a, st);
        case 2: return launch_mfma<8, 4, 8>(a, st);
        case 3: return launch_mfma<4, 8, 8>(a, st);
        case 4: return launch_mfma<4, 4, 8>(a, st);
        case 5: return launch_mfma<16, 4, 8>(a, st);
        case 6: return launch_mfma<8, 4, 16>(a, st);
        case 7: return launch_mfma<4, 8, 16>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace ingot
