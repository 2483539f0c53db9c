// QLinearConv on gfx950 (reference: qlinearConvOp.Run, ops/quant.go:343-420).
//
// Two routes, both exact in int32 and requantised with the reference's
// expression (vek.RequantU8/I8, kernels/vek/quant_amd64.go:52-70):
//  * im2col → int8 GEMM: qim2col_kernel writes, per group, the byte column
//    matrix col[row = image·P + pixel][k = (c, kh, kw)] of the raw activations
//    (u8 or s8, taps outside the image hold the zero point zx, k past the
//    group's K zero) in whole 128-byte k-tiles, the A operand of the int8 MFMA
//    GEMM; its epilogue adds −zx′·ΣW + bias per output channel, requantises
//    with that channel's multiplier and stores the NCHW planes. The
//    reference's pointwise and im2colTiled paths (:612-673) are this route.
//  * direct: one thread per output element sums w·(x − zx) over the taps
//    inside the image (padded taps contribute exactly 0). Used for depthwise
//    and narrow groups, where a GEMM would be a sliver (the reference's
//    depthwise path, :472-598).
#include <hip/hip_runtime.h>

#include "kernels.hpp"

#pragma clang fp contract(off)

namespace ingot {

namespace {

__device__ __forceinline__ uint8_t requant_byte(int32_t v, float mult, float zy, int u8) {
    // float32(v)·mult and + zy rounded separately, half to even, saturate
    const float t = (float)v * mult;
    const float r = rintf(t + zy);
    const int iv = u8 ? (r <= 0.f ? 0 : (r >= 255.f ? 255 : (int)r))
                      : (r <= -128.f ? -128 : (r >= 127.f ? 127 : (int)r));
    return (uint8_t)iv;
}

// One thread writes 16 consecutive k of one row (a 16-byte store); a row is
// kgl / 16 threads. blockIdx.y is the group.
__global__ void __launch_bounds__(256) qim2col_kernel(const uint8_t* __restrict__ x, QconvGeom g, int rows,
                                                      int kg, int kgl, uint8_t pad, uint8_t* __restrict__ col,
                                                      int64_t col_group) {
    const int chunks = kgl >> 4;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)rows * chunks) return;
    const int r = (int)(t / chunks);
    const int ch = (int)(t - (int64_t)r * chunks);
    const int P = g.OH * g.OW;
    const int img = r / P;
    const int pix = r - img * P;
    const int oh = pix / g.OW, ow = pix - (pix / g.OW) * g.OW;
    const int grp = blockIdx.y;
    const int64_t hw = (int64_t)g.H * g.W;
    const uint8_t* xb = x + ((int64_t)img * g.C + (int64_t)grp * g.Cg) * hw;
    const int taps = g.KH * g.KW;
    int k = ch << 4;
    int cg = k / taps;
    int rem = k - cg * taps;
    int kh = rem / g.KW;
    int kw = rem - kh * g.KW;
    const int ih0 = oh * g.sh - g.pt, iw0 = ow * g.sw - g.pl;
    uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        uint32_t b = 0;
        if (k + i < kg) {
            const int ih = ih0 + kh * g.dh, iw = iw0 + kw * g.dw;
            b = (ih >= 0 && ih < g.H && iw >= 0 && iw < g.W) ? xb[(int64_t)cg * hw + (int64_t)ih * g.W + iw] : pad;
            if (++kw == g.KW) {
                kw = 0;
                if (++kh == g.KH) {
                    kh = 0;
                    ++cg;
                }
            }
        }
        words[i >> 2] |= b << (8 * (i & 3));
    }
    uint8_t* dst = col + (int64_t)grp * col_group + (int64_t)r * kgl + (ch << 4);
    *(uint4*)dst = make_uint4(words[0], words[1], words[2], words[3]);
}

// y[n][m][oh][ow] = requant(Σ w[m][cg][kh][kw]·(x − zx) + bias[m]); w rows are
// ldw bytes apart (the packed int8 weight). Grid-stride over all outputs.
__global__ void __launch_bounds__(256) qconv_direct_kernel(const uint8_t* __restrict__ x, int x_u8, QconvGeom g,
                                                           const int8_t* __restrict__ w, int64_t ldw,
                                                           const int32_t* __restrict__ bias,
                                                           const float* __restrict__ mult, int32_t zx, float zy,
                                                           int y_u8, uint8_t* __restrict__ y, int64_t total) {
    const int64_t hw = (int64_t)g.H * g.W;
    const int Mg = g.M / g.G;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (int64_t)gridDim.x * blockDim.x) {
        const int ow = (int)(o % g.OW);
        int64_t t = o / g.OW;
        const int oh = (int)(t % g.OH);
        t /= g.OH;
        const int m = (int)(t % g.M);
        const int img = (int)(t / g.M);
        const int grp = m / Mg;
        const int8_t* wr = w + (int64_t)m * ldw;
        const uint8_t* xb = x + ((int64_t)img * g.C + (int64_t)grp * g.Cg) * hw;
        uint32_t acc = bias ? (uint32_t)bias[m] : 0u;
        const int ih0 = oh * g.sh - g.pt, iw0 = ow * g.sw - g.pl;
        for (int cg = 0; cg < g.Cg; ++cg) {
            const uint8_t* xc = xb + (int64_t)cg * hw;
            const int8_t* wc = wr + cg * g.KH * g.KW;
            for (int kh = 0; kh < g.KH; ++kh) {
                const int ih = ih0 + kh * g.dh;
                if (ih < 0 || ih >= g.H) continue;
                for (int kw = 0; kw < g.KW; ++kw) {
                    const int iw = iw0 + kw * g.dw;
                    if (iw < 0 || iw >= g.W) continue;
                    const uint8_t b = xc[(int64_t)ih * g.W + iw];
                    const int32_t xv = x_u8 ? (int32_t)b : (int32_t)(int8_t)b;
                    acc += (uint32_t)((xv - zx) * (int32_t)wc[kh * g.KW + kw]);
                }
            }
        }
        y[o] = requant_byte((int32_t)acc, mult[m], zy, y_u8);
    }
}

}  // namespace

hipError_t launch_qim2col(const void* x, const QconvGeom& g, int rows, int kg, int kgl, uint8_t pad, void* col,
                          int64_t col_group, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int64_t threads = (int64_t)rows * (kgl / 16);
    const int64_t blocks = (threads + 255) / 256;
    hipLaunchKernelGGL(qim2col_kernel, dim3((unsigned)blocks, (unsigned)g.G), dim3(256), 0, st, (const uint8_t*)x, g,
                       rows, kg, kgl, pad, (uint8_t*)col, col_group);
    return hipGetLastError();
}

hipError_t launch_qconv_direct(const void* x, int x_u8, const QconvGeom& g, const int8_t* w, int64_t ldw,
                               const int32_t* bias, const float* mult, int32_t zx, float zy, int y_u8, void* y,
                               hipStream_t st) {
    const int64_t total = (int64_t)g.N * g.M * g.OH * g.OW;
    if (total <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 16384);
    hipLaunchKernelGGL(qconv_direct_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)x, x_u8, g, w,
                       ldw, bias, mult, zx, zy, y_u8, (uint8_t*)y, total);
    return hipGetLastError();
}

}  // namespace ingot
