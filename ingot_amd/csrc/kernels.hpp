// Internal launch interface between the runtime (runtime.cpp) and the gfx950
// kernels (gemm_mfma.hpp and its per-kind units, gemv_bf16.hip, elementwise.hip).
#pragma once

#include "common.hpp"

namespace ingot {

// Element kind of a packed GEMM operand pair (A and B share it).
// KIND_BF16X2: f32 activations carried as two bf16 planes (hi = bf16(a),
// lo = bf16(a − hi)) against bf16 weights; two MFMAs per step keep the
// activation error at ~2⁻¹⁷ relative (f32-class), where KIND_BF16 rounds
// the activations once (~2⁻⁹).
// KIND_I8G: int8 weights with one f32 scale per 64 k of a row (decode GEMV only).
enum GemmKind { KIND_BF16 = 0, KIND_F32 = 1, KIND_I8 = 2, KIND_BF16X2 = 3, KIND_I8G = 4 };

// Every kernel row of A and B is read in 128-byte k-tiles: 64 bf16, 32 f32 or
// 128 int8 elements. Packed operands are zero padded to whole k-tiles.
constexpr int KTILE_BYTES = 128;

// The operand and tile description every GEMM launch shares.
struct GemmCore {
    const char* a;       // A rows [M][...] (row pitch lda_bytes), k-contiguous
    int64_t lda_bytes;
    const char* b;       // packed weight [b_rows][...] (row pitch ldb_bytes)
    int64_t ldb_bytes;
    int M, N;
    int kt;              // number of 128-byte k-tiles to reduce over
    int b_rows;          // allocated rows of b (loads clamp to it)
    int tiles_m, tiles_n;
    int64_t stride_a_bytes;  // per blockIdx.y batch item
    int64_t stride_b_bytes;  // per blockIdx.y batch item (0: one weight for all)
    int64_t stride_y;        // elements, per batch item
    int a_xor;               // int8: flip the sign bit of A bytes (u8 → s8)
    int64_t a_plane_bytes;   // KIND_BF16X2: offset of the lo plane from the hi plane
    uint32_t a_bytes;        // extent of one batch item's A (all planes): loads past it return 0
    uint32_t b_bytes;        // extent of the packed weight
    void* y;
    int64_t ldy;
};

// What the host fills; a launch passes the kernel only the epilogue its kind
// reads (GemmArgsF or GemmArgsQ): the host cost of a launch grows with the
// size of its arguments.
struct GemmArgs : GemmCore {
    Epi epi;
    QEpi qepi;
};
struct GemmArgsF : GemmCore {
    Epi epi;
};
struct GemmArgsQ : GemmCore {
    QEpi qepi;
};

struct GemmConfig {
    int bm, bn;
    int occupancy;   // workgroups per CU the tile allows (eff 0: never picked by itself)
    float eff;       // relative per-CU efficiency (tile-size heuristic)
    bool one_round;  // only when every tile is resident at once (a latency-bound shape)
    int deep = -1;   // index of the same tile with loads issued two k-tiles ahead (operands from HBM)
};

// Tile configurations compiled for `kind`; index used by launch_gemm.
int gemm_configs(GemmKind kind, const GemmConfig** out);
hipError_t launch_gemm(GemmKind kind, int cfg, const GemmArgs& a, int batch, hipStream_t st);

struct GemvArgs {
    const float* x;
    int64_t ldx;
    int M, K;
    int x_vec;           // x rows 16-byte aligned (vector loads allowed)
    const uint16_t* w;   // packed bf16 [>= 16·ceil(N/16)][ldw]
    int64_t ldw;
    int64_t kp;          // padded K (multiple of 256)
    int N;
    int split;           // 1: x as bf16 hi + lo (f32-class); 0: x rounded to bf16 once
    // M > 4: x pre-packed by launch_pack_x as bf16 planes in MFMA fragment
    // order (16 rows, zero padded; hi, then lo at +xb_plane when split).
    const uint16_t* xb;
    int64_t xb_plane;
    Epi epi;
    void* y;  // f32 or bf16 per epi.y_bf16
    int64_t ldy;
    int cus;  // compute units of the device (sizes persistent grids; not read by kernels)
};
// cfg selects (waves per workgroup, 16-byte chunks per lane per round).
hipError_t launch_gemv_bf16(const GemvArgs& a, int cfg, hipStream_t st);
// Whether the LDS-DMA GEMV can take these operands (x staged whole in LDS:
// M <= 4 with rows up to 6144 k, M = 5..8 up to 2048 k; K % 4 == 0; 32-bit
// buffer offsets). At cfg 0 it serves M = 2..8, without the x pre-pass.
bool gemv_dma_fits(int M, int64_t K, int64_t kp, int64_t N, int64_t ldw, int64_t ldx);
// Forced configurations (INGOT_GEMV_CFG) of the LDS-DMA GEMV.
bool gemv_cfg_is_dma(int cfg);
// The common decode case in a small argument block (the host cost of a launch
// grows with the argument size; these 40 bytes launch as 48, against 152 for
// GemvArgs): M = 1, f32 x 16-byte aligned, f32-class math (split), y = x·Wᵀ
// stored as f32 with no epilogue. The caller checks gemv_plain_ok.
struct GemvPlainArgs {
    const float* x;
    const uint16_t* w;
    void* y;
    int32_t ldw, kp, N, K;
};
bool gemv_plain_ok(const GemvArgs& a);
hipError_t launch_gemv_plain(const GemvArgs& a, hipStream_t st);
// x (f32 [M <= 16][ldx]) → the fragment-ordered bf16 planes the M > 4 GEMV
// reads: dst holds (split ? 2 : 1) planes of 16·kp elements.
hipError_t launch_pack_x(const float* x, int64_t ldx, int M, int K, int64_t kp, int split, uint16_t* dst,
                         hipStream_t st);

// Grouped-int8 decode GEMV (gemv_i8g.hip).
struct I8gArgs {
    const int8_t* q;   // weight [>= N][ldk], int8
    const float* sw;   // weight scales [>= N][kp / 64]
    int64_t ldk, kp;
    int N, M;          // M <= 4 rows per launch
    const int8_t* xh;  // activation planes [M][kp] (launch_quantize_x16)
    const int8_t* xl;
    const float* sx;   // [M][kp / 64]
    Epi epi;
    void* y;  // f32 or bf16 per epi.y_bf16
    int64_t ldy;
};
// Quantises a weight (f32 or bf16 bits; trans = 1: [n][k] rows, 0: [k][n])
// to int8 q[np][ldk] and f32 scales[np][kp / 64] (zero padded).
hipError_t launch_quantize_i8g(const void* src, int src_dtype, int64_t ld, int trans, int64_t n, int64_t k, int8_t* q,
                               float* scales, int64_t np, int64_t kp, int64_t ldk, hipStream_t st);
// Splits x (f32 [M][ldx]) into xh, xl ([M][kp] int8) and sx ([M][kp / 64]).
hipError_t launch_quantize_x16(const float* x, int64_t ldx, int M, int64_t K, int64_t kp, int8_t* xh, int8_t* xl,
                               float* sx, hipStream_t st);
// cfg: weight rows per wave (0: chosen from N).
hipError_t launch_gemv_i8g(const I8gArgs& a, int cfg, hipStream_t st);

// Packs a weight into [np][kp] of dst_kind, zero padded. src_dtype is an
// INGOT_DT_* code; trans = 1: src is [n][k] (row pitch ld), 0: src is [k][n].
// Rows of dst are ldk elements apart (ldk >= kp).
// items > 1 packs that many matrices, src_item / dst_item elements apart.
hipError_t launch_pack_weight(const void* src, int src_dtype, int64_t ld, int trans, int64_t n, int64_t k,
                              void* dst, GemmKind dst_kind, int64_t np, int64_t kp, int64_t ldk, hipStream_t st,
                              int items = 1, int64_t src_item = 0, int64_t dst_item = 0);
// colsum[j] = Σ_k packed[j][k] over an int8 packed weight (row pitch ldk).
hipError_t launch_colsum_i8(const int8_t* packed, int64_t kp, int64_t ldk, int64_t n, int32_t* colsum,
                            hipStream_t st);
// Packs activations A[M][K] (or [K][M] when trans) into [M][kl] of dst_kind
// (kl = whole k-tiles), batch items at src_stride / dst_stride elements.
hipError_t launch_pack_a(const void* src, int src_dtype, int64_t lda, int trans, int64_t m, int64_t k,
                         int64_t src_stride, void* dst, GemmKind dst_kind, int64_t kl, int64_t dst_stride, int batch,
                         hipStream_t st);
// QLinearConv geometry (qconv.hip): x [N][C][H][W], weight [M][Cg][KH][KW],
// G groups (C = G·Cg), resolved top/left pads, output [N][M][OH][OW].
struct QconvGeom {
    int N, C, H, W, M, G, Cg, KH, KW, sh, sw, dh, dw, pt, pl, OH, OW;
};
// col[grp][row][kgl] bytes for rows = images·OH·OW of x (grid y = G): the raw
// x bytes of tap k = (c, kh, kw), pad outside the image, 0 for k >= kg.
// Groups are col_group bytes apart; kgl is a multiple of 16.
hipError_t launch_qim2col(const void* x, const QconvGeom& g, int rows, int kg, int kgl, uint8_t pad, void* col,
                          int64_t col_group, hipStream_t st);
// Direct QLinearConv of every output element (weight rows ldw bytes apart).
hipError_t launch_qconv_direct(const void* x, int x_u8, const QconvGeom& g, const int8_t* w, int64_t ldw,
                               const int32_t* bias, const float* mult, int32_t zx, float zy, int y_u8, void* y,
                               hipStream_t st);
hipError_t launch_dequant(const void* x, int x_dtype, int64_t n, const float* scale, int64_t n_scale, int64_t inner,
                          const void* zp, int zp_dtype, int64_t n_zp, float* y, hipStream_t st);
hipError_t launch_activation(const float* x, float* y, int64_t rows, int64_t cols, const float* bias, int act,
                             float a, float b, int post, float ps, float pb, hipStream_t st);
hipError_t launch_cast_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t st);
hipError_t launch_fill(void* dst, int value, size_t bytes, hipStream_t st);

}  // namespace ingot
