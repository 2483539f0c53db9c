// Tile configuration tables and dispatch of the MFMA GEMM (the kernel itself
// is in gemm_mfma.hpp; each kind's instances are in their own source file).

#include "gemm_mfma.hpp"

namespace ingot {

namespace {

// Tile configurations per kind. occupancy: workgroups per CU the LDS and
// register footprint allow; eff: relative throughput per CU slot (measured
// on MI355X for the bf16 kernel).
// Small tiles mostly keep two LDS stages: with several tiles per CU, occupancy
// (more resident workgroups) hides latency better than a deeper ring. With one
// tile per CU or fewer (small M, or few columns) each k-tile waits for its own
// DMA round trip instead, and a four-stage ring pays: the 32×32 and 64×64
// four-stage entries (bf16 and bf16 hi/lo), measured on MI355X with bf16
// weights at K = 2048: M = 17–128 × N = 2048–6144 6.5–6.8 µs with 32×32
// (10.7–11.3 with two-stage 64×64; the hi/lo kind 11.0 vs 35 with 128×128),
// M = 64 × N = 11264 and M = 256 × N = 6144 11.1 and 15.4 µs with 64×64
// (18.1 and 18.5 with two stages). Their weights keep the DiT shapes on the
// large tiles, and they are taken only when every tile is resident at once.
// Entry 9 is entry 1 with the weight staged through registers (gemm_kernel's
// RS = 2): every load issued two k-tiles ahead instead of one. On MI355X, the
// DiT MLP-down (M = 4096, N = 3072, K = 12288) right after the MLP-up GEMM
// (whose 201 MB of output fill the Infinity Cache) took 253–257 µs instead of
// 293–294, and after a 1 GiB fill 241 instead of 310; with its operands
// already cached it is 8–12% slower (249 vs 230 µs), so the runtime takes it
// only for products whose operands are too large to stay cached.
// bf16 64×96: at M = 1024, K = 768 (the BERT-size FFN-up and QKV products) two tiles per CU
// instead of three 64×64 ones: 11.4 vs 12.0–13.1 µs at N = 3072, 10.1 vs 11.5 µs at N = 2304 on
// MI355X; slower at N = 768 (fewer tiles than CUs), where the weight keeps 64×64 ahead.
const GemmConfig kBF16Cfgs[] = {{256, 256, 1, 1.00f}, {256, 192, 1, 0.95f, false, 9}, {128, 128, 2, 0.80f}, {128, 64, 3, 0.78f},
                                {64, 64, 4, 0.65f},   {192, 256, 1, 0.95f}, {64, 96, 3, 0.72f}, {32, 32, 4, 0.60f, true},
                                {64, 64, 2, 1.00f, true}, {256, 192, 1, 0.f}};
// f32 32×96: on MI355X 15% faster than 64×64 over the BERT projections (M = 1024;
// N = 768 gives exactly 256 tiles), slightly slower on ties, so weighted 0.97.
// 64×96, 64×128, 96×64, 32×128 and 64×192 were no faster on any of them.
// f32 32×32, four-stage ring: for products with few tiles. The configs[0] Gemm
// (M = 128, N = 512, K = 256) runs 64 of them instead of 24 32×96 ones: 3.8 vs
// 6.2 µs per call on MI355X; at M = 32, N = 6144, K = 2048 (64 k-tiles) the ring
// depth matters: 14.2 µs with four stages, 26.8 with two. 6–12% slower than 32×96
// on the BERT projections, so weighted 0.8.
// f32 32×96 with a four-stage ring, when every tile is resident at once (one
// per CU): the BERT FFN-down (M = 1024, N = 768, K = 3072, 96 k-tiles, one
// wave per SIMD, so nothing else covers a k-tile's DMA round trip) took 41.6
// instead of 45.0 µs on MI355X; at three tiles per CU the two-stage ring stays
// ahead (FFN-up 41.3 vs 43.7), and six stages were slower again (42.1).
const GemmConfig kF32Cfgs[] = {{128, 128, 2, 0.90f}, {128, 64, 3, 0.95f}, {64, 64, 4, 1.00f}, {32, 96, 4, 0.97f},
                               {32, 32, 4, 0.80f},   {32, 96, 2, 0.98f, true}};
// int8 64×96: two tiles per CU at M = 1024, N = 3072 (512 tiles) instead of three 64×64 ones:
// 9.0 vs 9.6 µs on MI355X (fewer panel re-reads through L2); 128×96, 32×96, 64×128,
// 64×192, 32-row tiles (32×32 to 32×128) and deeper rings were slower there.
// int8 32×32 with a four-stage ring, for products whose tiles are all resident
// at once: M = 1–128 at K = 768–2048 took 3.8–5.3 µs instead of 4.7–6.9.
const GemmConfig kI8Cfgs[] = {{256, 256, 1, 1.00f}, {128, 128, 2, 0.60f}, {128, 64, 3, 0.70f}, {64, 64, 4, 1.00f},
                              {64, 96, 3, 1.06f}, {32, 32, 4, 0.60f, true}};

}  // namespace

int gemm_configs(GemmKind kind, const GemmConfig** out) {
    switch (kind) {
        case KIND_BF16: *out = kBF16Cfgs; return (int)(sizeof(kBF16Cfgs) / sizeof(kBF16Cfgs[0]));
        case KIND_F32: *out = kF32Cfgs; return (int)(sizeof(kF32Cfgs) / sizeof(kF32Cfgs[0]));
        case KIND_I8: *out = kI8Cfgs; return (int)(sizeof(kI8Cfgs) / sizeof(kI8Cfgs[0]));
        // the hi/lo kind uses the bf16 kind's tiles (see gemm_kernel for how it runs on them)
        case KIND_BF16X2: *out = kBF16Cfgs; return (int)(sizeof(kBF16Cfgs) / sizeof(kBF16Cfgs[0]));
        default: break;
    }
    return 0;
}

hipError_t launch_gemm(GemmKind kind, int cfg, const GemmArgs& a, int batch, hipStream_t st) {
    switch (kind) {
        case KIND_BF16: return launch_gemm_bf16(cfg, a, batch, st);
        case KIND_BF16X2: return launch_gemm_bf16x2(cfg, a, batch, st);
        case KIND_F32: return launch_gemm_f32(cfg, a, batch, st);
        case KIND_I8: return launch_gemm_i8(cfg, a, batch, st);
        default: break;
    }
    return hipErrorInvalidValue;
}

}  // namespace ingot
