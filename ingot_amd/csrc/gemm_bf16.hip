// Tile configurations of the bf16 (bf16 activations × bf16 weights) MFMA GEMM (indices of its gemm_configs table).

#include "gemm_mfma.hpp"

namespace ingot {

hipError_t launch_gemm_bf16(int cfg, const GemmArgs& a, int batch, hipStream_t st) {
    switch (cfg) {
        case 0: return launch_one<KIND_BF16, 256, 256, 4, 2, 2>(a, batch, st);
        // 8 waves as 4×2 (64×96 per wave): fewer LDS fragment bytes per
        // MFMA than 2×4 (128×48); 3–6% faster on the DiT QKV (MI355X)
        case 1: return launch_one<KIND_BF16, 256, 192, 4, 2, 2>(a, batch, st);
        case 2: return launch_one<KIND_BF16, 128, 128, 2, 2, 2>(a, batch, st);
        case 3: return launch_one<KIND_BF16, 128, 64, 2, 2, 2>(a, batch, st);
        case 4: return launch_one<KIND_BF16, 64, 64, 2, 2, 2>(a, batch, st);
        case 5: return launch_one<KIND_BF16, 192, 256, 2, 4, 2>(a, batch, st);
        case 6: return launch_one<KIND_BF16, 64, 96, 2, 2, 2>(a, batch, st);
        case 7: return launch_one<KIND_BF16, 32, 32, 2, 2, 4>(a, batch, st);
        case 8: return launch_one<KIND_BF16, 64, 64, 2, 2, 4>(a, batch, st);
        // 256×192 with the weight staged through registers: every load two k-tiles ahead
        case 9: return launch_one<KIND_BF16, 256, 192, 4, 2, 2, 2>(a, batch, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace ingot
