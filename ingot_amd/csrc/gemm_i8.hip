// Tile configurations of the int8 (MatMulInteger, QLinearMatMul, QLinearConv) MFMA GEMM (indices of its gemm_configs table).

#include "gemm_mfma.hpp"

namespace ingot {

hipError_t launch_gemm_i8(int cfg, const GemmArgs& a, int batch, hipStream_t st) {
    switch (cfg) {
        case 0: return launch_one<KIND_I8, 256, 256, 2, 4, 2>(a, batch, st);
        case 1: return launch_one<KIND_I8, 128, 128, 2, 2, 2>(a, batch, st);
        case 2: return launch_one<KIND_I8, 128, 64, 2, 2, 2>(a, batch, st);
        case 3: return launch_one<KIND_I8, 64, 64, 2, 2, 2>(a, batch, st);
        case 4: return launch_one<KIND_I8, 64, 96, 2, 2, 2>(a, batch, st);
        case 5: return launch_one<KIND_I8, 32, 32, 2, 2, 4>(a, batch, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace ingot
