// k_gemm_tn_pro.hip -- instantiates the MFMA GEMM for layout TN, dB = A^T.dC (A stored [K][M], B[K][N]),
// with the activation-derivative prologue on the dC operand (ReLU and GELU).
// Kept in its own translation unit so it compiles in parallel with the
// plain instances.
#include "fg_gemm_kernel.h"

namespace fg {
namespace gemm {

void launch_tn_pro(const GemmArgs &a, bool vec, bool pipe, int cfg, int pro, hipStream_t st) {
    if (pro == kProBReLU)
        launch_layout<false, true, kProBReLU>(a, vec, pipe, false, cfg, st);
    else
        launch_layout<false, true, kProBGelu>(a, vec, pipe, false, cfg, st);
}

}  // namespace gemm
}  // namespace fg
