// k_gemm_nt_pro.hip -- instantiates the MFMA GEMM for layout NT, dA = dC.B^T (A[M][K], B stored [N][K]),
// with the activation-derivative prologue on the dC operand (ReLU and GELU).
// Kept in its own translation unit so it compiles in parallel with the
// plain instances.
#include "fg_gemm_kernel.h"

namespace fg {
namespace gemm {

void launch_nt_pro(const GemmArgs &a, bool vec, bool pipe, int cfg, int pro, hipStream_t st) {
    if (pro == kProAReLU)
        launch_layout<true, false, kProAReLU>(a, vec, pipe, false, cfg, st);
    else
        launch_layout<true, false, kProAGelu>(a, vec, pipe, false, cfg, st);
}

}  // namespace gemm
}  // namespace fg
