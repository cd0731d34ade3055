// k_gemm_tn.hip -- instantiates the MFMA GEMM for layout TN: dB = A^T.dC (A stored [K][M], B[K][N]).
// Kept in its own translation unit so the three layouts compile in parallel.
#include "fg_gemm_kernel.h"

namespace fg {
namespace gemm {

void launch_tn(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, int pro,
               hipStream_t st) {
    if (pro == kProNone)
        launch_layout<false, true, kProNone>(a, vec, pipe, ktail, cfg, st);
    else
        launch_tn_pro(a, vec, pipe, cfg, pro, st);
}

}  // namespace gemm
}  // namespace fg
