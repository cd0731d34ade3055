// k_gemm_nt.hip -- instantiates the MFMA GEMM for layout NT: dA = dC.B^T (A[M][K], B stored [N][K]).
// Kept in its own translation unit so the three layouts compile in parallel.
#include "fg_gemm_kernel.h"

namespace fg {
namespace gemm {

void launch_nt(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, int pro,
               hipStream_t st) {
    if (pro == kProNone)
        launch_layout<true, false, kProNone>(a, vec, pipe, ktail, cfg, st);
    else
        launch_nt_pro(a, vec, pipe, cfg, pro, st);
}

}  // namespace gemm
}  // namespace fg
