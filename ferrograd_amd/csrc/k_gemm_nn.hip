// k_gemm_nn.hip -- instantiates the MFMA GEMM for layout NN: forward C = A.B (A[M][K], B[K][N]).
// Kept in its own translation unit so the three layouts compile in parallel.
#include "fg_gemm_kernel.h"

namespace fg {
namespace gemm {

void launch_nn(const GemmArgs &a, bool vec, bool pipe, bool ktail, int cfg, hipStream_t st) {
    launch_layout<true, true, kProNone>(a, vec, pipe, ktail, cfg, st);
}

}  // namespace gemm
}  // namespace fg
