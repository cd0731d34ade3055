// k_gemm16_f16.hip -- instantiates the 16-bit MFMA GEMM for f16 storage, all
// three layouts (NN forward, NT dA, TN dB).  One translation unit per type
// so the two compile in parallel.
#include "fg_gemm16_kernel.h"
#include "fg_internal.h"

namespace fg {
namespace gemm16 {

void launch_f16(int layout, const Args &a, bool vec, bool pipe, int cfg, hipStream_t st) {
    switch (layout) {
        case FG_NN: launch_layout<true, true, false>(a, vec, pipe, cfg, st); break;
        case FG_NT: launch_layout<true, false, false>(a, vec, pipe, cfg, st); break;
        default: launch_layout<false, true, false>(a, vec, pipe, cfg, st); break;
    }
}

void launch_pair_f16(const Args &a1, const Args &a2, hipStream_t st) {
    launch_pair16<false>(a1, a2, st);
}

}  // namespace gemm16
}  // namespace fg
