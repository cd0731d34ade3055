// k_gemm16_bf16.hip -- instantiates the 16-bit MFMA GEMM for bf16 storage, all
// three layouts (NN forward, NT dA, TN dB).  One translation unit per type
// so the two compile in parallel.
#include "fg_gemm16_kernel.h"
#include "fg_internal.h"

namespace fg {
namespace gemm16 {

void launch_bf16(int layout, const Args &a, bool vec, bool pipe, int cfg, hipStream_t st) {
    switch (layout) {
        case FG_NN: launch_layout<true, true, true>(a, vec, pipe, cfg, st); break;
        case FG_NT: launch_layout<true, false, true>(a, vec, pipe, cfg, st); break;
        default: launch_layout<false, true, true>(a, vec, pipe, cfg, st); break;
    }
}

void launch_pair_bf16(const Args &a1, const Args &a2, hipStream_t st) {
    launch_pair16<true>(a1, a2, st);
}

}  // namespace gemm16
}  // namespace fg
