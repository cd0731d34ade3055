// k_gemm_skinny.hip -- launches of the skinny GEMM kernel (fg_gemm_skinny.h).
#include "fg_gemm_skinny.h"

namespace fg {
namespace gemm {
namespace {

template <bool AK, bool BNC>
__global__ __launch_bounds__(kSkThreads) void gemm_f32_skinny(GemmArgs p) {
    gemm_f32_skinny_body<AK, BNC>(p, blockIdx.x);
}

}  // namespace

void launch_skinny(const GemmArgs &a, int layout, hipStream_t st) {
    const dim3 grid(skinny_workgroups(a.M)), block(kSkThreads);
    switch (layout) {
        case 0: gemm_f32_skinny<true, true><<<grid, block, 0, st>>>(a); break;   // NN
        case 1: gemm_f32_skinny<true, false><<<grid, block, 0, st>>>(a); break;  // NT
        default: gemm_f32_skinny<false, true><<<grid, block, 0, st>>>(a); break;  // TN
    }
}

}  // namespace gemm
}  // namespace fg
