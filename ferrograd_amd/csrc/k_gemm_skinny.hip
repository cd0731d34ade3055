// k_gemm_skinny.hip -- launches of the skinny GEMM kernel (fg_gemm_skinny.h).
#include "fg_gemm_skinny.h"

namespace fg {
namespace gemm {
namespace {

template <bool AK, bool BNC>
__global__ __launch_bounds__(kSkThreads) void gemm_f32_skinny(GemmArgs p) {
    gemm_f32_skinny_body<AK, BNC>(p, blockIdx.x);
}

// NN, A summed from the slices of the split GEMM `pre`.
__global__ __launch_bounds__(kSkThreads) void gemm_f32_skinny_pre(GemmArgs p, GemmArgs pre) {
    gemm_f32_skinny_pre_body<false>(p, pre, blockIdx.x, CeOut{});
}

// The same, finishing the softmax + CE of the head's rows.
__global__ __launch_bounds__(kSkThreads) void gemm_f32_skinny_pre_ce(GemmArgs p, GemmArgs pre,
                                                                     CeOut ce) {
    gemm_f32_skinny_pre_body<true>(p, pre, blockIdx.x, ce);
}

}  // namespace

void launch_skinny_pre(const GemmArgs &a, const GemmArgs &pre, hipStream_t st,
                       const CeOut *ce) {
    const dim3 grid(skinny_pre_workgroups(a.M)), block(kSkThreads);
    if (ce)
        gemm_f32_skinny_pre_ce<<<grid, block, 0, st>>>(a, pre, *ce);
    else
        gemm_f32_skinny_pre<<<grid, block, 0, st>>>(a, pre);
}

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
