// k_gemm_pair.hip -- a layer's two gradient GEMMs in one launch.  dW = X^T.dZ
// (TN, with the fused bias gradient) and dX = (dZ.W^T) * act'(Z) (NT) read
// the same dZ and write different tensors, so neither waits for the other.
// On a latency-bound step (c1: every kernel a few microseconds, dispatches
// back to back) launching them separately costs one whole dispatch; here the
// first n1 workgroups run the dW body and the rest the dX body, each exactly
// as its own kernel would (same tile walk, same K slices, same bits).  The
// small 256-thread kernels pair with each other (the skinny kernel and the
// 64x64 tiles, element loads or pipelined); the pipelined 128x64 tiles and
// the large layers' 8-wave tiles each pair with their own kind.
#include "fg_gemm_skinny.h"

namespace fg {
namespace gemm {
namespace {

template <bool AK, bool BNC>
struct PkSkinny {
    __device__ static void run(const GemmArgs &p, int bx, int) {
        gemm_f32_skinny_body<AK, BNC>(p, bx);
    }
};
template <bool AK, bool BNC>
struct PkElem {  // 64x64, element loads (gemm_f32_mfma, VEC false)
    __device__ static void run(const GemmArgs &p, int bx, int by) {
        gemm_f32_mfma_body<64, 64, 16, 2, 2, AK, BNC, false, kProNone>(p, bx, by);
    }
};
template <bool AK, bool BNC>
struct PkPipe {  // 64x64, pipelined whole K tiles
    __device__ static void run(const GemmArgs &p, int bx, int by) {
        gemm_f32_pipe_body<64, 64, 16, 2, 2, AK, BNC, kProNone, false>(p, bx, by);
    }
};

// Workgroup w < n1: GEMM 1 at (w % x1, w / x1); else GEMM 2 at
// (v % x2, v / x2) with v = w - n1 (x: output tiles, the quotient: K slice).
template <class G1, class G2>
__global__ __launch_bounds__(256) void gemm_pair(GemmArgs a1, GemmArgs a2, int x1, int n1,
                                                 int x2) {
    const int w = blockIdx.x;
    if (w < n1) {
        G1::run(a1, w % x1, w / x1);
    } else {
        const int v = w - n1;
        G2::run(a2, v % x2, v / x2);
    }
}

template <class G1>
void launch_with(int k2, const GemmArgs &a1, const GemmArgs &a2, int x1, int n1, int x2, int n2,
                 hipStream_t st) {
    const dim3 grid(n1 + n2), block(256);
    switch (k2) {  // GEMM 2 is the NT data gradient
        case kPairSkinny:
            gemm_pair<G1, PkSkinny<true, false>><<<grid, block, 0, st>>>(a1, a2, x1, n1, x2);
            break;
        case kPairElem:
            gemm_pair<G1, PkElem<true, false>><<<grid, block, 0, st>>>(a1, a2, x1, n1, x2);
            break;
        default:
            gemm_pair<G1, PkPipe<true, false>><<<grid, block, 0, st>>>(a1, a2, x1, n1, x2);
            break;
    }
}

// Three GEMMs in one launch: the skinny weight gradient of a small head
// (G1: workgroups below n1) and a layer's dW and dX (the pair's two kinds).
template <class G2, class G3>
__global__ __launch_bounds__(256) void gemm_triple(GemmArgs a1, GemmArgs a2, GemmArgs a3, int n1,
                                                   int x2, int n2, int x3) {
    const int w = blockIdx.x;
    if (w < n1) {
        PkSkinny<false, true>::run(a1, w, 0);
    } else if (w < n1 + n2) {
        const int v = w - n1;
        G2::run(a2, v % x2, v / x2);
    } else {
        const int v = w - n1 - n2;
        G3::run(a3, v % x3, v / x3);
    }
}

template <class G2>
void triple_with(int k3, const GemmArgs &a1, const GemmArgs &a2, const GemmArgs &a3, int n1,
                 int x2, int n2, int x3, int n3, hipStream_t st) {
    const dim3 grid(n1 + n2 + n3), block(256);
    switch (k3) {
        case kPairSkinny:
            gemm_triple<G2, PkSkinny<true, false>><<<grid, block, 0, st>>>(a1, a2, a3, n1, x2, n2, x3);
            break;
        case kPairElem:
            gemm_triple<G2, PkElem<true, false>><<<grid, block, 0, st>>>(a1, a2, a3, n1, x2, n2, x3);
            break;
        default:
            gemm_triple<G2, PkPipe<true, false>><<<grid, block, 0, st>>>(a1, a2, a3, n1, x2, n2, x3);
            break;
    }
}

// The large layers' pair: dW (TN, 256x256 tiles, 8 waves) in workgroups
// below n1, dX (NT, 256x128, 8 waves) in the rest.  Each workgroup holds a
// CU's LDS for its whole life, so a CU takes a dX tile only when a dW tile
// has left it: the dW tiles' output writes drain while dX tiles compute,
// where two launches would leave the chip idle through them.
constexpr int kBigLds = PipeLds<256, 256, 32, 2, 4>::floats > PipeLds<256, 128, 32, 4, 2>::floats
                            ? PipeLds<256, 256, 32, 2, 4>::floats
                            : PipeLds<256, 128, 32, 4, 2>::floats;
// Captured Adam steps run the optimiser's update beside these launches; the
// pair's waves take a raised issue priority (s_setprio 1) so that a CU's
// arbiter serves their MFMAs ahead of the update's waves: c5 fp32 step
// 9.649-9.690 -> 9.638-9.684 ms with 256-workgroup updates (two passes, A/B
// on one box); with the 512-workgroup updates the planner now issues,
// priority 0, 1 and 3 measure within noise (9.562-9.572 ms).
#ifndef FG_PAIR_PRIO  // a knob for measurement builds
#define FG_PAIR_PRIO 1
#endif
__global__ __launch_bounds__(512) void gemm_pair_big(GemmArgs a1, GemmArgs a2, int x1, int n1,
                                                     int x2) {
    if (FG_PAIR_PRIO > 0) __builtin_amdgcn_s_setprio(FG_PAIR_PRIO);
    const int w = blockIdx.x;
    if (w < n1) {
        gemm_f32_pipe_body<256, 256, 32, 2, 4, false, true, kProNone, false, kBigLds>(a1, w % x1,
                                                                                     w / x1);
    } else {
        const int v = w - n1;
        gemm_f32_pipe_body<256, 128, 32, 4, 2, true, false, kProNone, false, kBigLds>(a2, v % x2,
                                                                                     v / x2);
    }
}

// The 1024-wide layers' pair: dW and dX both on the 4-wave 128x64 tiles (one
// LDS buffer, the same size for both).  Alone, a 128x64 data gradient of
// 256 tiles runs one wave per SIMD; beside the weight gradient's tiles the
// CUs hold three workgroups and the waves hide each other's waits.
__global__ __launch_bounds__(256) void gemm_pair_mid(GemmArgs a1, GemmArgs a2, int x1, int n1,
                                                     int x2) {
    if (FG_PAIR_PRIO > 0) __builtin_amdgcn_s_setprio(FG_PAIR_PRIO);
    const int w = blockIdx.x;
    if (w < n1) {
        gemm_f32_pipe_body<128, 64, 32, 2, 2, false, true, kProNone, false>(a1, w % x1, w / x1);
    } else {
        const int v = w - n1;
        gemm_f32_pipe_body<128, 64, 32, 2, 2, true, false, kProNone, false>(a2, v % x2, v / x2);
    }
}

}  // namespace

void launch_triple(const GemmArgs &a1, int n1, int k2, const GemmArgs &a2, int x2, int n2, int k3,
                   const GemmArgs &a3, int x3, int n3, hipStream_t st) {
    switch (k2) {  // GEMM 2 is a TN weight gradient, GEMM 3 the NT data gradient
        case kPairSkinny:
            triple_with<PkSkinny<false, true>>(k3, a1, a2, a3, n1, x2, n2, x3, n3, st);
            break;
        case kPairElem:
            triple_with<PkElem<false, true>>(k3, a1, a2, a3, n1, x2, n2, x3, n3, st);
            break;
        default: triple_with<PkPipe<false, true>>(k3, a1, a2, a3, n1, x2, n2, x3, n3, st); break;
    }
}

void launch_pair(int k1, int k2, const GemmArgs &a1, const GemmArgs &a2, int x1, int n1, int x2,
                 int n2, hipStream_t st) {
    if (k1 == kPairBig) {  // then k2 is too (pairable)
        gemm_pair_big<<<dim3(n1 + n2), dim3(512), 0, st>>>(a1, a2, x1, n1, x2);
        return;
    }
    if (k1 == kPairMid) {  // likewise
        gemm_pair_mid<<<dim3(n1 + n2), dim3(256), 0, st>>>(a1, a2, x1, n1, x2);
        return;
    }
    switch (k1) {  // GEMM 1 is the TN weight gradient
        case kPairSkinny: launch_with<PkSkinny<false, true>>(k2, a1, a2, x1, n1, x2, n2, st); break;
        case kPairElem: launch_with<PkElem<false, true>>(k2, a1, a2, x1, n1, x2, n2, st); break;
        default: launch_with<PkPipe<false, true>>(k2, a1, a2, x1, n1, x2, n2, st); break;
    }
}

}  // namespace gemm
}  // namespace fg
