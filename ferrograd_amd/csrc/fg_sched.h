// fg_sched.h -- wait-count helpers shared by the MFMA GEMM main loops.
#pragma once

#include <hip/hip_runtime.h>

namespace fg {

// s_waitcnt with vmcnt <= N and no wait on the other counters.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) only: every LDS read of this wave has returned.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// global_load_lds_dwordx4: 16 bytes per lane from `src` into LDS at
// lds_dst + 16 * lane (lds_dst uniform across the wave).  Written as inline
// assembly so that the compiler does not count it as an LDS write: it would
// otherwise make every transposing LDS read that follows wait for all such
// loads in flight (s_waitcnt vmcnt(0)), as it cannot tell the addresses
// apart.  The caller orders them itself: s_waitcnt vmcnt and s_barrier
// before any wave reads the stage the loads fill.  M0 carries the LDS
// address (one wait state before the load reads it); nothing else in the
// kernels that use this relies on M0.
__device__ __forceinline__ void lds_dma16(const void *src, const void *lds_dst) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds_dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
                 "s"(l)
                 : "memory");
}

// 4x4 transpose within each quad of lanes, for the GEMMs' register
// epilogues: lane e (of its quad) holds x[q] = M[q][e]; returns M[e][0..3].
// First an exchange with lane e^1 (DPP quad_perm [1,0,3,2]) that swaps the
// off-diagonal elements of each 2x2 block, then one with lane e^2
// ([2,3,0,1]) that swaps the off-diagonal 2x2 blocks.  Moves and selects
// only: every value keeps its bits.
typedef float qt_f32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp_mov_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ qt_f32x4 quad_transpose4(qt_f32x4 x, int e) {
    constexpr int kSwap1 = 0xB1, kSwap2 = 0x4E;
    const bool odd = (e & 1) != 0, high = (e & 2) != 0;
    qt_f32x4 y, z;
    const float u0 = dpp_mov_f32<kSwap1>(odd ? x[0] : x[1]);
    const float u1 = dpp_mov_f32<kSwap1>(odd ? x[2] : x[3]);
    y[0] = odd ? u0 : x[0];
    y[1] = odd ? x[1] : u0;
    y[2] = odd ? u1 : x[2];
    y[3] = odd ? x[3] : u1;
    const float w0 = dpp_mov_f32<kSwap2>(high ? y[0] : y[2]);
    const float w1 = dpp_mov_f32<kSwap2>(high ? y[1] : y[3]);
    z[0] = high ? w0 : y[0];
    z[1] = high ? w1 : y[1];
    z[2] = high ? y[2] : w0;
    z[3] = high ? y[3] : w1;
    return z;
}

}  // namespace fg
