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

}  // namespace fg
