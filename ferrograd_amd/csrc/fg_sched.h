// fg_sched.h -- wait-count and instruction-scheduling helpers shared by the
// MFMA GEMM main loops.
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

// Scheduling groups for one step of a main loop: MFMA q (of NM) followed by
// its share (PER) of the NR LDS reads of the next step.  The scheduler
// builtin takes compile-time arguments only, hence the recursion.
template <int Q, int NM, int NR, int PER>
__device__ __forceinline__ void sched_interleave() {
    if constexpr (Q < NM) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        constexpr int left = NR - Q * PER;
        if constexpr (left > 0)
            __builtin_amdgcn_sched_group_barrier(0x100, left < PER ? left : PER, 0);  // LDS reads
        sched_interleave<Q + 1, NM, NR, PER>();
    }
}

}  // namespace fg
