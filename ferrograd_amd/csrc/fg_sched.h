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

}  // namespace fg
