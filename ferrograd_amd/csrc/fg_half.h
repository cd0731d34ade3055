// fg_half.h -- 16-bit storage types (fp16, bf16) of the device kernels.
//
// Tensors of SimpleDType F16 / BF16 (crates/fused_gpu/src/dispatch/backend/
// mod.rs:335-427) are stored as 16-bit words; kernels widen them to fp32,
// compute in fp32 and round once to the storage type (round to nearest
// even) where a node value is stored.  For + - * / a single fp32 operation
// followed by that rounding equals the IEEE operation in the 16-bit type
// (fp32 carries more than twice the 11-bit / 8-bit significands plus two).
#pragma once

// hipRTC (the compiled elementwise kernels, fg_elt_jit.cpp) declares the
// runtime and the fixed-width integer types itself.
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>

#include <cstdint>
#endif

namespace fg {

// Element type codes shared with the C ABI (FG_DTYPE_*).
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

__device__ __forceinline__ float bf16_to_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float f16_to_f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint16_t f_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Widen / narrow by a run-time type code (uniform per launch).
__device__ __forceinline__ float h16_to_f(int dt, uint16_t h) {
    return dt == kBF16 ? bf16_to_f(h) : f16_to_f(h);
}
__device__ __forceinline__ uint16_t f_to_h16(int dt, float f) {
    return dt == kBF16 ? f_to_bf16(f) : f_to_f16(f);
}
// Round an fp32 value to the 16-bit type and back (identity for fp32).
__device__ __forceinline__ float round_to(int dt, float f) {
    if (dt == kBF16) return bf16_to_f(f_to_bf16(f));
    if (dt == kF16) return f16_to_f(f_to_f16(f));
    return f;
}

// Load / store one element of a buffer of type dt as fp32.
__device__ __forceinline__ float load_as_f(const void *p, int dt, uint64_t i) {
    if (dt == kF32) return static_cast<const float *>(p)[i];
    return h16_to_f(dt, static_cast<const uint16_t *>(p)[i]);
}
__device__ __forceinline__ void store_from_f(void *p, int dt, uint64_t i, float v) {
    if (dt == kF32)
        static_cast<float *>(p)[i] = v;
    else
        static_cast<uint16_t *>(p)[i] = f_to_h16(dt, v);
}

}  // namespace fg
