// fg_act.h -- activation functions and derivatives shared by the GEMM
// epilogues and the elementwise kernels.
//
// ReLU: forward max(z, 0) (crates/ferrograd-nn/src/op/unary.rs:449); the
//   derivative is [z > 0].  The reference masks on its own output >= 0
//   (unary.rs:460-469), which never blocks a gradient; this is the corrected
//   form, 0 at z == 0.
// GELU: tanh form 0.5 z (1 + tanh(0.7978846 (z + 0.044715 z^3))) with the
//   reference's constants (unary.rs:493-494, 501-587); the derivative is the
//   exact one in z (the reference evaluates it with tanh(u) in place of z,
//   unary.rs:588-714).  Evaluated through the identity
//   0.5 (1 + tanh(u)) = s = 1 / (1 + exp(-2u)):  gelu = z s and
//   gelu' = s + 2 z s (1 - s) c0 (1 + 3 c1 z^2), with the hardware exp2 and
//   reciprocal (about 1e-6 relative at |u| = 44, where exp(-2u) is still
//   finite; beyond it s is 0 or 1 as the limits require).  This avoids the
//   cancellation of 1 + tanh(u) near -1 and costs a fraction of tanhf, which
//   dominated the activation epilogues.
// Contraction is off in these functions: with multiply-adds left to the
// compiler, it fused them differently where the same function was inlined
// into different code (a GEMM's staged and register epilogues gave fp16
// GELU values one unit apart), so every caller now evaluates the same
// sequence of roundings.
#pragma once

#ifndef __HIPCC_RTC__  // hipRTC declares the runtime itself
#include <hip/hip_runtime.h>
#endif

namespace fg {

enum : int { kActNone = 0, kActRelu = 1, kActGelu = 2 };

constexpr float kGeluC0 = 0.7978846f;
constexpr float kGeluC1 = 0.044715f;

// s = 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)) for the GELU argument u of z.
__device__ __forceinline__ float gelu_s(float z) {
#pragma clang fp contract(off)
    constexpr float kM2Log2e = -2.0f * 1.4426950408889634f;  // -2 / ln 2
    const float u = kGeluC0 * (z + kGeluC1 * z * z * z);
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(kM2Log2e * u));
}

__device__ __forceinline__ float act_fwd(int act, float z) {
#pragma clang fp contract(off)
    if (act == kActRelu) return z > 0.0f ? z : 0.0f;
    if (act == kActGelu) return z * gelu_s(z);
    return z;
}

__device__ __forceinline__ float act_grad(int act, float z) {
#pragma clang fp contract(off)
    if (act == kActRelu) return z > 0.0f ? 1.0f : 0.0f;
    if (act == kActGelu) {
        const float s = gelu_s(z);
        return s + 2.0f * z * s * (1.0f - s) * kGeluC0 * (1.0f + 3.0f * kGeluC1 * z * z);
    }
    return 1.0f;
}

}  // namespace fg
