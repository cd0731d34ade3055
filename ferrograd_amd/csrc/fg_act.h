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
//   unary.rs:588-714).
#pragma once

#include <hip/hip_runtime.h>

namespace fg {

enum : int { kActNone = 0, kActRelu = 1, kActGelu = 2 };

constexpr float kGeluC0 = 0.7978846f;
constexpr float kGeluC1 = 0.044715f;

__device__ __forceinline__ float act_fwd(int act, float z) {
    if (act == kActRelu) return z > 0.0f ? z : 0.0f;
    if (act == kActGelu) {
        const float u = kGeluC0 * (z + kGeluC1 * z * z * z);
        return 0.5f * z * (1.0f + tanhf(u));
    }
    return z;
}

__device__ __forceinline__ float act_grad(int act, float z) {
    if (act == kActRelu) return z > 0.0f ? 1.0f : 0.0f;
    if (act == kActGelu) {
        const float z2 = z * z;
        const float u = kGeluC0 * (z + kGeluC1 * z2 * z);
        const float t = tanhf(u);
        return 0.5f * (1.0f + t) + 0.5f * z * (1.0f - t * t) * kGeluC0 * (1.0f + 3.0f * kGeluC1 * z2);
    }
    return 1.0f;
}

}  // namespace fg
