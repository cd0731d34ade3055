// fg_elt_ops.h -- one element of each elementwise-program op (fg_eltwise.h):
// the single definition that the interpreter (k_eltwise_prog.hip) and the
// kernels compiled at run time (fg_elt_jit.h) both evaluate, so that the two
// give the same bits.  Unary ops follow crates/ferrograd-nn/src/op/unary.rs
// (ReLU / GELU with the corrections described in fg_act.h; ELU 329-434).
//
// exp, log and tanh are written here from the hardware's base-2 exponential
// and logarithm (v_exp_f32 / v_log_f32, about 1 ulp on their reduced
// ranges) rather than taken from the device math library: the two paths are
// built by different compilers -- hipcc for the interpreter; for compiled
// kernels the compiler behind the process's hipRTC (comgr), which in a
// PyTorch process is the older copy PyTorch's HIP runtime loads -- and that
// compiler's build of logf ends with an add where hipcc's ends with an fma
// (a one-ulp difference in a third of the results).  Every operation below
// is explicit (contraction off, multiply-adds as fma), so both compilers
// emit the same arithmetic (tests/test_eltwise_jit.py compares them).
// Accuracy against float64: exp and log within 2 ulp, tanh within 3 ulp
// (tests/test_eltwise_jit_gpu.py).
#pragma once

#include "fg_act.h"
#include "fg_half.h"

namespace fg {

// e^x = 2^(x log2 e).  x log2 e is carried as ph + pl (the product's
// rounding error recovered by an fma, plus the low part of log2 e), split
// into k = rint(ph) and t = (ph - k) + pl in about [-0.5, 0.5] (ph - k is
// exact); the result 2^t (hardware) is scaled by 2^k with ldexp, which also
// rounds subnormal results and overflows to inf.  x is clamped to
// [-104, 89] first (beyond it the result is 0 or inf anyway), NaN returned.
__device__ __forceinline__ float elt_exp(float x) {
#pragma clang fp contract(off)
    constexpr float kL2E = 0x1.715476p+0f, kL2ELo = 0x1.4ae0c0p-26f;
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);
    const float ph = xc * kL2E;
    float pl = __builtin_fmaf(xc, kL2E, -ph);
    pl = __builtin_fmaf(xc, kL2ELo, pl);
    const float k = __builtin_rintf(ph);
    const float t = (ph - k) + pl;
    const float r = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(t), (int)k);
    return x != x ? x : r;
}

// ln x = log2(x) ln 2: log2 from the hardware, the product carried as
// hi + lo (hi's rounding error recovered by an fma, plus the low part of
// ln 2) and summed once.  Inputs below the normal range (and 0, negatives)
// are scaled by 2^32 first and 32 ln 2 taken off after; infinities and NaN
// from the hardware logarithm pass through (log 0 = -inf, log of a negative
// number NaN).
__device__ __forceinline__ float elt_log(float x) {
#pragma clang fp contract(off)
    constexpr float kLn2 = 0x1.62e430p-1f, kLn2Lo = -0x1.05c610p-29f, k32Ln2 = 0x1.62e430p+4f;
    const bool sub = x < 0x1p-126f;
    const float y = __builtin_amdgcn_logf(sub ? x * 0x1p32f : x);
    const float hi = y * kLn2;
    float lo = __builtin_fmaf(y, kLn2, -hi);
    lo = __builtin_fmaf(y, kLn2Lo, lo);
    const float r = __builtin_fabsf(y) < __builtin_inff() ? hi + lo : y;
    return sub ? r - k32Ln2 : r;
}

// tanh x: for |x| < 0.55 the odd polynomial x + x^3 P(x^2) (a least-squares
// fit of degree 4 in x^2 on that range, weighted for relative error: 0.61
// ulp evaluated in fp32), above it sign(x) (1 - 2 / (e^{2|x|} + 1)), whose
// subtraction no longer cancels (the result is at least 0.5).
__device__ __forceinline__ float elt_tanh(float x) {
#pragma clang fp contract(off)
    const float a = __builtin_fabsf(x);
    if (a < 0.55f) {
        const float z = x * x;
        float p = -0x1.9c1070p-8f;
        p = __builtin_fmaf(p, z, 0x1.596866p-6f);
        p = __builtin_fmaf(p, z, -0x1.b92e5ap-5f);
        p = __builtin_fmaf(p, z, 0x1.110d50p-3f);
        p = __builtin_fmaf(p, z, -0x1.55554cp-2f);
        return __builtin_fmaf(z * x, p, x);
    }
    const float e = elt_exp(2.0f * a);
    return __builtin_copysignf(1.0f - 2.0f / (e + 1.0f), x);
}

__device__ __forceinline__ float elt_relu(float v) { return act_fwd(kActRelu, v); }
__device__ __forceinline__ float elt_gelu(float v) { return act_fwd(kActGelu, v); }
__device__ __forceinline__ float elt_elu(float v) { return v >= 0.0f ? v : elt_exp(v) - 1.0f; }
__device__ __forceinline__ float elt_abs(float v) { return fabsf(v); }
__device__ __forceinline__ float elt_relu_d(float v) { return act_grad(kActRelu, v); }
__device__ __forceinline__ float elt_gelu_d(float v) { return act_grad(kActGelu, v); }
__device__ __forceinline__ float elt_elu_d(float v) { return v >= 0.0f ? 1.0f : elt_exp(v); }
__device__ __forceinline__ float elt_sign(float v) {
    return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
}
__device__ __forceinline__ float elt_select(float c, float t, float f) { return c != 0.0f ? t : f; }
__device__ __forceinline__ float elt_max(float a, float b) { return fmaxf(a, b); }
// Add, subtract, multiply, divide and negate are the plain fp32 operators.

}  // namespace fg
