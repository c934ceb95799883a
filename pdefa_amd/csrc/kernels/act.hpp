// Device-side activation functions shared by the conv epilogues and the
// elementwise kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../kernels.hpp"

namespace pdefa {
namespace k {

// The SiLU form of the reference's Winograd epilogue
// (PDEFA1.0/src/kernels/simd/avx2/conv2d_winograd.cpp:81-101): e^-x is formed
// as 2^n * P(f) with n = round(-x log2 e), f the remainder in log2 units and P
// the polynomial below.  The reference applies it on 3x3/s1 layers with
// 16 < Cin <= 512, and its outputs are matched only with the same function.
// near (when given): -x log2 e lies within window * max(1, |x log2 e|) of
// a half-integer, where the form jumps, inside the range where its
// polynomial branch applies.
__device__ __forceinline__ float silu_winograd_form(float x, float window = 0.0f, bool* near = nullptr) {
    // The product -x log2 e is rounded before it is used, as in the reference:
    // no contraction into the rounding add or the remainder.
#pragma clang fp contract(off)
    const float neg_x = -x;
    const float fx = neg_x * 1.44269504088896341f;
    // round half away from zero: for every float |fx| < 2^23,
    // trunc(fx + copysign(0.49999997, fx)) rounds fx that way (an exhaustive
    // check over all such floats agrees); the add is the only rounding step
    const float n = __builtin_truncf(fx + __builtin_copysignf(0.49999997f, fx));
    const float f = fx - n;
    if (near) {
        const float ax = __builtin_fabsf(fx);
        *near = (__builtin_fabsf(f) >= 0.5f - window * (ax > 1.0f ? ax : 1.0f)) & (ax < 128.0f);
    }
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, f, 1.3981999507e-3f);
    p = __builtin_fmaf(p, f, 8.3334519073e-3f);
    p = __builtin_fmaf(p, f, 4.1665795894e-2f);
    p = __builtin_fmaf(p, f, 1.6666665459e-1f);
    p = __builtin_fmaf(p, f, 5.0000001201e-1f);
    p = __builtin_fmaf(p, f, 1.0f);
    const int32_t e = (static_cast<int32_t>(n) + 127) << 23;
    // x / d as x * (1/d) with the hardware reciprocal (1 ulp)
    const float r = x * __builtin_amdgcn_rcpf(__builtin_fmaf(p, __int_as_float(e), 1.0f));
    // the range cut-offs are selects, not branches (the polynomial result of
    // an out-of-range x is discarded)
    const float lo = __builtin_unpredictable(neg_x > 88.37626f) ? 0.0f : r;
    return __builtin_unpredictable(neg_x < -88.37626f) ? x : lo;
}

typedef float act_float4 __attribute__((ext_vector_type(4)));
typedef int act_int4 __attribute__((ext_vector_type(4)));

// silu_winograd_form of four values, each by the same operations in the same
// order (bit-identical to four scalar calls), written over 4-wide vectors so
// that the four dependency chains interleave instruction by instruction
// instead of running one after another (a wave alone on its SIMD would
// otherwise wait out every instruction's latency).  dist (when given)
// receives, per value, (0.5 - window * max(1, |x log2 e|)) - |f| where the
// polynomial branch applies (|x log2 e| < 128), +inf elsewhere: <= 0 exactly
// where silu_winograd_form sets near (the difference of two floats is zero
// only when they are equal), so callers test the minimum of four first.
__device__ __forceinline__ act_float4 silu_winograd_form4(act_float4 x, float window = 0.0f,
                                                          act_float4* dist = nullptr) {
#pragma clang fp contract(off)
    const act_float4 neg_x = -x;
    const act_float4 fx = neg_x * 1.44269504088896341f;
    const act_float4 n = __builtin_elementwise_trunc(fx + __builtin_elementwise_copysign((act_float4)0.49999997f, fx));
    const act_float4 f = fx - n;
    if (dist) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float ax = __builtin_fabsf(fx[k]);
            const float d = (0.5f - window * (ax > 1.0f ? ax : 1.0f)) - __builtin_fabsf(f[k]);
            (*dist)[k] = __builtin_unpredictable(ax < 128.0f) ? d : __builtin_inff();
        }
    }
    act_float4 p = (act_float4)1.9875691500e-4f;
    p = __builtin_elementwise_fma(p, f, (act_float4)1.3981999507e-3f);
    p = __builtin_elementwise_fma(p, f, (act_float4)8.3334519073e-3f);
    p = __builtin_elementwise_fma(p, f, (act_float4)4.1665795894e-2f);
    p = __builtin_elementwise_fma(p, f, (act_float4)1.6666665459e-1f);
    p = __builtin_elementwise_fma(p, f, (act_float4)5.0000001201e-1f);
    p = __builtin_elementwise_fma(p, f, (act_float4)1.0f);
    const act_int4 e = (__builtin_convertvector(n, act_int4) + 127) << 23;
    const act_float4 d = __builtin_elementwise_fma(p, __builtin_bit_cast(act_float4, e), (act_float4)1.0f);
    act_float4 out;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float r = x[k] * __builtin_amdgcn_rcpf(d[k]);
        const float lo = __builtin_unpredictable(neg_x[k] > 88.37626f) ? 0.0f : r;
        out[k] = __builtin_unpredictable(neg_x[k] < -88.37626f) ? x[k] : lo;
    }
    return out;
}

// SiLU for the fused conv epilogues: x * 1/(1 + 2^(-x log2 e)) with the
// hardware exp2 and reciprocal (1 ulp each; the relative error of the result
// stays below 1e-6 on the fp32 range, far inside the 1e-3 parity tolerance).
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}

__device__ __forceinline__ float apply_act(float v, int act, float slope) {
    switch (act) {
        case kActRelu: return v > 0.0f ? v : 0.0f;
        case kActLeaky: return v > 0.0f ? v : v * slope;
        case kActSigmoid: return 1.0f / (1.0f + expf(-v));
        case kActTanh: return tanhf(v);
        case kActSilu: return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.44269504088896341f));
        case kActSiluWinogradForm: return silu_winograd_form(v);
        case kActGeluTanh: {
            const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
            return 0.5f * v * (1.0f + tanhf(inner));
        }
        case kActRecip1p: return 1.0f / (1.0f + v);
        default: return v;
    }
}

// Activation fixed at compile time, for epilogues that hoist the choice out
// of their per-element code; kActGeneric defers to the runtime code `act`.
constexpr int kActGeneric = -1;
template <int ACT>
__device__ __forceinline__ float act_fixed(float v, int act, float slope) {
    if constexpr (ACT == kActGeneric) return apply_act(v, act, slope);
    else if constexpr (ACT == kActNone) return v;
    else if constexpr (ACT == kActSilu) return silu_fast(v);
    else if constexpr (ACT == kActSiluWinogradForm) return silu_winograd_form(v);
    else return apply_act(v, ACT, slope);
}

}  // namespace k
}  // namespace pdefa
