// Small device helpers: wavefront (64-lane) reductions, GELU, and the MFMA operand vector type.
#pragma once

#include <hip/hip_runtime.h>

namespace tah {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// GELU as PyTorch defines it by default, x * (1 + erf(x / sqrt 2)) / 2 (src/kern.rs:255-261), with the device
// library's erff.
__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }

constexpr float LOG2E = 1.44269504088896340736f;

// 2^x straight from v_exp_f32 (1 ulp): results below 2^-126, which only ever weight a softmax term, flush to 0
// instead of taking exp2f's denormal rescaling path.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// e^x for the softmax weights: exp2 of x * log2(e) on the hardware's exp2 unit. Arguments are <= 0 here.
__device__ __forceinline__ float fast_exp(float x) { return exp2_hw(x * LOG2E); }

}  // namespace tah
