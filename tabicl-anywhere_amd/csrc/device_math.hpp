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

constexpr float LOG2E = 1.44269504088896340736f;

// The reference's own elementary functions (src/kern.rs), restated so the card computes what it computes:
// e^x by range reduction and a degree-7 polynomial, clamped to [-87, 88] (exp1, src/kern.rs:191-206); erf by
// Abramowitz & Stegun 7.1.26 away from zero and its power series below |x| = 0.5 (erf1, src/kern.rs:230-255);
// tanh through one exponential (tanh1, src/kern.rs:263-268); GELU as x (1 + erf(x / sqrt 2)) / 2
// (src/kern.rs:257-261). In erf1 the reciprocal is v_rcp_f32's and e^(-a^2) the hardware exp2's (1 ulp each, against
// exp1's own few ulp; the term they form is below 0.3).
__device__ __forceinline__ float exp1(float x) {
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    const float n = floorf(x * LOG2E + 0.5f);
    const float r = (x - n * 0.6933594f) - n * -2.1219444e-4f;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return p * __int_as_float(((int)n + 127) << 23);
}

__device__ __forceinline__ float erf1(float x) {
    const float a = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
    float p = 1.0614054f;
    p = p * t - 1.4531521f;
    p = p * t + 1.4214138f;
    p = p * t - 0.28449674f;
    p = p * t + 0.2548296f;
    const float far = copysignf(1.0f - p * t * __builtin_amdgcn_exp2f(-a * a * LOG2E), x);
    const float x2 = x * x;
    float q = -1.0f / 1320.0f;
    q = q * x2 + 1.0f / 216.0f;
    q = q * x2 - 1.0f / 42.0f;
    q = q * x2 + 0.1f;
    q = q * x2 - 1.0f / 3.0f;
    q = q * x2 + 1.0f;
    const float near = q * x * 1.12837916709551257390f;
    return a < 0.5f ? near : far;
}

__device__ __forceinline__ float tanh1(float x) {
    const float e = exp1(2.0f * fminf(fmaxf(x, -10.0f), 10.0f));
    return (e - 1.0f) / (e + 1.0f);
}

// GELU takes erf from A&S 7.1.26 at every argument: below |x| = 0.5 the reference's power series differs from it by
// at most 1.5e-7 (the formula's absolute error bound), which moves x (1 + erf) / 2 by under 1e-7 there, and the
// series and its selection cost as much as the formula itself (GELU is most of the feed-forward kernels' vector work).
// With erf(z) = sign(z) (1 - q(|z|)), q = p(t) t e^(-z^2), the product x (1 + erf(x / sqrt 2)) / 2 is
// max(x, 0) - |x| q / 2 for either sign of x: one fused multiply-add, with p's coefficients halved. |x| is taken of
// min(x, FLT_MAX), so that +inf gives +inf (q is 0 there) while -inf and NaN give NaN, as the product form does.
__device__ __forceinline__ float gelu(float x) {
    const float a = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(fmaf(a, 0.3275911f * 0.70710678118654752440f, 1.0f));
    float p = 0.5f * 1.0614054f;
    p = p * t - 0.5f * 1.4531521f;
    p = p * t + 0.5f * 1.4214138f;
    p = p * t - 0.5f * 0.28449674f;
    p = p * t + 0.5f * 0.2548296f;
    const float q = p * t * __builtin_amdgcn_exp2f(x * x * (-0.5f * LOG2E));
    return fmaf(-fabsf(fminf(x, 3.40282347e38f)), q, fmaxf(x, 0.0f));
}

// 2^x straight from v_exp_f32 (1 ulp): results below 2^-126, which only ever weight a softmax term, flush to 0
// instead of taking exp2f's denormal rescaling path.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// e^x for the softmax weights: exp2 of x * log2(e) on the hardware's exp2 unit. Arguments are <= 0 here.
__device__ __forceinline__ float fast_exp(float x) { return exp2_hw(x * LOG2E); }

// ---- f32 products on the fp16 matrix cores ------------------------------------------------------------------
// x = hi + lo with hi = fp16(x) and lo = fp16(x - hi) (the residual is exact in f32); x y is then formed as
// hi*hi + hi*lo + lo*hi by three v_mfma_f32_32x32x16_f16, accumulated in f32 (the splitting of Ootomo & Yokota,
// "Recovering single precision accuracy from Tensor Cores while surpassing the FP32 theoretical peak performance",
// IJHPCA 2022): 2^-22 of sum |x y| at worst, as an f32 dot product. Operands are first scaled by a power of two
// (exact) so that their largest magnitude is below 2^14: no half overflows and the low halves stay normal for all
// elements above 2^-17 of the largest.
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
// Reinterpret whole vectors only: this compiler turns __builtin_bit_cast(T, v[i]) of a vector element into element 0
// for every i (copy the element into a scalar first).

// eight consecutive floats (16-byte aligned) into v
__device__ __forceinline__ void load8(const float *p, float *v) {
    const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// 14 - e for max = m 2^e, m in [0.5, 1): scaling by 2^(14 - e) leaves every magnitude below 2^14.
__device__ __forceinline__ int shift_for(uint32_t max_bits) {
    int e = 0;
    (void)frexpf(__uint_as_float(max_bits), &e);
    return 14 - e;
}
__device__ __forceinline__ int shift_for_max(float max_abs) { return shift_for(__float_as_uint(max_abs)); }

__device__ __forceinline__ floatx16 mfma16(halfx8 a, halfx8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// acc += a * b for split operands (three products)
__device__ __forceinline__ floatx16 mfma16x3(halfx8 ah, halfx8 al, halfx8 bh, halfx8 bl, floatx16 c) {
    c = mfma16(ah, bh, c);
    c = mfma16(ah, bl, c);
    return mfma16(al, bh, c);
}

__device__ __forceinline__ uint32_t bits(fp16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// hi/lo fp16 halves of two floats, hi rounded toward zero (the residual x - hi is exact in f32). The residuals come
// from v_fma_mix_f32 reading each fp16 half of hi directly (x + (-1) hi, one instruction each, where a conversion
// back to f32 and a subtraction would take two). The last writer of lo stays an ordinary instruction (the packing
// conversion): the compiler inserts the wait states a matrix instruction needs after it, which it cannot do after
// inline assembly (v_fma_mix{lo,hi}_f16 writing lo directly gave wrong products).
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
    hi = bits(__builtin_amdgcn_cvt_pkrtz(a, b));
    float ra, rb;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(ra) : "v"(hi), "v"(a));
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(rb) : "v"(hi), "v"(b));
    lo = bits(__builtin_amdgcn_cvt_pkrtz(ra, rb));
}

// The floats hi + lo of two split values (hi: their two fp16 high halves, lo: their low halves), exact, one
// v_fma_mix_f32 each (hi * 1 + lo with both read as fp16).
__device__ __forceinline__ void join2(uint32_t hi, uint32_t lo, float &x, float &y) {
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(x) : "v"(hi), "v"(lo));
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(y) : "v"(hi), "v"(lo));
}

// eight floats times f (a power of two) as hi/lo halves
__device__ __forceinline__ void split8(const float *v, float f, halfx8 &hi, halfx8 &lo) {
    u32x4 hw, lw;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        uint32_t a, b;
        split2(v[2 * t] * f, v[2 * t + 1] * f, a, b);
        hw[t] = a;
        lw[t] = b;
    }
    hi = __builtin_bit_cast(halfx8, hw);
    lo = __builtin_bit_cast(halfx8, lw);
}

// eight int16 codes (16 bytes, in order) times their factors f, in f32, as hi/lo halves: the dequantised values of
// an i16 cache, split as split8 splits floats
__device__ __forceinline__ void dequant_split8(uint4 codes, const float (&f)[8], halfx8 &hi, halfx8 &lo) {
    const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
    u32x4 hw, lw;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        uint32_t a, b;
        split2((float)(int16_t)(w[t] & 0xffffu) * f[2 * t], (float)(int16_t)(w[t] >> 16) * f[2 * t + 1], a, b);
        hw[t] = a;
        lw[t] = b;
    }
    hi = __builtin_bit_cast(halfx8, hw);
    lo = __builtin_bit_cast(halfx8, lw);
}

// Row i of a 32-row MFMA A operand holding row sigma(i) (bits 3 and 2 swapped): the accumulators v = 8 hh .. 8 hh + 7
// of lane l of a 32 x 32 v_mfma_f32_32x32x16 result then hold rows 16 hh + 8 (l / 32) + 0..7 -- eight consecutive
// rows, which is how a B operand of a following product over those rows wants them.
__device__ __forceinline__ int sigma32(int i) { return (i & 16) | ((i & 4) << 1) | ((i & 8) >> 1) | (i & 3); }

}  // namespace tah
