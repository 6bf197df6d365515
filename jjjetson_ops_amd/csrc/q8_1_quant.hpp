// Device pieces of the Q8_1 quantizer shared by every kernel that writes Q8_1
// bytes (the standalone quantizer and GEMM epilogues that quantize their output):
// one 32-value group is 8 consecutive lanes of 4 values each, reduced with the
// xor-4, xor-2, xor-1 butterfly of quantize_q8_1_kernel (src/cuda/q8_1.cu:56-68).
#pragma once

#include <hip/hip_fp16.h>
#include <stdint.h>

namespace jjo {
namespace {

// ds_swizzle bit-mode pattern: and_mask = 0x1f, xor_mask = `x` (within 32 lanes).
template <int X>
__device__ __forceinline__ float swz_xor(float v) {
    constexpr int pattern = 0x1f | (X << 10);
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), pattern));
}

// v0..v3 are the rounded fp32 products x*d_inv (no contraction into what follows).
__device__ __forceinline__ uint32_t pack_q(float v0, float v1, float v2, float v3) {
#pragma clang fp contract(off)
    const int32_t a = (int32_t)roundf(v0);
    const int32_t b = (int32_t)roundf(v1);
    const int32_t c = (int32_t)roundf(v2);
    const int32_t d = (int32_t)roundf(v3);
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// silu(g) * u of swiglu_silu_mul_kernel (src/cuda/swiglu.cu:5-14), g / (1 + e^-g)
// times u, with e^-g = 2^(-g*log2(e)) and the reciprocal on the hardware's
// v_exp_f32 / v_rcp_f32 (about 1 ulp each) instead of the IEEE-exact expf and
// divide: a relative error below 1e-6 for |g| < 100, against about 25 VALU
// operations per value for the exact forms.  The limits match: g -> -inf gives
// e^-g = inf, 1/inf = 0 and a zero result; g -> +inf gives 1/1 = 1.
__device__ __forceinline__ float swiglu(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896340736f);
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    return g * r * u;
}

// Q8_1 bytes of one 32-value group held as 4 values per lane by 8 consecutive
// lanes (lane j: values 4j..4j+3), every lane of the wave active.  Returns the
// lane's 4 quantized bytes; *ds receives the group's half2 {d, s} bits (the
// same in all 8 lanes).  Arithmetic of src/cuda/q8_1.cu:56-103.
__device__ __forceinline__ uint32_t quantize_group8(float x0, float x1, float x2, float x3, uint32_t *ds) {
    // The inputs are rounded fp32 values (the reference quantizes values that were
    // stored to memory): no contraction of a caller's multiply into these adds.
#pragma clang fp contract(off)
    float amax = fmaxf(fabsf(x0), fmaxf(fabsf(x1), fmaxf(fabsf(x2), fabsf(x3))));
    float sum = x0 + x1;
    sum = sum + x2;
    sum = sum + x3;
    amax = fmaxf(amax, swz_xor<4>(amax));
    sum = sum + swz_xor<4>(sum);
    amax = fmaxf(amax, swz_xor<2>(amax));
    sum = sum + swz_xor<2>(sum);
    amax = fmaxf(amax, swz_xor<1>(amax));
    sum = sum + swz_xor<1>(sum);
    const float d_inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
    const __half hd = __float2half_rn(1.0f / d_inv);
    const __half hs = __float2half_rn(sum);
    *ds = (uint32_t)__half_as_ushort(hd) | ((uint32_t)__half_as_ushort(hs) << 16);
    return pack_q(x0 * d_inv, x1 * d_inv, x2 * d_inv, x3 * d_inv);
}

}  // namespace
}  // namespace jjo
