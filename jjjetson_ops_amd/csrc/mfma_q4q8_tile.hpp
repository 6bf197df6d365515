// Pieces shared by the int8-MFMA Q4_0 x Q8_1 GEMM kernels: operand types, the
// accumulator bias trick and the per-block epilogue of one 32x32 MFMA tile.
//
// Math (src/cuda/mm_q4_0_q8_1.cu:71-93): per 32-block b,
//     y[m][n] += d_w[n,b] * (sumi[n,m,b] * d_x[m,b] - 8 * s_x[m,b]).
// One v_mfma_i32_32x32x32_i8 produces the exact int32 sumi tile of one block.  Its
// accumulator input is the integer 0x4B400000 (the bits of 1.5*2^23), so the result
// read as fp32 is exactly 1.5*2^23 + sumi (|sumi| < 2^16) and the epilogue needs no
// int->float conversion: t = fma(D, d_x/8, -1.5*2^23*d_x/8) = round(sumi*d_x)/8, then
// acc = fma(d_w, t, acc) with d_w read as fp16.  The kernels add the -8*s_x term on
// an f16 MFMA and store y = 8*acc.
#pragma once

#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));           // 16-B aligned
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t kBiasBits = 0x4B400000u;  // 1.5 * 2^23
constexpr float kBias = 12582912.0f;

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] + [15:14],
// expcnt[6:4] = 7, lgkmcnt[11:8] = 15).
#define JJO_GEMM_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n)&15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// Position of tile-local row r (0..31) in the epilogue scale layout: the 16 rows
// a lane half owns in the 32x32 MFMA output (rows 8q + 4h + i) become contiguous.
__device__ __forceinline__ int epi_perm(int r) {
    const int q = r >> 3, h = (r >> 2) & 1, i = r & 3;
    return h * 16 + q * 4 + i;
}

// Epilogue of one 32x32 int MFMA tile with fp32 scales: acc += d_w * round(sumi * d_x / 8)
// as two plain v_fma_f32 per element (v_fma_mix_f32 issues at about half their rate).
__device__ __forceinline__ void epilogue_f32(f32x16 &acc, const i32x16 &d, const float (&wv)[16], float dx8,
                                             float nb8) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const float t = fmaf(__int_as_float(d[v]), dx8, nb8);
        acc[v] = fmaf(wv[v], t, acc[v]);
    }
}

// Epilogue of one 32x32 int MFMA tile: acc += d_w * round(sumi * d_x / 8).
__device__ __forceinline__ void epilogue(f32x16 &acc, const i32x16 &d, const uint32_t (&wv)[8], float dx8,
                                         float nb8) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const f16x2 pr = __builtin_bit_cast(f16x2, wv[v >> 1]);
        const float dwv = (float)((v & 1) ? pr.y : pr.x);
        const float t = fmaf(__int_as_float(d[v]), dx8, nb8);
        acc[v] = fmaf(dwv, t, acc[v]);
    }
}

// d_x/8 and -1.5*2^23*d_x/8 straight from the fp16 bits in the low half of `h`.
__device__ __forceinline__ void x_scales(uint32_t h, float &dx8, float &nb8) {
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(dx8) : "v"(h), "s"(0.125f));
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(nb8) : "v"(h), "s"(-kBias * 0.125f));
}

}  // namespace
}  // namespace jjo
