// Q8_1 activation quantizer for gfx950 (wave64).
//
// Semantics follow quantize_q8_1_kernel (src/cuda/q8_1.cu:20-104) bit for bit:
//   * a 32-value group is spread over 8 lanes holding 4 consecutive floats each;
//   * amax = max |x| and sum = sum x are reduced over those 8 lanes with the
//     xor-4, xor-2, xor-1 butterfly; the per-lane sum is ((x0+x1)+x2)+x3, so the
//     group sum is ((t0+t4)+(t2+t6))+((t1+t5)+(t3+t7)) exactly as the reference;
//   * d_inv = amax > 0 ? 127/amax : 0 (IEEE divide), q = roundf(x*d_inv);
//   * ds4[g] = half2(1/d_inv, sum), round-to-nearest-even (zero group: d = +inf).
//
// MI355X mapping: a 256-thread workgroup covers 1024 consecutive values of one
// token (8 superblocks); each lane does one 16-byte load, the butterfly uses
// ds_swizzle inside 32-lane groups (no LDS memory traffic), each half-wave
// stores one contiguous 128-byte qs run plus four 4-byte ds words.  The kernel
// is HBM-bound (4 B read + 1.125 B written per value).
#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"
#include "q8_1_quant.hpp"

namespace jjo {
namespace {

// SWIGLU: the quantized value is silu(gate) * up, with gate = x[m*ldx + i] and
// up = x[m*ldx + K + i] (the two halves of a [rows][2K] gate|up matrix);
// mid_out (optional) receives the fp32 values.
template <bool SWIGLU>
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float *__restrict__ x,
                                                            uint8_t *__restrict__ y, int64_t K,
                                                            int64_t K_pad, int64_t ne1,
                                                            int64_t slice_blocks, int64_t ldx,
                                                            float *__restrict__ mid_out) {
    const int64_t i0 = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 4;  // value index in the token
    if (i0 >= K_pad) return;  // whole 32-groups leave together (K_pad % 128 == 0)
    const int64_t m = blockIdx.x;
    const int64_t z = blockIdx.z;

    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    const bool live = i0 < K;  // uniform over each 8-lane group since K % 32 == 0
    if constexpr (SWIGLU) {
        if (live) {
            const float4 g = *reinterpret_cast<const float4 *>(x + m * ldx + i0);
            const float4 u = *reinterpret_cast<const float4 *>(x + m * ldx + K + i0);
            v = make_float4(swiglu(g.x, u.x), swiglu(g.y, u.y), swiglu(g.z, u.z), swiglu(g.w, u.w));
            if (mid_out != nullptr) *reinterpret_cast<float4 *>(mid_out + m * K + i0) = v;
        }
    } else {
        if (live) v = *reinterpret_cast<const float4 *>(x + (z * ne1 + m) * K + i0);
    }

    uint32_t ds;
    const uint32_t q = quantize_group8(v.x, v.y, v.z, v.w, &ds);

    const int64_t blk = z * slice_blocks + (i0 / kQSuper) * ne1 + m;
    uint8_t *out = y + blk * kQ8BlockBytes;
    const int iqs = (int)(i0 % kQSuper);
    if (live) {
        *reinterpret_cast<uint32_t *>(out + 16 + iqs) = q;
        if ((iqs & 31) == 0) *reinterpret_cast<uint32_t *>(out + 4 * (iqs / 32)) = ds;
    } else {
        // Groups past K in the last superblock: deterministic zero bytes.
        *reinterpret_cast<uint32_t *>(out + 16 + iqs) = 0u;
        if ((iqs & 31) == 0) *reinterpret_cast<uint32_t *>(out + 4 * (iqs / 32)) = 0u;
    }
}

}  // namespace

hipError_t launch_quantize_q8_1(const float *x, void *y, int64_t K, int64_t ne1, int64_t nz,
                                hipStream_t stream) {
    const int64_t K_pad = (K + kQSuper - 1) / kQSuper * kQSuper;
    // Per-slice block stride of the reference kernel: ne1 * gridDim.y * 128/32 with
    // gridDim.y = ceil(K/512) (src/cuda/q8_1.cu:84,173).  Irrelevant when nz == 1.
    const int64_t slice_blocks = ne1 * 4 * ((K + 511) / 512);
    const dim3 grid((unsigned)ne1, (unsigned)((K_pad + 1023) / 1024), (unsigned)nz);
    hipLaunchKernelGGL(quantize_q8_1_kernel<false>, grid, dim3(256), 0, stream, x, (uint8_t *)y, K, K_pad,
                       ne1, slice_blocks, (int64_t)0, (float *)nullptr);
    return hipGetLastError();
}

hipError_t launch_swiglu_quantize_q8_1(const float *gate_up, void *y, float *mid_out, int64_t K, int64_t rows,
                                       hipStream_t stream) {
    const int64_t K_pad = (K + kQSuper - 1) / kQSuper * kQSuper;
    const dim3 grid((unsigned)rows, (unsigned)((K_pad + 1023) / 1024), 1u);
    hipLaunchKernelGGL(quantize_q8_1_kernel<true>, grid, dim3(256), 0, stream, gate_up, (uint8_t *)y, K, K_pad,
                       rows, (int64_t)0, 2 * K, mid_out);
    return hipGetLastError();
}

}  // namespace jjo
