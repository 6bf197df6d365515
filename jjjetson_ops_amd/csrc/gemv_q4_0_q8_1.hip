// Decode GEMV (batch M <= 8) of Q4_0 weights x Q8_1 activations on gfx950.
//
// Math per (row n, token m, 32-block b) is the reference's
// q4_0_q8_1_vec_dot_impl (src/cuda/mm_q4_0_q8_1.cu:71-93):
//   sumi = sum_j nib_j * q_j   (unsigned nibbles, exact int32)
//   y   += d_w * (sumi * d_x - 8 * s_x)   (fp32)
//
// MI355X design (HBM-bound: 0.5625 B of weight per MAC at M = 1):
//   * The weight matrix is streamed exactly once.  A row is cut into K-slices of
//     64 block pairs (4096 values, 2304 bytes); lane l of a wave owns the 36-byte
//     pair l of the slice (two 18-byte blocks are 4-byte aligned together),
//     fetched with dwordx4 + dwordx4 + dword, so one wave instruction triple
//     covers a whole K=4096 row slice.
//   * A wave owns U rows x one K-slice: it issues all its weight loads first,
//     then reads its activation pair (M tokens x 72 bytes) straight from L2 into
//     registers — every HBM request of the kernel is in flight at once, with no
//     barrier in front of it.
//   * Even block of a pair: scale in the low half of dword 0, nibbles at byte 2
//     (re-aligned with v_alignbyte); odd block: scale in the high half of dword
//     4, nibbles in dwords 5..8.  Nibbles are masked into int8 lanes for
//     v_dot4_i32_i8: 16 dot4 per pair per token.
//   * Lane partials are summed with DPP (quad perms, row rotates) and four
//     v_readlane; the JS K-slices of a row group (JS waves of one workgroup)
//     are then added through LDS in slice order.
#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a8 __attribute__((ext_vector_type(2)));

struct PairW {
    uint32_t d[9];
};

// Activation data of one block pair for one token: 16 int8x4 dwords + 2 (d,s) words.
struct PairX {
    uint32_t q[16];
    uint32_t ds[2];
};

__device__ __forceinline__ void load_pair(PairW &w, const uint8_t *p) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(p);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(p + 16);
    const uint32_t c = *reinterpret_cast<const uint32_t *>(p + 32);
    w.d[0] = a.x; w.d[1] = a.y; w.d[2] = a.z; w.d[3] = a.w;
    w.d[4] = b.x; w.d[5] = b.y; w.d[6] = b.z; w.d[7] = b.w;
    w.d[8] = c;
}

// blk points at the 144-byte block of the pair's superblock; g0 = first group.
__device__ __forceinline__ void load_x(PairX &x, const uint8_t *blk, int g0) {
    const u32x2a8 ds = *reinterpret_cast<const u32x2a8 *>(blk + 4 * g0);
    x.ds[0] = ds.x;
    x.ds[1] = ds.y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4a16 v = *reinterpret_cast<const u32x4a16 *>(blk + 16 + 32 * g0 + 16 * i);
        x.q[4 * i + 0] = v.x; x.q[4 * i + 1] = v.y; x.q[4 * i + 2] = v.z; x.q[4 * i + 3] = v.w;
    }
}

__device__ __forceinline__ float half_lo(uint32_t v) {
    return __half2float(__ushort_as_half((unsigned short)(v & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
    return __half2float(__ushort_as_half((unsigned short)(v >> 16)));
}

// Integer dot of one Q4_0 block's 4 nibble dwords with 8 activation dwords.
__device__ __forceinline__ int32_t block_sumi(const uint32_t q[4], const uint32_t *x) {
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t lo = (int32_t)(q[i] & 0x0f0f0f0fu);
        const int32_t hi = (int32_t)((q[i] >> 4) & 0x0f0f0f0fu);
        s = __builtin_amdgcn_sdot4(lo, (int32_t)x[i], s, false);
        s = __builtin_amdgcn_sdot4(hi, (int32_t)x[i + 4], s, false);
    }
    return s;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes, returned as a wave-uniform value.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x124>(v);  // row_ror:4
    v += dpp<0x128>(v);  // row_ror:8  -> every lane holds its 16-lane row sum
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Workgroup = RG row groups x JS K-slices (one wave each).  JS = ceil(K / 4096).
template <int M, int U, int JS, int RG>
__global__ __launch_bounds__(64 * JS * RG) void gemv_q4_0_q8_1_kernel(const uint8_t *__restrict__ w,
                                                                      const uint8_t *__restrict__ xq,
                                                                      float *__restrict__ y, int K,
                                                                      int N) {
    __shared__ float part[JS > 1 ? RG * JS * U * M : 1];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int js = wave % JS;              // K-slice of this wave
    const int rg = wave / JS;              // row group inside the workgroup
    const int P = K / 64;                  // block pairs per row
    const int p = lane + 64 * js;          // this lane's pair
    const bool live = p < P;
    const size_t row_bytes = (size_t)(K / kQK) * kQ4BlockBytes;
    const int r0 = (blockIdx.x * RG + rg) * U;

    // 1) weight requests for all U rows
    PairW wb[U];
    if (live) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = min(r0 + u, N - 1);
            load_pair(wb[u], w + (size_t)r * row_bytes + (size_t)p * 36);
        }
    }
    // 2) activation pair of every token (L2-resident, tiny)
    PairX xr[M];
    if (live) {
#pragma unroll
        for (int m = 0; m < M; ++m)
            load_x(xr[m], xq + ((size_t)(p >> 1) * M + m) * kQ8BlockBytes, (p & 1) * 2);
    }

    float acc[U][M];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[u][m] = 0.0f;

    if (live) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t qa[4], qb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qa[i] = __builtin_amdgcn_alignbyte(wb[u].d[i + 1], wb[u].d[i], 2);
                qb[i] = wb[u].d[i + 5];
            }
            const float dwa = half_lo(wb[u].d[0]);
            const float dwb = half_hi(wb[u].d[4]);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const int32_t sa = block_sumi(qa, xr[m].q);
                const int32_t sb = block_sumi(qb, xr[m].q + 8);
                float a = fmaf(dwa, fmaf((float)sa, half_lo(xr[m].ds[0]), -8.0f * half_hi(xr[m].ds[0])), 0.0f);
                a = fmaf(dwb, fmaf((float)sb, half_lo(xr[m].ds[1]), -8.0f * half_hi(xr[m].ds[1])), a);
                acc[u][m] = a;
            }
        }
    }

    if constexpr (JS == 1) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float s = wave_sum(acc[u][m]);
                if (lane == ((u * M + m) & 63) && r0 + u < N) y[(size_t)m * N + r0 + u] = s;
            }
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float s = wave_sum(acc[u][m]);
                if (lane == 0) part[((rg * U + u) * M + m) * JS + js] = s;
            }
        __syncthreads();
        if (js == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    if (lane == ((u * M + m) & 63) && r0 + u < N) {
                        const float *pp = part + ((rg * U + u) * M + m) * JS;
                        float s = pp[0];
#pragma unroll
                        for (int j = 1; j < JS; ++j) s += pp[j];
                        y[(size_t)m * N + r0 + u] = s;
                    }
                }
        }
    }
}

template <int M, int U, int JS>
hipError_t launch_js(const void *w, const void *xq, float *y, int K, int N, hipStream_t stream) {
    constexpr int RG = JS >= 4 ? 1 : (JS == 3 ? 1 : 4 / JS);
    const int groups = (N + U - 1) / U;
    const int blocks = (groups + RG - 1) / RG;
    hipLaunchKernelGGL((gemv_q4_0_q8_1_kernel<M, U, JS, RG>), dim3(blocks), dim3(64 * JS * RG), 0, stream,
                       (const uint8_t *)w, (const uint8_t *)xq, y, K, N);
    return hipGetLastError();
}

template <int M, int U>
hipError_t launch_m(const void *w, const void *xq, float *y, int K, int N, hipStream_t stream) {
    const int js = (K / 64 + 63) / 64;
    switch (js) {
        case 1: return launch_js<M, U, 1>(w, xq, y, K, N, stream);
        case 2: return launch_js<M, U, 2>(w, xq, y, K, N, stream);
        case 3: return launch_js<M, U, 3>(w, xq, y, K, N, stream);
        case 4: return launch_js<M, U, 4>(w, xq, y, K, N, stream);
        case 5: return launch_js<M, U, 5>(w, xq, y, K, N, stream);
        case 6: return launch_js<M, U, 6>(w, xq, y, K, N, stream);
        case 7: return launch_js<M, U, 7>(w, xq, y, K, N, stream);
        case 8: return launch_js<M, U, 8>(w, xq, y, K, N, stream);
        default: return hipErrorInvalidValue;  // K > 32768: rejected by the C ABI
    }
}

#ifndef JJO_GEMV_U1
#define JJO_GEMV_U1 4
#endif

}  // namespace

hipError_t launch_gemv_dot4(const void *w, const void *xq, float *y, int K, int N, int M,
                            hipStream_t stream) {
    switch (M) {
        case 1: return launch_m<1, JJO_GEMV_U1>(w, xq, y, K, N, stream);
        case 2: return launch_m<2, 4>(w, xq, y, K, N, stream);
        case 3: return launch_m<3, 4>(w, xq, y, K, N, stream);
        case 4: return launch_m<4, 2>(w, xq, y, K, N, stream);
        case 5: return launch_m<5, 2>(w, xq, y, K, N, stream);
        case 6: return launch_m<6, 2>(w, xq, y, K, N, stream);
        case 7: return launch_m<7, 1>(w, xq, y, K, N, stream);
        case 8: return launch_m<8, 1>(w, xq, y, K, N, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace jjo
