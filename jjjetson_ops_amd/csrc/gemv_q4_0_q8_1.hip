// Decode GEMV (batch M <= 8) of Q4_0 weights x Q8_1 activations on gfx950.
//
// Math per (row n, token m, 32-block b) is the reference's
// q4_0_q8_1_vec_dot_impl (src/cuda/mm_q4_0_q8_1.cu:71-93):
//   sumi = sum_j nib_j * q_j   (unsigned nibbles, exact int32)
//   y   += d_w * (sumi * d_x - 8 * s_x)   (fp32)
//
// MI355X design (HBM-bound: 0.5625 B of weight per MAC at M = 1):
//   * The weight matrix is streamed once.  Lane l of a wave owns the 36-byte
//     pair of Q4_0 blocks p = l + 64 j of a row (two 18-byte blocks are 4-byte
//     aligned together), fetched with dwordx4 + dwordx4 + dword loads, so one
//     wave instruction triple reads a whole 2304-byte K=4096 row.
//   * Even block of the pair: scale in the low half of dword 0, nibbles at
//     byte offset 2 (re-aligned with v_alignbyte); odd block: scale in the high
//     half of dword 4, nibbles in dwords 5..8 (aligned).
//   * Nibbles are masked into int8 lanes and fed to v_dot4_i32_i8 against the
//     int8 activations; 16 dot4 per pair per token.
//   * The Q8_1 activation blocks of all M tokens are copied once per workgroup
//     into LDS; each lane reads its own 72 bytes (per pair, per token) with
//     ds_read_b128 / b64.
//   * U rows are in flight per wave with a two-stage register pipeline (loads of
//     the next row group are issued before the current one is reduced).
//   * Cross-lane sums use DPP row shifts + row broadcasts (no LDS).
#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a8 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

struct PairW {
    uint32_t d[9];
};

__device__ __forceinline__ void load_pair(PairW &w, const uint8_t *p) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(p);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(p + 16);
    const uint32_t c = *reinterpret_cast<const uint32_t *>(p + 32);
    w.d[0] = a.x; w.d[1] = a.y; w.d[2] = a.z; w.d[3] = a.w;
    w.d[4] = b.x; w.d[5] = b.y; w.d[6] = b.z; w.d[7] = b.w;
    w.d[8] = c;
}

__device__ __forceinline__ float half_lo(uint32_t v) {
    return __half2float(__ushort_as_half((unsigned short)(v & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
    return __half2float(__ushort_as_half((unsigned short)(v >> 16)));
}

// Integer dot of one Q4_0 block's 4 nibble dwords with 8 activation dwords.
__device__ __forceinline__ int32_t block_sumi(const uint32_t q[4], const uint32_t x[8]) {
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

// Full-wave sum; the result is valid in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += __shfl_xor(v, 32, 64);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    return v;
}

template <int M, int U>
__global__ __launch_bounds__(kThreads) void gemv_q4_0_q8_1_kernel(const uint8_t *__restrict__ w,
                                                                  const uint8_t *__restrict__ xq,
                                                                  float *__restrict__ y, int K,
                                                                  int N) {
    extern __shared__ __align__(16) uint8_t smem_x[];  // M * K/128 blocks of 144 B

    // ---- stage all activation blocks of the M tokens into LDS (contiguous run) ----
    const int x_bytes = M * (K / kQSuper) * kQ8BlockBytes;
    for (int off = threadIdx.x * 16; off < x_bytes; off += kThreads * 16)
        *reinterpret_cast<u32x4a16 *>(smem_x + off) = *reinterpret_cast<const u32x4a16 *>(xq + off);
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int P = K / 64;                  // block pairs per row
    const int J = (P + 63) / 64;           // pair iterations per lane
    const size_t row_bytes = (size_t)(K / kQK) * kQ4BlockBytes;
    const int n_groups = (N + U - 1) / U;
    const int wave_id = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int n_waves = gridDim.x * kWaves;

    // Iteration space of this wave: (group g, pair iteration j) flattened.
    const int my_groups = wave_id < n_groups ? (n_groups - 1 - wave_id) / n_waves + 1 : 0;
    const int T = my_groups * J;

    auto issue = [&](PairW (&buf)[U], int it) {
        const int g = wave_id + (it / J) * n_waves;
        const int p = lane + 64 * (it % J);
        if (p < P) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int r = g * U + u;
                r = r < N ? r : N - 1;
                load_pair(buf[u], w + (size_t)r * row_bytes + (size_t)p * 36);
            }
        }
    };

    float acc[U][M];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[u][m] = 0.0f;

    auto consume = [&](PairW (&buf)[U], int it) {
        const int g = wave_id + (it / J) * n_waves;
        const int j = it % J;
        const int p = lane + 64 * j;
        if (p < P) {
            // Unpack both blocks' nibble dwords and scales once for all tokens.
            uint32_t qa[U][4], qb[U][4];
            float dwa[U], dwb[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    qa[u][i] = __builtin_amdgcn_alignbyte(buf[u].d[i + 1], buf[u].d[i], 2);
                    qb[u][i] = buf[u].d[i + 5];
                }
                dwa[u] = half_lo(buf[u].d[0]);
                dwb[u] = half_hi(buf[u].d[4]);
            }
            const int sb = p >> 1;           // superblock of the pair
            const int g0 = (p & 1) * 2;      // first group inside the superblock
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint8_t *blk = smem_x + (sb * M + m) * kQ8BlockBytes;
                const u32x2a8 ds = *reinterpret_cast<const u32x2a8 *>(blk + 4 * g0);
                const u32x4a16 x0 = *reinterpret_cast<const u32x4a16 *>(blk + 16 + 32 * g0);
                const u32x4a16 x1 = *reinterpret_cast<const u32x4a16 *>(blk + 32 + 32 * g0);
                const u32x4a16 x2 = *reinterpret_cast<const u32x4a16 *>(blk + 48 + 32 * g0);
                const u32x4a16 x3 = *reinterpret_cast<const u32x4a16 *>(blk + 64 + 32 * g0);
                const uint32_t xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const uint32_t xb[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                const float dxa = half_lo(ds.x), sxa = half_hi(ds.x);
                const float dxb = half_lo(ds.y), sxb = half_hi(ds.y);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t sa = block_sumi(qa[u], xa);
                    const int32_t sbv = block_sumi(qb[u], xb);
                    acc[u][m] = fmaf(dwa[u], fmaf((float)sa, dxa, -8.0f * sxa), acc[u][m]);
                    acc[u][m] = fmaf(dwb[u], fmaf((float)sbv, dxb, -8.0f * sxb), acc[u][m]);
                }
            }
        }
        if (j == J - 1) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = g * U + u;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float s = wave_sum(acc[u][m]);
                    acc[u][m] = 0.0f;
                    if (lane == 0 && r < N) y[(size_t)m * N + r] = s;
                }
            }
        }
    };

    PairW bufA[U], bufB[U];
    if (T > 0) issue(bufA, 0);
    for (int it = 0; it < T; it += 2) {
        if (it + 1 < T) issue(bufB, it + 1);
        consume(bufA, it);
        if (it + 2 < T) issue(bufA, it + 2);
        if (it + 1 < T) consume(bufB, it + 1);
    }
}

template <int M, int U>
hipError_t launch_m(const void *w, const void *xq, float *y, int K, int N, hipStream_t stream) {
    const size_t smem = (size_t)M * (K / kQSuper) * kQ8BlockBytes;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)gemv_q4_0_q8_1_kernel<M, U>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int n_groups = (N + U - 1) / U;
    int blocks = (n_groups + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((gemv_q4_0_q8_1_kernel<M, U>), dim3(blocks), dim3(kThreads), smem, stream,
                       (const uint8_t *)w, (const uint8_t *)xq, y, K, N);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_dot4(const void *w, const void *xq, float *y, int K, int N, int M,
                            hipStream_t stream) {
    switch (M) {
        case 1: return launch_m<1, 4>(w, xq, y, K, N, stream);
        case 2: return launch_m<2, 4>(w, xq, y, K, N, stream);
        case 3: return launch_m<3, 4>(w, xq, y, K, N, stream);
        case 4: return launch_m<4, 4>(w, xq, y, K, N, stream);
        case 5: return launch_m<5, 2>(w, xq, y, K, N, stream);
        case 6: return launch_m<6, 2>(w, xq, y, K, N, stream);
        case 7: return launch_m<7, 2>(w, xq, y, K, N, stream);
        case 8: return launch_m<8, 2>(w, xq, y, K, N, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace jjo
