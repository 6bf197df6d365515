// fp32 -> Q4_0 weight quantizer on gfx950 (the repacker behind the on-disk
// Q4_0 format; the reference's loader only reads F32, src/model/weight_loader.h:12-14,
// and its MMQ consumes ready-made ggml Q4_0 blocks, src/cuda/mm_q4_0_q8_1.cu:35-38).
//
// Per 32-value block (ggml's Q4_0 rule):
//   mx  = the value of largest magnitude, the first one on ties, 0 if every |v| is
//         0 (NaN never wins: a value is taken only when |v| > the running max)
//   d   = mx / -8, stored as fp16 (round to nearest even)
//   id  = d != 0 ? 1 / d : 0            (IEEE divide, fp32 d)
//   nib = clamp((int)(v * id + 8.5), 0, 15)   (two roundings: multiply, then add)
//   byte j (j < 16) = nib_j | nib_{j+16} << 4
//
// The output is the flat block array of the input read as rows of K values, so the
// kernel works on the flat sequence of blocks: a workgroup of 256 lanes quantizes
// 64 consecutive blocks (four lanes per block, 8 values per lane, two 16-byte loads
// per lane so a wave reads 2 KB contiguously) and writes their 1152 bytes through
// LDS as whole dwords (non-temporal stores).  HBM-bound: 128 bytes read and 18
// written per block.
#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ4Threads = 256;
constexpr int kQ4BlocksPerWG = kQ4Threads / 4;                      // 64
constexpr int kQ4OutBytesPerWG = kQ4BlocksPerWG * kQ4BlockBytes;    // 1152

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}

// 64-block groups per workgroup (2 and 4, with all loads issued first, measured
// slower on MI355X: 48.7 and 50.6 us against 47.5 us for 14336 x 4096).
constexpr int kQ4Groups = 1;

// Quantizes one block quarter (values 8q..8q+7 in v) into LDS record `o` (lanes of
// quarters 0/1 write; all four lanes must call it together: DPP exchanges).
__device__ __forceinline__ void quantize_quarter(const float (&v)[8], int quarter, bool live, uint8_t *o) {
    // Sequential rule inside the lane: only |v| > running max replaces it.
    float am = 0.0f, mx = 0.0f;
    int im = -1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float av = fabsf(v[j]);
        if (av > am) {
            am = av;
            mx = v[j];
            im = 8 * quarter + j;
        }
    }
    // Across the four lanes of the block: the largest |v|, the smallest index on
    // ties.  (A lane with no candidate carries key -1 and loses to any candidate;
    // with none anywhere mx stays +0.)
    float key = im >= 0 ? am : -1.0f;
    int kid = im >= 0 ? im : 64;
    float kmx = mx;
    {
        // xor 1 (quad_perm [1,0,3,2])
        const float k1 = dpp_f<0xB1>(key);
        const int i1 = dpp_i<0xB1>(kid);
        const float m1 = dpp_f<0xB1>(kmx);
        if (k1 > key || (k1 == key && i1 < kid)) { key = k1; kid = i1; kmx = m1; }
        // xor 2 (quad_perm [2,3,0,1])
        const float k2 = dpp_f<0x4E>(key);
        const int i2 = dpp_i<0x4E>(kid);
        const float m2 = dpp_f<0x4E>(kmx);
        if (k2 > key || (k2 == key && i2 < kid)) { key = k2; kid = i2; kmx = m2; }
    }
    const float best = key >= 0.0f ? kmx : 0.0f;

    const float d = best / -8.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint32_t nib[2] = {0u, 0u};  // 8 nibbles of this lane, one per byte, value order
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // two roundings (no fma): the product, then the add
#pragma clang fp contract(off)
        const float t = v[j] * id + 8.5f;
        int q = __float2int_rz(t);
        q = min(15, max(0, q));
        nib[j >> 2] |= (uint32_t)q << (8 * (j & 3));
    }
    // Byte j of the block packs values j (low nibble) and j+16 (high nibble):
    // quarters 0/1 hold values 0..15, 2/3 hold 16..31; the partner is lane ^ 2.
    const uint32_t p0 = (uint32_t)dpp_i<0x4E>((int)nib[0]);
    const uint32_t p1 = (uint32_t)dpp_i<0x4E>((int)nib[1]);
    if (live && quarter < 2) {
        const uint32_t lo0 = nib[0] | (p0 << 4), lo1 = nib[1] | (p1 << 4);
        // 2-byte aligned in LDS: write as halves
        unsigned short *o16 = reinterpret_cast<unsigned short *>(o + 2 + 8 * quarter);
        o16[0] = (unsigned short)(lo0 & 0xffffu);
        o16[1] = (unsigned short)(lo0 >> 16);
        o16[2] = (unsigned short)(lo1 & 0xffffu);
        o16[3] = (unsigned short)(lo1 >> 16);
        if (quarter == 0) *reinterpret_cast<unsigned short *>(o) = __half_as_ushort(__float2half_rn(d));
    }
}

__global__ __launch_bounds__(kQ4Threads) void quantize_q4_0_kernel(const float *__restrict__ w,
                                                                   uint8_t *__restrict__ out, int64_t n_blocks) {
    __shared__ __align__(16) uint8_t ob[kQ4Groups * kQ4OutBytesPerWG];
    const int tid = threadIdx.x;
    const int quarter = tid & 3;
    const int64_t blk0 = (int64_t)blockIdx.x * (kQ4Groups * kQ4BlocksPerWG);

    // All loads first (clamped addresses: every lane loads), then the math.
    f32x4 a[kQ4Groups], b[kQ4Groups];
#pragma unroll
    for (int g = 0; g < kQ4Groups; ++g) {
        const int64_t blk = min(blk0 + g * kQ4BlocksPerWG + (tid >> 2), n_blocks - 1);
        const float *src = w + blk * kQK + 8 * quarter;
        a[g] = *reinterpret_cast<const f32x4 *>(src);
        b[g] = *reinterpret_cast<const f32x4 *>(src + 4);
    }
#pragma unroll
    for (int g = 0; g < kQ4Groups; ++g) {
        const float v[8] = {a[g].x, a[g].y, a[g].z, a[g].w, b[g].x, b[g].y, b[g].z, b[g].w};
        const int64_t blk = blk0 + g * kQ4BlocksPerWG + (tid >> 2);
        quantize_quarter(v, quarter, blk < n_blocks, ob + (g * kQ4BlocksPerWG + (tid >> 2)) * kQ4BlockBytes);
    }
    __syncthreads();
    const int64_t live_blocks = min((int64_t)(kQ4Groups * kQ4BlocksPerWG), n_blocks - blk0);
    uint8_t *dst = out + blk0 * kQ4BlockBytes;
    if (live_blocks == kQ4Groups * kQ4BlocksPerWG && (reinterpret_cast<uintptr_t>(out) & 3) == 0) {
        const uint32_t *ob32 = reinterpret_cast<const uint32_t *>(ob);
        uint32_t *d32 = reinterpret_cast<uint32_t *>(dst);
#pragma unroll
        for (int i = tid; i < kQ4Groups * kQ4OutBytesPerWG / 4; i += kQ4Threads) {
            __builtin_nontemporal_store(ob32[i], d32 + i);  // streaming output: 5.6 -> 5.9 TB/s
        }
    } else {
        const int nbytes = (int)live_blocks * kQ4BlockBytes;
        for (int i = tid; i < nbytes; i += kQ4Threads) dst[i] = ob[i];
    }
}

}  // namespace

hipError_t launch_quantize_q4_0(const float *w, void *out, int64_t n_blocks, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t per_wg = (int64_t)kQ4Groups * kQ4BlocksPerWG;
    const int64_t grid = (n_blocks + per_wg - 1) / per_wg;
    hipLaunchKernelGGL(quantize_q4_0_kernel, dim3((unsigned)grid), dim3(kQ4Threads), 0, stream, w, (uint8_t *)out,
                       n_blocks);
    return hipGetLastError();
}

}  // namespace jjo
