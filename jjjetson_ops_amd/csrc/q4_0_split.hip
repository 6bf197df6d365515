// The split Q4_0 weight layout and its repackers (host and gfx950).
//
// block_q4_0 (src/cuda/mm_q4_0_q8_1.cu:35-38) is 18 bytes: an fp16 scale then 16
// nibble bytes, so consecutive blocks are only 2-byte aligned and a kernel cannot
// read one block with one aligned 16-byte load.  The split layout of an N x nb
// block matrix keeps every byte and moves the scales out:
//     qs plane: block (n, b)'s 16 nibble bytes at (n*nb + b)*16
//     d plane : block (n, b)'s fp16 scale at N*nb*16 + (n*nb + b)*2
// The total size is unchanged (18 bytes per block).  The nibble order inside a
// block is the Q4_0 one (byte j: element j low, element j+16 high).
#include <hip/hip_runtime.h>
#include <string.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

// One thread per block: nine 2-byte loads (the source is 2-byte aligned), one
// 16-byte store into the qs plane, one 2-byte store into the d plane.
__global__ __launch_bounds__(256) void q4_0_to_split_kernel(const uint16_t *__restrict__ src,
                                                            uint8_t *__restrict__ dst, int64_t n_blocks) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_blocks) return;
    const uint16_t *b = src + i * 9;
    uint32_t q[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = (uint32_t)b[1 + 2 * k] | ((uint32_t)b[2 + 2 * k] << 16);
    *reinterpret_cast<uint4 *>(dst + i * 16) = make_uint4(q[0], q[1], q[2], q[3]);
    reinterpret_cast<uint16_t *>(dst + n_blocks * 16)[i] = b[0];
}

}  // namespace

hipError_t launch_q4_0_to_split(const void *w, void *out, int64_t n_blocks, hipStream_t stream) {
    const int64_t grid = (n_blocks + 255) / 256;
    hipLaunchKernelGGL(q4_0_to_split_kernel, dim3((unsigned)grid), dim3(256), 0, stream, (const uint16_t *)w,
                       (uint8_t *)out, n_blocks);
    return hipGetLastError();
}

}  // namespace jjo

extern "C" {

int64_t q4_0_split_bytes(int64_t nrows, int64_t ncols_k) {
    if (nrows <= 0 || ncols_k <= 0 || ncols_k % jjo::kQK != 0) return -1;
    return nrows * (ncols_k / jjo::kQK) * jjo::kQ4BlockBytes;
}

int q4_0_to_split(const void *w_q4_0, void *w_split, int64_t nrows, int64_t ncols_k) {
    jjo::clear_error();
    if (q4_0_split_bytes(nrows, ncols_k) < 0)
        return jjo::set_error(JJO_ERR_INVALID_ARG, "q4_0_to_split: nrows=%lld ncols_k=%lld (ncols_k %% 32 == 0)",
                              (long long)nrows, (long long)ncols_k);
    if (w_q4_0 == nullptr || w_split == nullptr || w_q4_0 == w_split)
        return jjo::set_error(JJO_ERR_INVALID_ARG, "q4_0_to_split: null or aliased buffers");
    const int64_t n = nrows * (ncols_k / jjo::kQK);
    const uint8_t *s = (const uint8_t *)w_q4_0;
    uint8_t *qs = (uint8_t *)w_split;
    uint8_t *d = qs + n * 16;
    for (int64_t i = 0; i < n; ++i) {
        memcpy(d + 2 * i, s + 18 * i, 2);
        memcpy(qs + 16 * i, s + 18 * i + 2, 16);
    }
    return JJO_OK;
}

int q4_0_from_split(const void *w_split, void *w_q4_0, int64_t nrows, int64_t ncols_k) {
    jjo::clear_error();
    if (q4_0_split_bytes(nrows, ncols_k) < 0)
        return jjo::set_error(JJO_ERR_INVALID_ARG, "q4_0_from_split: nrows=%lld ncols_k=%lld (ncols_k %% 32 == 0)",
                              (long long)nrows, (long long)ncols_k);
    if (w_q4_0 == nullptr || w_split == nullptr || w_q4_0 == w_split)
        return jjo::set_error(JJO_ERR_INVALID_ARG, "q4_0_from_split: null or aliased buffers");
    const int64_t n = nrows * (ncols_k / jjo::kQK);
    const uint8_t *qs = (const uint8_t *)w_split;
    const uint8_t *d = qs + n * 16;
    uint8_t *o = (uint8_t *)w_q4_0;
    for (int64_t i = 0; i < n; ++i) {
        memcpy(o + 18 * i, d + 2 * i, 2);
        memcpy(o + 18 * i + 2, qs + 16 * i, 16);
    }
    return JJO_OK;
}

}  // extern "C"
