// Prefill GEMM of Q4_0 weights x Q8_1 activations on gfx950 int8 matrix cores,
// second schedule: one wave per 32 weight rows x all 128 tokens of the tile.
//
// Math is the reference's per-block epilogue (src/cuda/mm_q4_0_q8_1.cu:71-93,
// summed over K at :256-269):
//     y[m][n] = sum_b d_w[n,b] * (sumi[n,m,b] * d_x[m,b] - 8 * s_x[m,b])
// with the exact int32 block sums of v_mfma_i32_32x32x32_i8, read as fp32 through
// the 1.5*2^23 accumulator bias (mfma_q4q8_tile.hpp), the two-FMA epilogue per
// element and block, and the s_x term on an f16 MFMA.
//
// MI355X design
//   * The epilogue's two v_fma_f32 per element and block are the kernel's floor
//     (about 2.6-2.9 clocks per wave64 FMA per SIMD against 33 clocks per 32x32x32
//     int8 MFMA, i.e. 88 VALU clocks per 33 MFMA clocks per tile and block), so the
//     layout minimises everything else a wave issues per element.
//   * Workgroup tile 128 weight rows x 128 tokens x 128 K per stage, 4 waves; wave
//     w owns rows 32w..32w+31 and all four 32-token columns.  A lane's 16 output
//     rows are then the same for its 4 column tiles, so each block needs 16 weight
//     scales per lane (4 ds_read_b128) for 64 elements, and every weight tile is
//     read from LDS by one wave only.
//   * Weights stay packed in LDS: 16 nibble bytes per (block, row), block-major,
//     so consecutive lanes read consecutive 16-byte rows (no bank conflicts).  A
//     lane expands its MFMA operand with one shift and one mask per dword: the low
//     nibbles are K elements 0..15 (lanes 0-31), the high ones 16..31 (lanes 32-63).
//   * Split layout (qs plane + d plane): the nibbles of a stage are gathered
//     straight into LDS by LDS DMA (global_load_lds_dwordx4, one 16-byte block row
//     per lane, no registers); scales come through one 4-byte load per thread.
//     block_q4_0 layout: two blocks (36 bytes) per thread through registers.
//   * Activations use the quantizer's superblock-major layout: the 128 tokens of a
//     superblock are one contiguous 18 KB run, copied to LDS by LDS DMA.
//   * Double-buffered LDS (29 KB per stage), one barrier per stage, two
//     workgroups per CU: the two waves of a SIMD belong to different workgroups,
//     so one's barrier wait does not stall the other.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "mfma_q4q8_tile.hpp"
#include "q4q8_common.hpp"

namespace jjo {
namespace {

namespace g2 {
constexpr int BN = 128;
constexpr int BM = 128;
constexpr int KB = 4;
constexpr int kThreads = 256;
constexpr int kXsBytes = BM * kQ8BlockBytes;        // 18432: [BM][144]
constexpr int kWqBytes = KB * BN * 16;              // 8192: [KB][BN][16] packed nibbles
constexpr int kWdeBytes = KB * BN * 4;              // 2048: fp32 [KB][BN], rows permuted
constexpr int kWdrBytes = BN * KB * 2;              // 1024: fp16 [BN][KB]
constexpr int kOffWq = kXsBytes;
constexpr int kOffWde = kOffWq + kWqBytes;
constexpr int kOffWdr = kOffWde + kWdeBytes;
constexpr int kBufBytes = kOffWdr + kWdrBytes;      // 29696
constexpr int kSmemBytes = 2 * kBufBytes;           // 59392
constexpr int kXRuns = kXsBytes / 1024;             // 18 wave-sized runs
}  // namespace g2

template <bool SPLIT>
__global__ __launch_bounds__(g2::kThreads, 2) void gemm_q4s_mfma_kernel(const uint8_t *__restrict__ w,
                                                                       const uint8_t *__restrict__ xq,
                                                                       float *__restrict__ y, int K, int N, int M,
                                                                       int n_tiles_n, int n_full) {
    using namespace g2;
    extern __shared__ __align__(16) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    // Tiles in launch order: n_full tiles of 128 rows x 128 tokens (row tile
    // fastest), then the remaining 128-token tiles cut into two 64-token halves, so
    // the grid's last round holds twice as many (half-sized) workgroups.
    const int bid = blockIdx.x;
    int tile, half = -1;
    if (bid < n_full) {
        tile = bid;
    } else {
        tile = n_full + ((bid - n_full) >> 1);
        half = (bid - n_full) & 1;
    }
    const int n0 = (tile % n_tiles_n) * BN;
    const int m0 = (tile / n_tiles_n) * BM + (half > 0 ? BM / 2 : 0);
    const int tile_tokens = half < 0 ? BM : BM / 2;
    const int nb = K / kQK;
    const int n_stages = nb / KB;

    // ---- activation DMA: stage c = superblock c, tokens m0.., one 18 KB run ----
    const size_t x_stride = (size_t)M * kQ8BlockBytes;
    const uint8_t *x_base = xq + (size_t)m0 * kQ8BlockBytes;
    const int x_valid_tokens = min(tile_tokens, M - m0);
    const int x_valid_units = x_valid_tokens * (kQ8BlockBytes / 16);
    uint32_t x_off[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int unit = min(wave + 4 * i, kXRuns - 1) * 64 + lane;
        x_off[i] = unit < x_valid_units ? unit * 16 : 0;
    }
    auto dma_x = [&](int c, int buf) {
        const uint32_t xs = (uint32_t)(uintptr_t)(smem + buf * kBufBytes);
        const uint8_t *src = x_base + (size_t)c * x_stride;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int run = min(wave + 4 * i, kXRuns - 1);
            if (run * 64 >= x_valid_units) continue;  // wave-uniform
            const uint32_t m0v = __builtin_amdgcn_readfirstlane(xs + run * 1024);
            asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src + x_off[i]), "{m0}"(m0v) : "memory");
        }
    };

    // ---- weights ----
    const size_t qs_plane = (size_t)N * nb * 16;
    // Split: wave w moves block w of the stage for rows 0..63 and 64..127 (two DMA
    // runs of 64 rows x 16 bytes); thread t loads the two fp16 scales of row t/2,
    // blocks 2(t&1), 2(t&1)+1.
    const int st_row = tid >> 1, st_pair = tid & 1;
    const uint8_t *wq_src0 = w + ((size_t)min(n0 + lane, N - 1) * nb + wave) * 16;
    const uint8_t *wq_src1 = w + ((size_t)min(n0 + 64 + lane, N - 1) * nb + wave) * 16;
    const uint32_t *wd_src =
        reinterpret_cast<const uint32_t *>(w + qs_plane + ((size_t)min(n0 + st_row, N - 1) * nb + 2 * st_pair) * 2);
    // block_q4_0: thread t holds the 36 bytes of row t/2, blocks 2(t&1), 2(t&1)+1.
    const uint8_t *wr_src = w + (size_t)min(n0 + st_row, N - 1) * nb * kQ4BlockBytes + st_pair * 36;
    uint32_t wst[SPLIT ? 1 : 9];

    auto load_w = [&](int c, int buf) {
        if constexpr (SPLIT) {
            const uint32_t wqs = (uint32_t)(uintptr_t)(smem + buf * kBufBytes + kOffWq) + wave * (BN * 16);
            const uint32_t m0a = __builtin_amdgcn_readfirstlane(wqs);
            const uint32_t m0b = __builtin_amdgcn_readfirstlane(wqs + 64 * 16);
            asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(wq_src0 + (size_t)c * (KB * 16)), "{m0}"(m0a)
                         : "memory");
            asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(wq_src1 + (size_t)c * (KB * 16)), "{m0}"(m0b)
                         : "memory");
            wst[0] = wd_src[c * 2];  // 4 blocks per stage = 8 bytes = 2 dwords per row
        } else {
            const uint8_t *p = wr_src + (size_t)c * (KB * kQ4BlockBytes);
            const u32x4a4 a = *reinterpret_cast<const u32x4a4 *>(p);
            const u32x4a4 b = *reinterpret_cast<const u32x4a4 *>(p + 16);
            wst[0] = a.x; wst[1] = a.y; wst[2] = a.z; wst[3] = a.w;
            wst[4] = b.x; wst[5] = b.y; wst[6] = b.z; wst[7] = b.w;
            wst[8] = *reinterpret_cast<const uint32_t *>(p + 32);
        }
    };
    // Registers -> LDS: scales (both layouts) and, for block_q4_0, the nibbles.
    auto store_w = [&](int buf) {
        uint8_t *base = smem + buf * kBufBytes;
        float *wde = reinterpret_cast<float *>(base + kOffWde);
        uint16_t *wdr = reinterpret_cast<uint16_t *>(base + kOffWdr);
        uint32_t dbits[2];
        if constexpr (SPLIT) {
            dbits[0] = wst[0] & 0xffffu;
            dbits[1] = wst[0] >> 16;
        } else {
            dbits[0] = wst[0] & 0xffffu;
            dbits[1] = wst[4] >> 16;
            uint32_t qa[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) qa[k] = __builtin_amdgcn_alignbyte(wst[k + 1], wst[k], 2);
            uint8_t *wq = base + kOffWq;
            *reinterpret_cast<u32x4 *>(wq + ((2 * st_pair) * BN + st_row) * 16) = u32x4{qa[0], qa[1], qa[2], qa[3]};
            *reinterpret_cast<u32x4 *>(wq + ((2 * st_pair + 1) * BN + st_row) * 16) =
                u32x4{wst[5], wst[6], wst[7], wst[8]};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int b = 2 * st_pair + i;
            wde[b * BN + (st_row & ~31) + epi_perm(st_row & 31)] =
                __half2float(__ushort_as_half((unsigned short)dbits[i]));
        }
        reinterpret_cast<uint32_t *>(wdr)[st_row * 2 + st_pair] = dbits[0] | (dbits[1] << 16);
    };

    // Tokens past M (a tail tile) hold stale LDS bytes: their (d, s) headers are
    // zeroed once the tile has landed, so every product with them is zero.
    auto zero_tail_headers = [&](int buf) {
        if (x_valid_tokens < tile_tokens) {  // uniform over the workgroup
            if (tid >= x_valid_tokens && tid < tile_tokens) {
                u32x4 z = {0u, 0u, 0u, 0u};
                asm volatile("" : "+v"(z));
                *reinterpret_cast<u32x4 *>(smem + buf * kBufBytes + tid * kQ8BlockBytes) = z;
            }
            __syncthreads();
        }
    };

    i32x16 bias;
#pragma unroll
    for (int v = 0; v < 16; ++v) bias[v] = (int32_t)kBiasBits;
    asm volatile("" : "+v"(bias));

    // ---- prologue: stage 0 into buffer 0, stage 1 in flight into buffer 1 ----
    dma_x(0, 0);
    load_w(0, 0);
    JJO_GEMM_VMCNT(0);
    store_w(0);
    __syncthreads();
    zero_tail_headers(0);
    if (n_stages > 1) {
        dma_x(1, 1);
        load_w(1, 1);
    }

    auto run = [&](auto ct_tag) {
        constexpr int CT = decltype(ct_tag)::value;  // 32-token column tiles of this tile
        f32x16 acc[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[ct][v] = 0.0f;
        const int shift = 4 * hh;
        for (int c = 0; c < n_stages; ++c) {
            const int buf = c & 1;
            const uint8_t *xs = smem + buf * kBufBytes;
            const uint8_t *wqs = xs + kOffWq;
            const float *wde = reinterpret_cast<const float *>(xs + kOffWde);
            const uint8_t *wdr = xs + kOffWdr;

            uint32_t hdr[CT][4];
    #pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const u32x4 h = *reinterpret_cast<const u32x4 *>(xs + (32 * ct + l32) * kQ8BlockBytes);
                hdr[ct][0] = h.x; hdr[ct][1] = h.y; hdr[ct][2] = h.z; hdr[ct][3] = h.w;
            }
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                const u32x4 raw = *reinterpret_cast<const u32x4 *>(wqs + (b * BN + 32 * wave + l32) * 16);
                i32x4 aop;
                aop.x = (int32_t)((raw.x >> shift) & 0x0f0f0f0fu);
                aop.y = (int32_t)((raw.y >> shift) & 0x0f0f0f0fu);
                aop.z = (int32_t)((raw.z >> shift) & 0x0f0f0f0fu);
                aop.w = (int32_t)((raw.w >> shift) & 0x0f0f0f0fu);
                float wv[16];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 w4 = *reinterpret_cast<const f32x4 *>(wde + b * BN + 32 * wave + 16 * hh + 4 * j);
                    wv[4 * j] = w4.x; wv[4 * j + 1] = w4.y; wv[4 * j + 2] = w4.z; wv[4 * j + 3] = w4.w;
                }
                i32x4 bop[CT];
                float dx8[CT], nb8[CT];
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    bop[ct] = *reinterpret_cast<const i32x4 *>(xs + (32 * ct + l32) * kQ8BlockBytes + 16 + 32 * b + 16 * hh);
                    x_scales(hdr[ct][b], dx8[ct], nb8[ct]);
                }
                i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[0], bias, 0, 0, 0);
                i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[1], bias, 0, 0, 0);
                epilogue_f32(acc[0], d0, wv, dx8[0], nb8[0]);
                if constexpr (CT == 4) {
                    d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[2], bias, 0, 0, 0);
                    epilogue_f32(acc[1], d1, wv, dx8[1], nb8[1]);
                    d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[3], bias, 0, 0, 0);
                    epilogue_f32(acc[2], d0, wv, dx8[2], nb8[2]);
                    epilogue_f32(acc[3], d1, wv, dx8[3], nb8[3]);
                } else {
                    epilogue_f32(acc[1], d1, wv, dx8[1], nb8[1]);
                }
            }
            // sum_b d_w * (-s_x) over the stage's 4 blocks on the f16 MFMA (K = 8: the
            // upper K half of B is zero; A stays finite so an infinite s_x meets no 0).
            {
                const f16x4 a16 = *reinterpret_cast<const f16x4 *>(wdr + (32 * wave + l32) * KB * 2);
    #pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const uint32_t *h = hdr[ct];
                    uint32_t lo = ((h[0] >> 16) | (h[1] & 0xffff0000u)) ^ 0x80008000u;
                    uint32_t hi = ((h[2] >> 16) | (h[3] & 0xffff0000u)) ^ 0x80008000u;
                    if (hh) { lo = 0u; hi = 0u; }
                    const u32x2 pk = {lo, hi};
                    acc[ct] = __builtin_amdgcn_mfma_f32_32x32x8f16(a16, __builtin_bit_cast(f16x4, pk), acc[ct], 0, 0, 0);
                }
            }

            if (c + 1 < n_stages) {
                JJO_GEMM_VMCNT(0);  // X(c+1), W(c+1) landed
                store_w(buf ^ 1);
                __syncthreads();    // publishes stage c+1, retires the reads of buffer `buf`
                zero_tail_headers(buf ^ 1);
                if (c + 2 < n_stages) {
                    dma_x(c + 2, buf);
                    load_w(c + 2, buf);
                }
            }
        }

        // ---- store: y[m][n] = 8 * acc ----
    #pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int m = m0 + 32 * ct + l32;
            if (m >= M) continue;
            float *yrow = y + (size_t)m * N;
    #pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + 32 * wave + 8 * q + 4 * hh;
                const float v0 = 8.0f * acc[ct][4 * q + 0];
                const float v1 = 8.0f * acc[ct][4 * q + 1];
                const float v2 = 8.0f * acc[ct][4 * q + 2];
                const float v3 = 8.0f * acc[ct][4 * q + 3];
                if (n + 3 < N && (N & 3) == 0) {
                    *reinterpret_cast<float4 *>(yrow + n) = make_float4(v0, v1, v2, v3);
                } else {
                    if (n + 0 < N) yrow[n + 0] = v0;
                    if (n + 1 < N) yrow[n + 1] = v1;
                    if (n + 2 < N) yrow[n + 2] = v2;
                    if (n + 3 < N) yrow[n + 3] = v3;
                }
            }
        }

    };
    if (half < 0)
        run(std::integral_constant<int, 4>{});
    else
        run(std::integral_constant<int, 2>{});
}

}  // namespace

hipError_t launch_gemm_q4s_mfma(const void *w, const void *xq, float *y, int K, int N, int M, bool split,
                                hipStream_t stream) {
    const void *kern = split ? (const void *)gemm_q4s_mfma_kernel<true> : (const void *)gemm_q4s_mfma_kernel<false>;
    hipError_t e = ensure_dynamic_lds(kern, g2::kSmemBytes);
    if (e != hipSuccess) return e;
    const int n_tiles_n = (N + g2::BN - 1) / g2::BN;
    const int64_t tiles = (int64_t)n_tiles_n * ((M + g2::BM - 1) / g2::BM);
    // Two workgroups per CU: when the tiles leave a partial last round of at most
    // half the slots, that round's tiles run as 64-token halves (twice the
    // workgroups, each half the work), so every slot of the last round is busy.
    // A batch whose tiles do not fill the slots runs every tile as two halves.
    const int64_t slots = 2 * (int64_t)device_cu_count();
    const int64_t rem = slots > 0 ? tiles % slots : 0;
    const int64_t n_split = tiles < slots ? tiles : (rem > 0 && 2 * rem <= slots) ? rem : 0;
    const int64_t n_full = tiles - n_split;
    const int64_t grid = n_full + 2 * n_split;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    if (split)
        hipLaunchKernelGGL(gemm_q4s_mfma_kernel<true>, dim3((unsigned)grid), dim3(g2::kThreads), g2::kSmemBytes, stream,
                           (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M, n_tiles_n, (int)n_full);
    else
        hipLaunchKernelGGL(gemm_q4s_mfma_kernel<false>, dim3((unsigned)grid), dim3(g2::kThreads), g2::kSmemBytes,
                           stream, (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M, n_tiles_n, (int)n_full);
    return hipGetLastError();
}

}  // namespace jjo
