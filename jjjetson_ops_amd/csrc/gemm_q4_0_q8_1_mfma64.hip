// Q4_0 x Q8_1 GEMM on gfx950 int8 matrix cores, 64 x 64 workgroup tiles: the form
// for batches too small to fill the chip with the 128 x 128 kernel's tiles.
//
// Same math and epilogue as that kernel (mfma_q4q8_tile.hpp; reference per-block
// epilogue src/cuda/mm_q4_0_q8_1.cu:71-93, summed over K at :256-269).  What
// changes is the tiling:
//   * a workgroup owns 64 weight rows x 64 tokens; four waves in 2 x 2, each owning
//     ONE 32 x 32 MFMA tile, so a workgroup streams half the weight rows and a wave
//     holds a quarter of the accumulators (about half the VGPRs, so more waves fit
//     on a SIMD);
//   * K stages of 128 values (one Q8_1 superblock), weights staged through
//     registers (one block per thread) with nibbles expanded to int8 in LDS, activations by
//     LDS DMA; both double-buffered, one barrier per stage, 38 KB of LDS;
//   * inside a stage the MFMA of block b+1 is issued before the epilogue of block b.
// At M = 64..512 and N = 14336 this launches 224..1792 workgroups instead of
// 112..448.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "mfma_q4q8_tile.hpp"
#include "q4q8_common.hpp"

namespace jjo {
namespace {

constexpr int SBM = 64;   // tokens per workgroup
constexpr int SKB = 4;    // 32-blocks per stage
constexpr int kSThreads = 256;

constexpr int kSXsBytes = SBM * kQ8BlockBytes;            // 9216 per stage: [SBM][144]
constexpr int kSWqStride = SKB * 32 + 16;                 // 144: one row's 4 unpacked blocks + pad
constexpr int kSXRuns = kSXsBytes / 1024;                 // 9 wave-sized (1 KB) runs per stage

// LDS layout for TR weight rows per workgroup (64, or 32).
template <int TR>
struct SmallTile {
    static constexpr int kWqBytes = TR * kSWqStride;
    static constexpr int kWdEpiBytes = SKB * TR * 4;      // [SKB][TR] fp32, rows permuted per 32
    static constexpr int kWdRowBytes = TR * SKB * 2;      // [TR][SKB] fp16
    static constexpr int kWBufBytes = kWqBytes + kWdEpiBytes + kWdRowBytes;
    static constexpr int kOffW = 2 * kSXsBytes;
    static constexpr int kOffWdEpi = kWqBytes;
    static constexpr int kOffWdRow = kWqBytes + kWdEpiBytes;
    static constexpr int kSmemBytes = kOffW + 2 * kWBufBytes;  // 40960 (TR = 64), 29696 (TR = 32)
    // K split between wave pairs: with 32 rows the four waves are 2 token halves x
    // 2 halves of each stage's blocks, joined at the end in a fixed order.
    static constexpr int KS = TR == 64 ? 1 : 2;
};

// kSplit: the weights are in the split layout (a nibble plane, then an fp16 scale
// plane); a thread's block is then one aligned 16-byte nibble load and one 2-byte
// scale load, the same two vector-memory instructions.
template <int TR, bool kSplit = false>
__global__ __launch_bounds__(kSThreads) void gemm_q4_0_q8_1_mfma64_kernel(const uint8_t *__restrict__ w,
                                                                         const uint8_t *__restrict__ xq,
                                                                         float *__restrict__ y, int K, int N,
                                                                         int M) {
    extern __shared__ __align__(16) uint8_t smem[];
    using L = SmallTile<TR>;
    constexpr int SBN = TR;
    constexpr int kSWBufBytes = L::kWBufBytes;
    constexpr int kSOffW = L::kOffW;
    constexpr int kSOffWdEpi = L::kOffWdEpi;
    constexpr int kSOffWdRow = L::kOffWdRow;
    constexpr int KS = L::KS;
    constexpr int kBlocksPerWave = SKB / KS;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1;                    // 32-token half
    const int wn = KS == 1 ? wave >> 1 : 0;     // 32-row half of the workgroup tile
    const int kh = KS == 1 ? 0 : wave >> 1;     // half of each stage's blocks
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    const int n0 = blockIdx.x * SBN;
    const int m0 = blockIdx.y * SBM;
    const size_t row_bytes = (size_t)(K / kQK) * kQ4BlockBytes;
    const int n_stages = K / (SKB * kQK);

    // ---- weights: one 18-byte block per thread (row tid/4, block tid%4 of the stage) ----
    // Block b of a stage starts 72c + 18b bytes into the row: 4-byte aligned for even b,
    // 2 bytes past a dword for odd b.  Five aligned dwords cover it either way.  With
    // 32 rows the upper 128 threads repeat the loads of the lower ones (so every wave
    // issues the same loads and the explicit waits hold) and store nothing.
    const int st_row = (tid >> 2) & (TR - 1);
    const bool st_store = TR == 64 || tid < 4 * TR;
    const int st_blk = tid & 3;
    const bool st_odd = st_blk & 1;
    const uint8_t *w_src =
        w + (size_t)min(n0 + st_row, N - 1) * row_bytes + (size_t)((st_blk * kQ4BlockBytes) & ~3);
    // Split layout: block (row, st_blk) of stage 0 in the nibble and scale planes.
    const int nb = K / kQK;
    const size_t sblk = (size_t)min(n0 + st_row, N - 1) * nb + st_blk;
    const uint8_t *wq_s = w + sblk * 16;
    const uint16_t *wd_s = reinterpret_cast<const uint16_t *>(w + (size_t)N * nb * 16) + sblk;
    uint32_t wr0[5], wr1[5];
    // Two vector-memory instructions per call (the explicit waits count on it).
    auto load_w = [&](int c, uint32_t(&wst)[5]) {
        if constexpr (kSplit) {  // wst[0..3] the block's nibbles, wst[4] its scale
            const u32x4 a = *reinterpret_cast<const u32x4 *>(wq_s + (size_t)c * (SKB * 16));
            wst[0] = a.x; wst[1] = a.y; wst[2] = a.z; wst[3] = a.w;
            wst[4] = wd_s[(size_t)c * SKB];
        } else {
            const uint8_t *p = w_src + (size_t)c * (SKB * kQ4BlockBytes);
            const u32x4a4 a = *reinterpret_cast<const u32x4a4 *>(p);
            wst[0] = a.x; wst[1] = a.y; wst[2] = a.z; wst[3] = a.w;
            wst[4] = *reinterpret_cast<const uint32_t *>(p + 16);
        }
    };
    auto store_w = [&](int buf, const uint32_t(&wst)[5]) {
        if (!st_store) return;
        uint8_t *wq = smem + kSOffW + buf * kSWBufBytes;
        uint32_t q[4], dbits;
        if constexpr (kSplit) {
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = wst[k];
            dbits = wst[4] & 0xffffu;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = st_odd ? wst[k + 1] : __builtin_amdgcn_alignbyte(wst[k + 1], wst[k], 2);
            dbits = st_odd ? (wst[0] >> 16) : (wst[0] & 0xffffu);
        }
        u32x4 lo, hi;
        lo.x = q[0] & 0x0f0f0f0fu; lo.y = q[1] & 0x0f0f0f0fu;
        lo.z = q[2] & 0x0f0f0f0fu; lo.w = q[3] & 0x0f0f0f0fu;
        hi.x = (q[0] >> 4) & 0x0f0f0f0fu; hi.y = (q[1] >> 4) & 0x0f0f0f0fu;
        hi.z = (q[2] >> 4) & 0x0f0f0f0fu; hi.w = (q[3] >> 4) & 0x0f0f0f0fu;
        uint8_t *dst = wq + st_row * kSWqStride + st_blk * 32;
        *reinterpret_cast<u32x4 *>(dst) = lo;
        *reinterpret_cast<u32x4 *>(dst + 16) = hi;
        const unsigned short dh = (unsigned short)dbits;
        reinterpret_cast<float *>(wq + kSOffWdEpi)[st_blk * SBN + (st_row & ~31) + epi_perm(st_row & 31)] =
            __half2float(__ushort_as_half(dh));
        reinterpret_cast<unsigned short *>(wq + kSOffWdRow)[st_row * SKB + st_blk] = dh;
    };

    // ---- activations: runs r = wave, wave + 4, wave + 8 (< 9) of 1 KB by LDS DMA ----
    // Units past the last valid token re-read unit 0; those tokens' (d, s) headers are
    // zeroed once the tile has landed, so every product with them is zero.
    const size_t x_stride = (size_t)M * kQ8BlockBytes;
    const uint8_t *x_base = xq + (size_t)m0 * kQ8BlockBytes;
    const int x_valid_tokens = min(SBM, M - m0);
    const int x_valid_units = x_valid_tokens * (kQ8BlockBytes / 16);
    uint32_t x_off[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int unit = min(wave + 4 * i, kSXRuns - 1) * 64 + lane;
        x_off[i] = unit < x_valid_units ? unit * 16 : 0;
    }
    // Inline-asm DMA, as in the 128 x 128 kernel: the compiler's wait insertion would
    // otherwise wait for every load in flight before the next LDS access.  Waited for
    // explicitly below; the hardware counter counts them like any load.
    auto load_x = [&](int c) {
        const uint32_t xs = (uint32_t)(uintptr_t)(smem + (c & 1) * kSXsBytes);
        const uint8_t *src = x_base + (size_t)c * x_stride;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int run = wave + 4 * i;
            if (run >= kSXRuns || run * 64 >= x_valid_units) continue;  // uniform per wave
            const uint32_t m0v = __builtin_amdgcn_readfirstlane(xs + run * 1024);
            asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src + x_off[i]), "{m0}"(m0v) : "memory");
        }
    };
    auto zero_tail_headers = [&](int buf) {
        if (x_valid_tokens < SBM) {  // uniform over the workgroup
            if (tid >= x_valid_tokens && tid < SBM)
                *reinterpret_cast<u32x4 *>(smem + buf * kSXsBytes + tid * kQ8BlockBytes) = u32x4{0u, 0u, 0u, 0u};
            __syncthreads();
        }
    };

    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    i32x16 bias;
#pragma unroll
    for (int v = 0; v < 16; ++v) bias[v] = (int32_t)kBiasBits;
    asm volatile("" : "+v"(bias));

    // Pipeline as in the 128 x 128 kernel: X(c+1) and W(c+1), W(c+2) in flight while
    // stage c is computed from buffers c & 1.
    load_x(0);
    load_w(0, wr0);
    load_w(min(1, n_stages - 1), wr1);
    JJO_GEMM_VMCNT(2);
    store_w(0, wr0);
    __syncthreads();
    zero_tail_headers(0);
    load_x(min(1, n_stages - 1));
    load_w(min(2, n_stages - 1), wr0);

    const int col = wm * 32 + l32;  // this lane's token in the tile
    const int row = wn * 32 + l32;  // this lane's weight row for the A operand
    auto stage = [&](int c, auto par_tag) {
        constexpr int PAR = decltype(par_tag)::value;
        uint32_t(&w_next)[5] = *[&]() { if constexpr (PAR) return &wr0; else return &wr1; }();
        const uint8_t *wq = smem + kSOffW + (c & 1) * kSWBufBytes;
        const uint8_t *xs = smem + (c & 1) * kSXsBytes;

        const u32x4 h = *reinterpret_cast<const u32x4 *>(xs + col * kQ8BlockBytes);
        const uint32_t hdr[4] = {h.x, h.y, h.z, h.w};
        auto operands = [&](int b, i32x4 &aop, i32x4 &bop) {
            aop = *reinterpret_cast<const i32x4 *>(wq + row * kSWqStride + b * 32 + 16 * hh);
            bop = *reinterpret_cast<const i32x4 *>(xs + col * kQ8BlockBytes + 16 + 32 * b + 16 * hh);
        };
        auto scales = [&](int b, float(&wv)[16]) {
            const float *wd_epi = reinterpret_cast<const float *>(wq + kSOffWdEpi);
            const int rbase = wn * 32 + hh * 16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 w4 = *reinterpret_cast<const f32x4 *>(wd_epi + b * SBN + rbase + 4 * j);
                wv[4 * j] = w4.x; wv[4 * j + 1] = w4.y; wv[4 * j + 2] = w4.z; wv[4 * j + 3] = w4.w;
            }
        };
        const int bb = kh * kBlocksPerWave;  // this wave's first block of the stage
        i32x4 a0, b0, a1, b1;
        operands(bb, a0, b0);
        i32x16 d_prev = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, bias, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < kBlocksPerWave; ++j) {
            i32x16 d_next;
            if (j + 1 < kBlocksPerWave) {
                operands(bb + j + 1, a1, b1);
                d_next = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, bias, 0, 0, 0);
            }
            float wv[16];
            scales(bb + j, wv);
            float dx8, nb8;
            x_scales(hdr[bb + j], dx8, nb8);
            epilogue_f32(acc, d_prev, wv, dx8, nb8);
            if (j + 1 < kBlocksPerWave) d_prev = d_next;
        }
        // sum_b d_w * (-s_x) over the stage's 4 blocks on the f16 MFMA (K = 8: the
        // lanes of the upper K half contribute zeros), by the waves of the first half.
        if (kh == 0) {
            const f16x4 aop =
                *reinterpret_cast<const f16x4 *>(wq + kSOffWdRow + (size_t)row * SKB * sizeof(_Float16));
            uint32_t lo = ((hdr[0] >> 16) | (hdr[1] & 0xffff0000u)) ^ 0x80008000u;
            uint32_t hi = ((hdr[2] >> 16) | (hdr[3] & 0xffff0000u)) ^ 0x80008000u;
            // Zero B (not A) in the upper K half: an infinite s_x must not meet 0.
            if (hh) { lo = 0u; hi = 0u; }
            const u32x2 pk = {lo, hi};
            acc = __builtin_amdgcn_mfma_f32_32x32x8f16(aop, __builtin_bit_cast(f16x4, pk), acc, 0, 0, 0);
        }
        // Unconditional (clamped past the last stage) so every path issues the same
        // loads and the waits stay exact.
        JJO_GEMM_VMCNT(2);  // all but W(c+2): X(c+1) and W(c+1) have landed
        store_w((c + 1) & 1, w_next);
        __syncthreads();
        zero_tail_headers((c + 1) & 1);
        load_x(min(c + 2, n_stages - 1));
        load_w(min(c + 3, n_stages - 1), w_next);
    };
    int c = 0;
    for (; c + 1 < n_stages; c += 2) {
        stage(c, std::integral_constant<int, 0>{});
        stage(c + 1, std::integral_constant<int, 1>{});
    }
    if (c < n_stages) stage(c, std::integral_constant<int, 0>{});
    JJO_GEMM_VMCNT(0);

    if constexpr (KS == 2) {
        __syncthreads();  // every wave's last (clamped) activation DMA has landed
        // Join the two block halves: the second half's waves hand their accumulators
        // over through LDS (the activation buffers, free after the last barrier) and
        // the first half adds them, always in this order.
        float *part = reinterpret_cast<float *>(smem) + (size_t)wm * 16 * 64;
        if (kh == 1) {
#pragma unroll
            for (int v = 0; v < 16; ++v) part[v * 64 + lane] = acc[v];
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] += part[v * 64 + lane];
    }

    // ---- store: y[m][n] = 8 * acc ----
    const int m = m0 + col;
    if (m < M) {
        float *yrow = y + (size_t)m * N;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n0 + wn * 32 + 8 * q + 4 * hh;
            const float v0 = 8.0f * acc[4 * q + 0], v1 = 8.0f * acc[4 * q + 1];
            const float v2 = 8.0f * acc[4 * q + 2], v3 = 8.0f * acc[4 * q + 3];
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
}

template <int TR, bool kSplit>
hipError_t launch_small(const void *w, const void *xq, float *y, int K, int N, int M, hipStream_t stream) {
    constexpr int smem = SmallTile<TR>::kSmemBytes;
    hipError_t e = ensure_dynamic_lds((const void *)gemm_q4_0_q8_1_mfma64_kernel<TR, kSplit>, smem);
    if (e != hipSuccess) return e;
    const dim3 grid((N + TR - 1) / TR, (M + SBM - 1) / SBM);
    hipLaunchKernelGGL((gemm_q4_0_q8_1_mfma64_kernel<TR, kSplit>), grid, dim3(kSThreads), smem, stream,
                       (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_mfma64(const void *w, const void *xq, float *y, int K, int N, int M, hipStream_t stream,
                              int tile_rows, bool split) {
    if (split)
        return tile_rows == 32 ? launch_small<32, true>(w, xq, y, K, N, M, stream)
                               : launch_small<64, true>(w, xq, y, K, N, M, stream);
    return tile_rows == 32 ? launch_small<32, false>(w, xq, y, K, N, M, stream)
                           : launch_small<64, false>(w, xq, y, K, N, M, stream);
}

}  // namespace jjo
