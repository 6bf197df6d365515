// Small-batch (M <= 16) Q4_0 x Q8_1 matmul on gfx950 int8 matrix cores, with the
// activation resident in LDS and each workgroup streaming several weight tiles.
//
// Math is the reference's per-block epilogue (src/cuda/mm_q4_0_q8_1.cu:71-93):
//     y[m][n] = sum_b d_w[n,b] * (sumi[n,m,b] * d_x[m,b] - 8 * s_x[m,b])
// evaluated exactly as in the streaming skinny kernel: the tokens as MFMA rows and
// 16 weight rows as columns, the accumulator seeded with the bits of 1.5*2^23 so
// the result read as fp32 is 1.5*2^23 + sumi, a two-op epilogue (fma with d_x/8,
// then v_fma_mix with the fp16 d_w), and the -8*s_x term as an f16 MFMA
// contraction over blocks; y = 8*acc.
//   * M = 9..16: one v_mfma_i32_16x16x32_i8 per block (16 token rows).
//   * M <= 8 (PAIR): one v_mfma_i32_16x16x64_i8 per pair of blocks.  Row r is token
//     r & 7 of block parity r >> 3 and K = 64 spans both blocks, each row's other
//     block zeroed, so every output is still one block's exact sumi while all 16
//     rows are useful: half the epilogue instructions per block.  The two parities'
//     partial sums meet in the final reduction.
//
// Layout of the work (one workgroup of 8 waves per CU):
//   * A workgroup owns T consecutive 16-row weight tiles (T <= 4) and all of K.
//   * K is walked in windows of up to 4096 values.  Wave w takes the window's
//     256-value stages w and w+8.  It copies their Q8_1 activation (M tokens x 2
//     superblocks per stage, a contiguous run of the quantizer's superblock-major
//     layout) into its own part of the window area, so no wave waits for another's
//     copy.  Per stage it loads its MFMA activation operands, (d_x/8,
//     -1.5*2^23*d_x/8) and -s_x into registers once, then runs the stage for every
//     tile of the workgroup.
//   * Weights stream through a per-wave LDS ring of 2 items (one item = one stage
//     of one tile: 16 rows x 144 bytes), in (stage, tile) order, with
//     global_load_lds_dwordx4 and explicit vmcnt waits.  With two items in flight
//     per wave the items land close to issue order, so each item's compute
//     overlaps the stream; with 4 or more in flight (or every load issued at once)
//     most items land near the end of the stream and the compute trails it.
//   * The 8 waves' K-slice partials of each tile are added through LDS in wave
//     order at the end (deterministic).
//
// SPLIT: weights in the split layout (nibble plane + fp16 scale plane).  An item
// is then the 16 rows' 8 nibble blocks (16 x 128 bytes, gathered by two DMA
// instructions; block j of row r in slot j ^ (r & 7) of the row, against LDS bank
// conflicts) followed by their 16 x 8 scales (one DMA instruction of 16 lanes):
// the same 2304 bytes and three DMA instructions, and every operand read aligned.
//
// Requirements (checked by the launcher): M <= 16, K % 256 == 0, w and xq 16-byte aligned.
#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kPW = 8;                                   // waves per workgroup
constexpr int kPStageBlocks = 8;                         // 256 K values per stage
constexpr int kPRowBytes = kPStageBlocks * kQ4BlockBytes;  // 144
constexpr int kPItemBytes = 16 * kPRowBytes;             // 2304: one stage of one tile
constexpr int kPItemChunks = kPItemBytes / 16;           // 144 chunks of 16 bytes
constexpr int kPRing = 2;                                // items in flight per wave
static_assert(kPRing == 2, "the per-item wait below is written for two items in flight");
constexpr int kPWinK = 4096;                             // K values per activation window
constexpr int kPMaxTiles = 4;
constexpr int kPXBytes = (kPWinK / kQSuper) * 16 * kQ8BlockBytes;   // 73728 (M = 16)
constexpr int kPRingBytes = kPW * kPRing * kPItemBytes;             // 36864
constexpr int kPSmemBytes = kPXBytes + kPRingBytes;                 // 110592
constexpr uint32_t kPBiasBits = 0x4B400000u;  // 1.5 * 2^23
constexpr float kPBias = 12582912.0f;

static_assert(kPW * kPMaxTiles * 64 * 16 <= kPSmemBytes, "reduction area must fit");

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] + [15:14],
// expcnt[6:4] = 7, lgkmcnt[11:8] = 15).
#define JJO_P_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n)&15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
__device__ __forceinline__ void p_vm_wait_items(int pre) {  // pre wave-uniform, 0..2; 3 DMAs per item
    if (pre == 2) JJO_P_VMCNT(6);
    else if (pre == 1) JJO_P_VMCNT(3);
    else JJO_P_VMCNT(0);
}

// 16 bytes per lane, global -> LDS at m0 + 16*lane.  Inline asm so that the
// compiler's wait insertion does not treat the ring writes as aliasing every other
// LDS access (it would wait for all loads in flight); completion is waited for
// explicitly.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_base) {
    asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
                 : "memory");
}

template <bool PAIR, bool SPLIT>
__global__ __launch_bounds__(64 * kPW) void gemm_skinny_persist_kernel(const uint8_t *__restrict__ w,
                                                                        const uint8_t *__restrict__ xq,
                                                                        float *__restrict__ y, int K, int N, int M,
                                                                        int tiles_per_wg) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *xs = smem;                     // activation: wave w's stages at w * kPXBytes / 8
    uint8_t *ring_all = smem + kPXBytes;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    const int nb = K / kQK;
    const size_t row_bytes = (size_t)nb * kQ4BlockBytes;
    const int n_tiles_total = (N + 15) / 16;
    const int tile0 = blockIdx.x * tiles_per_wg;
    const int T = max(0, min(tiles_per_wg, n_tiles_total - tile0));  // workgroup-uniform
    uint8_t *ring = ring_all + wave * (kPRing * kPItemBytes);

    i32x4 bias;
#pragma unroll
    for (int i = 0; i < 4; ++i) bias[i] = (int32_t)kPBiasBits;
    asm volatile("" : "+v"(bias));

    f32x4 acc[kPMaxTiles];
#pragma unroll
    for (int t = 0; t < kPMaxTiles; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // token row this lane feeds to the MFMA (clamped: rows >= M are never stored)
    const int tok = min(l16, M - 1);

    for (int k0 = 0; k0 < K; k0 += kPWinK) {
        const int win = min(kPWinK, K - k0);
        const int n_st = win / (kPStageBlocks * kQK);   // stages in the window
        const int x_stride_sb = M * kQ8BlockBytes;  // bytes per superblock in the window

        // ---- this wave's items: (stage s = wave + 8j, tile t) in (s, t) order ----
        const int my_st = (n_st - wave + kPW - 1) / kPW;
        const int n_items = my_st * T;
        auto issue = [&](int it, int j, int t) {  // item it = (stage wave + 8j, tile t)
            const int s = wave + kPW * j;
            uint8_t *slot = ring + (it % kPRing) * kPItemBytes;
            if constexpr (SPLIT) {
                // Nibbles: chunk c = 64*i + lane -> row c / 8, block c % 8 of the stage;
                // then the 16 rows' 8 scales (16 bytes per row, 16-byte aligned since
                // nb % 8 == 0).  Rows past N re-read row N-1 (never stored).
                const int blk0 = (k0 / kQK) + s * kPStageBlocks;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int c = 64 * i + lane;
                    // Slot (row c / 8, j = c % 8) holds block j ^ (row & 7) of that row: with
                    // 128-byte rows, the 16 lanes reading one block of 16 rows would
                    // otherwise all hit one LDS bank.
                    const int rr = c >> 3;
                    const int r = min((tile0 + t) * 16 + rr, N - 1);
                    dma16(w + ((size_t)r * nb + blk0 + ((c & 7) ^ (rr & 7))) * 16,
                          (uint32_t)(uintptr_t)(slot + 1024 * i));
                }
                if (lane < 16) {
                    const int r = min((tile0 + t) * 16 + lane, N - 1);
                    dma16(w + (size_t)N * nb * 16 + ((size_t)r * nb + blk0) * 2,
                          (uint32_t)(uintptr_t)(slot + 2048));
                }
            } else {
            const uint8_t *base = w + (size_t)((k0 / kQK) + s * kPStageBlocks) * kQ4BlockBytes;
            // Three DMA instructions per item (the third with lanes 0..15 only): chunk
            // c = 64*i + lane -> row c / 9, 16-byte piece c % 9 of the row's 144 bytes,
            // i.e. LDS slot offset 16*c.  Rows past N re-read row N-1 (never stored).
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const int c = min(64 * i + lane, kPItemChunks - 1);
                const int r = min((tile0 + t) * 16 + c / 9, N - 1);
                const uint8_t *src = base + (size_t)r * row_bytes + 16u * (uint32_t)(c % 9);
                if (i < 2 || lane < kPItemChunks - 128) dma16(src, (uint32_t)(uintptr_t)(slot + 1024 * i));
            }
            }
        };

        // ---- this wave's activation stages -> its own part of the window area ----
        uint8_t *xw = xs + wave * (kPXBytes / kPW);
        {
            const int x_stage_chunks = 2 * x_stride_sb / 16;
            for (int j = 0; j < my_st; ++j) {
                const int s = wave + kPW * j;
                const uint8_t *src = xq + (size_t)(k0 / kQSuper + 2 * s) * x_stride_sb;
                uint8_t *dst = xw + j * 2 * x_stride_sb;
                for (int c0 = 0; c0 < x_stage_chunks; c0 += 64) {
                    const int c = c0 + lane;
                    if (c < x_stage_chunks) dma16(src + 16 * (size_t)c, (uint32_t)(uintptr_t)(dst + 16 * c0));
                }
            }
        }
        const int pre = min(kPRing, n_items);
        for (int it = 0; it < pre; ++it) issue(it, it / T, it % T);
        p_vm_wait_items(pre);  // this wave's activation DMAs (issued first) have landed

        // After item it is consumed: refill its ring slot with item it + 2.
        auto refill = [&](int it, int j, int t) {
            if (it + kPRing < n_items) {
                __builtin_amdgcn_s_waitcnt(0xC07F);  // slot it % 2 fully read (lgkmcnt(0))
                int jn = j, tn = t + kPRing;  // (stage, tile) of item it + 2 without a divide
                while (tn >= T) { tn -= T; ++jn; }
                issue(it + kPRing, jn, tn);
            }
        };
        if constexpr (PAIR) {
        // M <= 8: one v_mfma_i32_16x16x64_i8 per pair of blocks.  MFMA row r is token
        // r & 7 of block parity r >> 3; the K range 0..63 holds the pair's two blocks,
        // and each row's other block is zero, so every output is one block's exact
        // sumi and all 16 output rows are useful.
        const int ta = min(l16 & 7, M - 1);  // token of this lane's A row
        const int pa = l16 >> 3;             // block parity of this lane's A row
        const int kc = g & 1;                // this lane's 8-byte chunk of a block's qs
        const int po = g >> 1;               // block parity of this lane's B operand and outputs
        for (int j = 0; j < my_st; ++j) {
            const uint8_t *xst = xw + j * 2 * x_stride_sb;
            i32x4 aop[kPStageBlocks / 2];
            float dx8[kPStageBlocks / 2][4], nb8[kPStageBlocks / 2][4];
            f16x4 sx_op;
            {
#pragma unroll
                for (int p = 0; p < kPStageBlocks / 2; ++p) {
                    const int bb = 2 * p + pa, h = bb >> 2, jj = bb & 3;
                    const uint8_t *xa = xst + h * x_stride_sb + ta * kQ8BlockBytes + 16 + 32 * jj + 8 * kc;
                    const uint2 lo8 = *reinterpret_cast<const uint2 *>(xa);
                    const uint2 hi8 = *reinterpret_cast<const uint2 *>(xa + 16);
                    const uint32_t keep = po == pa ? 0xffffffffu : 0u;
                    aop[p] = i32x4{(int32_t)(lo8.x & keep), (int32_t)(lo8.y & keep), (int32_t)(hi8.x & keep),
                                   (int32_t)(hi8.y & keep)};
                }
                // d_x of this lane's outputs: tokens 4kc..4kc+3 of blocks 2p + po
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = min(4 * kc + i, M - 1);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint4 v = *reinterpret_cast<const uint4 *>(xst + h * x_stride_sb + m * kQ8BlockBytes);
#pragma unroll
                        for (int q = 0; q < 2; ++q) {  // pair p = 2h + q: block 4h + 2q + po
                            const uint32_t vv = q == 0 ? (po ? v.y : v.x) : (po ? v.w : v.z);
                            const float d8 = __half2float(__ushort_as_half((unsigned short)(vv & 0xffffu))) * 0.125f;
                            dx8[2 * h + q][i] = d8;
                            nb8[2 * h + q][i] = -kPBias * d8;
                        }
                    }
                }
                // -s_x of the stage's 8 blocks as the f16 A operand of the s_x MFMA: rows of
                // parity 0 only (token ta), group g < 2 holds blocks 4g..4g+3.
                const uint4 v = *reinterpret_cast<const uint4 *>(xst + (g & 1) * x_stride_sb + ta * kQ8BlockBytes);
                const uint32_t keep = (g < 2 && pa == 0) ? 0xffffffffu : 0u;
                const uint32_t lo = (__builtin_amdgcn_perm(v.y, v.x, 0x07060302u) ^ 0x80008000u) & keep;
                const uint32_t hi = (__builtin_amdgcn_perm(v.w, v.z, 0x07060302u) ^ 0x80008000u) & keep;
                sx_op = __builtin_bit_cast(f16x4, (uint64_t)hi << 32 | lo);
            }
#pragma unroll
            for (int t = 0; t < kPMaxTiles; ++t) {
                if (t >= T) break;  // workgroup-uniform
                __builtin_amdgcn_sched_barrier(0);
                const int it = j * T + t;
                if (it + 1 < n_items) JJO_P_VMCNT(3); else JJO_P_VMCNT(0);  // item it has landed
                const uint8_t *slot = ring + (it % kPRing) * kPItemBytes;
                const uint8_t *wr0 = slot + l16 * kPRowBytes;
                const uint8_t *wq_s = slot + l16 * 128;                 // split: row's 8 nibble blocks
                const _Float16 *wd_s = reinterpret_cast<const _Float16 *>(slot + 2048 + l16 * 16);  // its 8 scales
                {
                    f16x4 dw_op;
                    if constexpr (SPLIT) {
                        dw_op = *reinterpret_cast<const f16x4 *>(wd_s + 4 * (g & 1));
                    } else {
                        const _Float16 *dr = reinterpret_cast<const _Float16 *>(wr0 + (g & 1) * 4 * kQ4BlockBytes);
#pragma unroll
                        for (int q = 0; q < 4; ++q) dw_op[q] = dr[q * kQ4BlockBytes / 2];
                    }
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(sx_op, dw_op, acc[t], 0, 0, 0);
                }
#pragma unroll
                for (int p = 0; p < kPStageBlocks / 2; ++p) {
                    uint32_t q0, q1;
                    _Float16 dw;
                    if constexpr (SPLIT) {
                        const uint2 qq =
                            *reinterpret_cast<const uint2 *>(wq_s + ((2 * p + po) ^ (l16 & 7)) * 16 + 8 * kc);
                        q0 = qq.x;
                        q1 = qq.y;
                        dw = wd_s[2 * p + po];
                    } else {
                        // qs bytes 8kc..8kc+7 of block 2p + po of this lane's weight row: at byte
                        // 18*bb + 2 + 8kc of the row, 2 mod 4 for even blocks, 0 mod 4 for odd ones.
                        const int off = (2 * p + po) * kQ4BlockBytes + 2 + 8 * kc;
                        const uint32_t *pp = reinterpret_cast<const uint32_t *>(wr0 + (off & ~3));
                        const uint32_t sh = off & 3;
                        const uint32_t d0 = pp[0], d1 = pp[1], d2 = pp[sh ? 2 : 1];
                        q0 = __builtin_amdgcn_alignbyte(d1, d0, sh);
                        q1 = __builtin_amdgcn_alignbyte(d2, d1, sh);
                        dw = *reinterpret_cast<const _Float16 *>(wr0 + (2 * p + po) * kQ4BlockBytes);
                    }
                    const i32x4 bop = i32x4{(int32_t)(q0 & 0x0f0f0f0fu), (int32_t)(q1 & 0x0f0f0f0fu),
                                            (int32_t)((q0 >> 4) & 0x0f0f0f0fu), (int32_t)((q1 >> 4) & 0x0f0f0f0fu)};
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop[p], bop, bias, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float tt = fmaf(__int_as_float(d[i]), dx8[p][i], nb8[p][i]);
                        acc[t][i] = fmaf((float)dw, tt, acc[t][i]);
                    }
                }
                asm volatile("" : "+v"(acc[t]));  // keep the tile's epilogue here
                refill(it, j, t);
            }
        }
        } else {
        for (int j = 0; j < my_st; ++j) {
            // stage operands from the wave's copy of stage wave + 8j (registers, reused for all tiles)
            const uint8_t *xst = xw + j * 2 * x_stride_sb;
            long aop[kPStageBlocks];
            f32x4 dx8[kPStageBlocks], nb8[kPStageBlocks];
            f16x4 sx_op;
            {
#pragma unroll
                for (int bb = 0; bb < kPStageBlocks; ++bb) {
                    const int h = bb >> 2, jj = bb & 3;
                    const uint32_t *qa = reinterpret_cast<const uint32_t *>(xst + h * x_stride_sb +
                                                                            tok * kQ8BlockBytes + 16 + 32 * jj + 4 * g);
                    aop[bb] = (long)((uint64_t)qa[4] << 32 | qa[0]);
                }
                // d_x of tokens 4g..4g+3 (the output rows of this lane)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = min(4 * g + i, M - 1);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint4 v = *reinterpret_cast<const uint4 *>(xst + h * x_stride_sb + m * kQ8BlockBytes);
                        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) {
                            const float d8 = __half2float(__ushort_as_half((unsigned short)(vv[jj] & 0xffffu))) * 0.125f;
                            dx8[4 * h + jj][i] = d8;
                            nb8[4 * h + jj][i] = -kPBias * d8;
                        }
                    }
                }
                // -s_x of the stage's 8 blocks as the f16 A operand of the s_x MFMA:
                // lane (token l16, group g < 2) holds blocks 4g..4g+3; groups 2, 3 are zero.
                const uint4 v = *reinterpret_cast<const uint4 *>(xst + (g & 1) * x_stride_sb + tok * kQ8BlockBytes);
                const uint32_t keep = g < 2 ? 0xffffffffu : 0u;
                const uint32_t lo = (__builtin_amdgcn_perm(v.y, v.x, 0x07060302u) ^ 0x80008000u) & keep;
                const uint32_t hi = (__builtin_amdgcn_perm(v.w, v.z, 0x07060302u) ^ 0x80008000u) & keep;
                sx_op = __builtin_bit_cast(f16x4, (uint64_t)hi << 32 | lo);
            }
#pragma unroll
            for (int t = 0; t < kPMaxTiles; ++t) {
                if (t >= T) break;  // workgroup-uniform
                // one tile at a time: no hoisting of the next tile's operand reads
                __builtin_amdgcn_sched_barrier(0);
                const int it = j * T + t;
                if (it + 1 < n_items) JJO_P_VMCNT(3); else JJO_P_VMCNT(0);  // item it has landed
                const uint8_t *slot = ring + (it % kPRing) * kPItemBytes;
                const uint8_t *wr0 = slot + l16 * kPRowBytes;
                const uint8_t *wq_s = slot + l16 * 128;
                const _Float16 *wd_s = reinterpret_cast<const _Float16 *>(slot + 2048 + l16 * 16);
                // s_x term: d_w of blocks 4(g&1)..4(g&1)+3 of this lane's weight row
                {
                    f16x4 dw_op;
                    if constexpr (SPLIT) {
                        dw_op = *reinterpret_cast<const f16x4 *>(wd_s + 4 * (g & 1));
                    } else {
                        const _Float16 *dr = reinterpret_cast<const _Float16 *>(wr0 + (g & 1) * 4 * kQ4BlockBytes);
#pragma unroll
                        for (int q = 0; q < 4; ++q) dw_op[q] = dr[q * kQ4BlockBytes / 2];
                    }
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(sx_op, dw_op, acc[t], 0, 0, 0);
                }
#pragma unroll
                for (int bb = 0; bb < kPStageBlocks; ++bb) {
                    uint32_t q;
                    _Float16 dw;
                    if constexpr (SPLIT) {
                        q = *reinterpret_cast<const uint32_t *>(wq_s + (bb ^ (l16 & 7)) * 16 + 4 * g);
                        dw = wd_s[bb];
                    } else {
                        const uint8_t *wr = wr0 + bb * kQ4BlockBytes;
                        if ((bb & 1) == 0) {  // nibble dword g at 2 mod 4: re-align
                            const uint32_t *p = reinterpret_cast<const uint32_t *>(wr + 4 * g);
                            q = __builtin_amdgcn_alignbyte(p[1], p[0], 2);
                        } else {
                            q = *reinterpret_cast<const uint32_t *>(wr + 2 + 4 * g);
                        }
                        dw = *reinterpret_cast<const _Float16 *>(wr);
                    }
                    const long bop = (long)((uint64_t)((q >> 4) & 0x0f0f0f0fu) << 32 | (q & 0x0f0f0f0fu));
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[bb], bop, bias, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float tt = fmaf(__int_as_float(d[i]), dx8[bb][i], nb8[bb][i]);
                        acc[t][i] = fmaf((float)dw, tt, acc[t][i]);
                    }
                }
                asm volatile("" : "+v"(acc[t]));  // keep the tile's epilogue here
                refill(it, j, t);
            }
        }
        }
        JJO_P_VMCNT(0);  // the wave's activation copy and ring are free again
    }

    // ---- K-slice partials of each tile -> LDS, summed in wave order ----
    __syncthreads();
    f32x4 *red = reinterpret_cast<f32x4 *>(smem);
#pragma unroll
    for (int t = 0; t < kPMaxTiles; ++t)
        if (t < T) red[(t * kPW + wave) * 64 + lane] = acc[t];
    __syncthreads();
    if (wave < T) {
        const int t = wave;
        f32x4 sum = red[(t * kPW + 0) * 64 + lane];
#pragma unroll
        for (int k = 1; k < kPW; ++k) sum = sum + red[(t * kPW + k) * 64 + lane];
        if constexpr (PAIR) {
            // lanes g and g + 2 hold the two block parities of tokens 4(g & 1)..+3
            f32x4 odd = red[(t * kPW + 0) * 64 + (lane ^ 32)];
#pragma unroll
            for (int k = 1; k < kPW; ++k) odd = odd + red[(t * kPW + k) * 64 + (lane ^ 32)];
            sum = sum + odd;
        }
        const int n = (tile0 + t) * 16 + l16;
        if (n < N && (!PAIR || g < 2)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * g + i;
                if (m < M) y[(size_t)m * N + n] = 8.0f * sum[i];
            }
        }
    }
}

}  // namespace

bool gemm_skinny_persist_supported(const void *w, const void *xq, int K, int M) {
    return K % 256 == 0 && M >= 1 && M <= 16 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)xq & 15) == 0;
}

hipError_t launch_gemm_skinny_persist_layout(const void *w, const void *xq, float *y, int K, int N, int M, bool split,
                                             hipStream_t stream) {
    if (!gemm_skinny_persist_supported(w, xq, K, M)) return hipErrorInvalidValue;
    const void *kern = M <= 8 ? (split ? (const void *)gemm_skinny_persist_kernel<true, true>
                                       : (const void *)gemm_skinny_persist_kernel<true, false>)
                              : (split ? (const void *)gemm_skinny_persist_kernel<false, true>
                                       : (const void *)gemm_skinny_persist_kernel<false, false>);
    hipError_t e = ensure_dynamic_lds(kern, kPSmemBytes);
    if (e != hipSuccess) return e;
    const int n_tiles = (N + 15) / 16;
    const int tiles_per_wg = min(kPMaxTiles, (n_tiles + 255) / 256);
    const int blocks = (n_tiles + tiles_per_wg - 1) / tiles_per_wg;
#define JJO_P_LAUNCH(P, S)                                                                                    \
    hipLaunchKernelGGL((gemm_skinny_persist_kernel<P, S>), dim3(blocks), dim3(64 * kPW), kPSmemBytes, stream, \
                       (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M, tiles_per_wg)
    if (M <= 8) {
        if (split) JJO_P_LAUNCH(true, true); else JJO_P_LAUNCH(true, false);
    } else {
        if (split) JJO_P_LAUNCH(false, true); else JJO_P_LAUNCH(false, false);
    }
#undef JJO_P_LAUNCH
    return hipGetLastError();
}

hipError_t launch_gemm_skinny_persist(const void *w, const void *xq, float *y, int K, int N, int M,
                                      hipStream_t stream) {
    return launch_gemm_skinny_persist_layout(w, xq, y, K, N, M, false, stream);
}

}  // namespace jjo
