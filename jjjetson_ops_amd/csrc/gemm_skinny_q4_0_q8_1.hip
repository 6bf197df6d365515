// Small-batch (M <= 32) Q4_0 x Q8_1 matmul on gfx950 int8 matrix cores.
//
// Math is the reference's per-block epilogue (src/cuda/mm_q4_0_q8_1.cu:71-93):
//     y[m][n] = sum_b d_w[n,b] * (sumi[n,m,b] * d_x[m,b] - 8 * s_x[m,b])
//
// At batch 2..32 the weight stream (0.5625 B per weight) still bounds the work, but
// the per-token dot products no longer fit the VALU of a dot-product GEMV.  Here the
// integer sums run on v_mfma_i32_16x16x32_i8 with the tokens as the MFMA rows and 16
// weight rows as its columns, so one MFMA = 16 tokens x 16 weight rows x one 32-wide
// K block, and an output lane holds four tokens of ONE weight row (one d_w per lane).
//
//   * Workgroup = 4 waves = 4 interleaved K-slices of the same RT*16 weight rows
//     (wave w takes stages w, w+4, ...).  Each wave streams its slice through its
//     own LDS ring of P stages; a stage is 8 K blocks:
//       weights:     RT*16 rows x 144 B (8 Q4_0 blocks), row-major, 144 B per row
//       activation:  the 2 Q8_1 superblocks of the stage for all M tokens, copied as
//                    the one contiguous 288*M-byte run they occupy in the
//                    quantizer's superblock-major layout
//     Both move with global_load_lds_dwordx4 (global -> LDS, no VGPRs), so a stage is
//     ~10 wide load instructions.  The wave waits for a stage with an explicit
//     s_waitcnt vmcnt(n) (n = loads issued for the stages still in flight); there is
//     no barrier inside the K loop.  The K-slice partials are added through LDS in
//     slice order at the end.
//   * K positions inside a block are permuted consistently for both operands: MFMA
//     k-group g (lanes 16g..16g+15) takes the nibble byte dword g of the Q4_0 block,
//     i.e. elements 4g..4g+3 (low nibbles) and 16+4g..16+4g+3 (high nibbles), and
//     activation dwords g and g+4 (one ds_read2_b32).
//   * The MFMA accumulator starts at 0x4B400000 (the bits of 1.5*2^23), so the
//     result read as fp32 is 1.5*2^23 + sumi exactly and the epilogue needs no
//     convert; two VALU ops per element and block:
//         t = fma(D, d_x/8, -1.5*2^23 * d_x/8)     (= round(sumi*d_x)/8)
//         acc += d_w * t                            (v_fma_mix: d_w stays fp16)
//     The (d_x/8, -1.5*2^23*d_x/8) pairs of a stage are converted once per stage
//     into a wave-private LDS table.
//   * The -8*s_x term, sum_b d_w[n,b]*s_x[m,b], is itself a contraction over the
//     blocks: one v_mfma_f32_16x16x16_f16 per stage and tile adds -d_w*s_x for the
//     stage's 8 blocks into the same accumulator (fp16 x fp16 products are exact
//     in fp32).  y = 8*acc.
//
// SPLIT: weights in the split layout (nibble plane + fp16 scale plane).  A stage of
// RT*16 rows is then RT*16 x 128 nibble bytes (block j of row r in slot j ^ (r & 7) of
// the row, against LDS bank conflicts) followed by the rows' 16-byte runs of 8 scales:
// the same RT*2304 bytes and the same 2*RT + 1 DMA instructions (RT = 1, 2), with
// aligned operand reads.
//
// Requirements (checked by the launcher): K % 256 == 0, w and xq 16-byte aligned.
#include <hip/hip_fp16.h>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kStageBlocks = 8;
constexpr int kStageRowBytes = kStageBlocks * kQ4BlockBytes;  // 144
constexpr uint32_t kBiasBits = 0x4B400000u;
constexpr float kBias = 12582912.0f;

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] + [15:14],
// expcnt[6:4] = 7, lgkmcnt[11:8] = 15).
#define JJO_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n)&15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
#define JJO_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)  // lgkmcnt(0); vmcnt 63 and expcnt 7 (no wait)
// runtime wave-uniform count -> immediate
__device__ __forceinline__ void vm_wait(int n) {
    switch (n) {
#define C_(k) \
    case k: JJO_VMCNT(k); break;
        C_(0) C_(1) C_(2) C_(3) C_(4) C_(5) C_(6) C_(7) C_(8) C_(9) C_(10) C_(11) C_(12) C_(13) C_(14) C_(15)
        C_(16) C_(17) C_(18) C_(19) C_(20) C_(21) C_(22) C_(23) C_(24) C_(25) C_(26) C_(27) C_(28) C_(29)
        C_(30) C_(31)
#undef C_
        default: JJO_VMCNT(0); break;
    }
}

template <int RT, int CT>
struct Geo {
    static constexpr int kWChunks = RT * 16 * (kStageRowBytes / 16);  // 16-B chunks per stage
    static constexpr int kWInstr = (kWChunks + 63) / 64;
    static constexpr int kWBytes = kWChunks * 16;                    // RT * 2304
    static constexpr int kXBytes = 2 * kQ8BlockBytes * 16 * CT;      // 288 * 16 * CT (max M)
    static constexpr int kXInstrMax = (kXBytes / 16 + 63) / 64;
    static constexpr int kStageBytes = kWBytes + kXBytes;
    static constexpr int kScBytes = kStageBlocks * 2 * 16 * CT * 4;   // dx8, nb8 per block/token
};

template <int RT, int CT, int P, int KW>
struct Lds {
    static constexpr int kWaveBytes = P * Geo<RT, CT>::kStageBytes + Geo<RT, CT>::kScBytes;
    static constexpr int kBytes = KW * kWaveBytes;
    static constexpr int kRedBytes = KW * RT * CT * 64 * 16;
    static_assert(kRedBytes <= kBytes, "reduction area must fit the rings");
};


template <int RT, int CT, int P, int KW, bool SPLIT = false>
__global__ __launch_bounds__(64 * KW) void gemm_skinny_kernel(const uint8_t *__restrict__ w,
                                                                  const uint8_t *__restrict__ xq,
                                                                  float *__restrict__ y, int K, int N, int M) {
    using G = Geo<RT, CT>;
    using L = Lds<RT, CT, P, KW>;
    __shared__ __align__(16) uint8_t smem[L::kBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    const int nb = K / kQK;
    const int n_stages = nb / kStageBlocks;
    const size_t row_bytes = (size_t)nb * kQ4BlockBytes;
    const int n0 = blockIdx.x * (16 * RT);

    // Stages of this wave: wave, wave + 4, wave + 8, ...  The 4 waves of the
    // workgroup read adjacent 144-byte pieces of the same rows at the same time,
    // 576 contiguous bytes per row, which keeps HBM pages and L2 lines shared.
    const int n_my = (n_stages - wave + KW - 1) / KW;

    uint8_t *ring = smem + wave * L::kWaveBytes;
    float *sc = reinterpret_cast<float *>(ring + P * G::kStageBytes);

    // ---- per-lane DMA sources ----
    // weights: chunk c = 64*i + lane -> row c/9, 16-B piece c%9 of the row's stage bytes
    uint32_t w_off[G::kWInstr];
#pragma unroll
    for (int i = 0; i < G::kWInstr; ++i) {
        const int c = min(64 * i + lane, G::kWChunks - 1);
        const int r = c / 9, piece = c % 9;
        const int row = min(n0 + r, N - 1);
        w_off[i] = (uint32_t)((size_t)(row - n0) * row_bytes) + 16u * piece;
    }
    const uint8_t *w_base = w + (size_t)n0 * row_bytes;
    // Split layout: nibble chunk c = 64*i + lane -> row c / 8 of the tile, slot c % 8
    // holding block (c % 8) ^ (row & 7) of the stage; scale run of row `lane` (< RT*16).
    static_assert(!SPLIT || 2 * RT + 1 == G::kWInstr, "split stages use the block layout's DMA count");
    uint32_t ws_off[2 * RT];
#pragma unroll
    for (int i = 0; i < 2 * RT; ++i) {
        const int c = 64 * i + lane, rr = c >> 3;
        const int row = min(n0 + rr, N - 1);
        ws_off[i] = (uint32_t)((size_t)(row - n0) * nb * 16) + 16u * (uint32_t)((c & 7) ^ (rr & 7));
    }
    const uint8_t *ws_base = w + (size_t)n0 * nb * 16;
    const uint8_t *wd_base = w + (size_t)N * nb * 16 + (size_t)n0 * nb * 2;
    const uint32_t wd_off = (uint32_t)((size_t)(min(n0 + lane, N - 1) - n0) * nb * 2);
    constexpr int kSplitNibBytes = RT * 16 * 128;  // scales follow the nibbles in a stage
    // activation: the stage's 288*M contiguous bytes
    const int x_run = 2 * kQ8BlockBytes * M;
    const int x_chunks = x_run / 16;
    const int x_instr = (x_chunks + 63) / 64;  // wave-uniform, <= kXInstrMax
    const int per_stage = G::kWInstr + x_instr;

    auto issue = [&](int s) {  // stage s of this wave's slice into slot s % P
        uint8_t *st = ring + (s % P) * G::kStageBytes;
        const int gs = wave + KW * s;
        if constexpr (SPLIT) {
            const size_t blk0 = (size_t)gs * kStageBlocks;
#pragma unroll
            for (int i = 0; i < 2 * RT; ++i)
                __builtin_amdgcn_global_load_lds((const void *)(ws_base + blk0 * 16 + ws_off[i]),
                                                 (lds_void *)(st + 1024 * i), 16, 0, 0);
            if (lane < RT * 16)
                __builtin_amdgcn_global_load_lds((const void *)(wd_base + blk0 * 2 + wd_off),
                                                 (lds_void *)(st + kSplitNibBytes), 16, 0, 0);
        } else {
        const uint8_t *ws = w_base + (size_t)gs * kStageRowBytes;
#pragma unroll
        for (int i = 0; i < G::kWInstr; ++i) {
            if (64 * i + lane < G::kWChunks || (G::kWChunks % 64) == 0)
                __builtin_amdgcn_global_load_lds((const void *)(ws + w_off[i]), (lds_void *)(st + 1024 * i), 16, 0, 0);
        }
        }
        const uint8_t *xs = xq + (size_t)gs * x_run;
        uint8_t *xd = st + G::kWBytes;
#pragma unroll
        for (int i = 0; i < G::kXInstrMax; ++i) {
            if (i < x_instr) {  // wave-uniform
                const int c = 64 * i + lane;
                if (c < x_chunks)
                    __builtin_amdgcn_global_load_lds((const void *)(xs + 16 * c), (lds_void *)(xd + 1024 * i), 16, 0,
                                                     0);
            }
        }
    };

    i32x4 bias;
#pragma unroll
    for (int i = 0; i < 4; ++i) bias[i] = (int32_t)kBiasBits;
    f32x4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    // token rows this lane feeds to the MFMA (clamped: rows >= M are never stored)
    int a_tok_row[CT], a_tok_off[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        a_tok_row[ct] = min(16 * ct + l16, M - 1) * kQ8BlockBytes;
        a_tok_off[ct] = a_tok_row[ct] + 16 + 4 * g;
    }

    auto consume = [&](int s) {
        const uint8_t *st = ring + (s % P) * G::kStageBytes;
        const uint8_t *xs = st + G::kWBytes;
        // activation scales of the stage -> sc[b][{dx8, nb8}][token]
        if (lane < 32 * CT) {
            const int m = lane & (16 * CT - 1), h = lane / (16 * CT);
            const uint4 v = *reinterpret_cast<const uint4 *>(xs + h * kQ8BlockBytes * M + min(m, M - 1) * kQ8BlockBytes);
            const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float dx8 = __half2float(__ushort_as_half((unsigned short)(vv[j] & 0xffffu))) * 0.125f;
                float *row = sc + (4 * h + j) * 2 * 16 * CT;
                row[m] = dx8;
                row[16 * CT + m] = -kBias * dx8;
            }
        }
        // The table is written as floats and read below as float4: keep type-based
        // alias analysis from moving those reads above these writes.
        asm volatile("" ::: "memory");
        // -s_x of the stage's 8 blocks as the f16 A operand of the s_x MFMA: lane
        // (token l16, group g < 2) holds blocks 4g..4g+3; groups 2, 3 are zero.
        f16x4 sx_op[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const uint4 v = *reinterpret_cast<const uint4 *>(xs + (g & 1) * kQ8BlockBytes * M + a_tok_row[ct]);
            const uint32_t keep = g < 2 ? 0xffffffffu : 0u;
            const uint32_t lo = (__builtin_amdgcn_perm(v.y, v.x, 0x07060302u) ^ 0x80008000u) & keep;
            const uint32_t hi = (__builtin_amdgcn_perm(v.w, v.z, 0x07060302u) ^ 0x80008000u) & keep;
            sx_op[ct] = __builtin_bit_cast(f16x4, (uint64_t)hi << 32 | lo);
        }
        // d_w of blocks 4(g&1)..4(g&1)+3 of this lane's weight row: the B operand of the s_x MFMA
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            f16x4 dw_op;
            if constexpr (SPLIT) {
                dw_op = *reinterpret_cast<const f16x4 *>(st + kSplitNibBytes + (rt * 16 + l16) * 16 + 8 * (g & 1));
            } else {
                const _Float16 *dr = reinterpret_cast<const _Float16 *>(st + (rt * 16 + l16) * kStageRowBytes +
                                                                        (g & 1) * 4 * kQ4BlockBytes);
#pragma unroll
                for (int j = 0; j < 4; ++j) dw_op[j] = dr[j * kQ4BlockBytes / 2];
            }
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(sx_op[ct], dw_op, acc[rt][ct], 0, 0, 0);
        }
#pragma unroll
        for (int bb = 0; bb < kStageBlocks; ++bb) {
            const int h = bb >> 2, j = bb & 3;
            long aop[CT];
            f32x4 dx8[CT], nb8[CT];
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                // activation dwords g and g+4 of the block: elements 4g..4g+3 and 16+4g..16+4g+3
                const uint32_t *qa =
                    reinterpret_cast<const uint32_t *>(xs + h * kQ8BlockBytes * M + a_tok_off[ct] + 32 * j);
                aop[ct] = (long)((uint64_t)qa[4] << 32 | qa[0]);
                const float *row = sc + bb * 2 * 16 * CT + 16 * ct + 4 * g;
                dx8[ct] = *reinterpret_cast<const f32x4 *>(row);
                nb8[ct] = *reinterpret_cast<const f32x4 *>(row + 16 * CT);
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                uint32_t q;
                _Float16 dw;
                if constexpr (SPLIT) {
                    q = *reinterpret_cast<const uint32_t *>(st + (rt * 16 + l16) * 128 + (bb ^ (l16 & 7)) * 16 + 4 * g);
                    dw = reinterpret_cast<const _Float16 *>(st + kSplitNibBytes + (rt * 16 + l16) * 16)[bb];
                } else {
                const uint8_t *wr = st + (rt * 16 + l16) * kStageRowBytes + bb * kQ4BlockBytes;
                if ((bb & 1) == 0) {  // nibble dword g at 2 mod 4: re-align
                    const uint32_t *p = reinterpret_cast<const uint32_t *>(wr + 4 * g);
                    q = __builtin_amdgcn_alignbyte(p[1], p[0], 2);
                } else {
                    q = *reinterpret_cast<const uint32_t *>(wr + 2 + 4 * g);
                }
                dw = *reinterpret_cast<const _Float16 *>(wr);
                }
                const long bop = (long)((uint64_t)((q >> 4) & 0x0f0f0f0fu) << 32 | (q & 0x0f0f0f0fu));
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[ct], bop, bias, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float t = fmaf(__int_as_float(d[i]), dx8[ct][i], nb8[ct][i]);
                        acc[rt][ct][i] = fmaf((float)dw, t, acc[rt][ct][i]);
                    }
                }
            }
        }
    };

    if (n_my > 0) {
        const int pre = min(P, n_my);
        for (int s = 0; s < pre; ++s) issue(s);
        for (int s = 0; s < n_my; ++s) {
            const int ahead = min(P, n_my - s) - 1;  // stages issued after s
            vm_wait(ahead * per_stage);
            __builtin_amdgcn_sched_barrier(0);
            consume(s);
            __builtin_amdgcn_sched_barrier(0);
            if (s + P < n_my) {
                JJO_LGKM0();  // slot s % P fully read before it is refilled
                __builtin_amdgcn_sched_barrier(0);
                issue(s + P);
            }
        }
    }

    // K-slice partials -> LDS (over the rings), summed in slice order by wave 0.
    __syncthreads();
    f32x4 *red = reinterpret_cast<f32x4 *>(smem);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) red[((wave * RT + rt) * CT + ct) * 64 + lane] = acc[rt][ct];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                f32x4 sum = red[((0 * RT + rt) * CT + ct) * 64 + lane];
#pragma unroll
                for (int k = 1; k < KW; ++k) sum = sum + red[((k * RT + rt) * CT + ct) * 64 + lane];
                const int n = n0 + 16 * rt + l16;
                if (n < N) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int m = 16 * ct + 4 * g + i;
                        if (m < M) y[(size_t)m * N + n] = 8.0f * sum[i];
                    }
                }
            }
    }
}

template <int RT, int CT, int P, int KW>
hipError_t launch_rcp(const void *w, const void *xq, float *y, int K, int N, int M, bool split, hipStream_t stream) {
    const int blocks = (N + 16 * RT - 1) / (16 * RT);
    if (split)
        hipLaunchKernelGGL((gemm_skinny_kernel<RT, CT, P, KW, true>), dim3(blocks), dim3(64 * KW), 0, stream,
                           (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M);
    else
        hipLaunchKernelGGL((gemm_skinny_kernel<RT, CT, P, KW, false>), dim3(blocks), dim3(64 * KW), 0, stream,
                           (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M);
    return hipGetLastError();
}

}  // namespace

// Row tiles per workgroup on large-N matrices and LDS ring depth per wave.
constexpr int kSkinnyRt = 2;
constexpr int kSkinnyP = 2;

bool gemm_skinny_supported(const void *w, const void *xq, int K, int M) {
    return K % 256 == 0 && M >= 1 && M <= kSkinnyMaxBatch && ((uintptr_t)w & 15) == 0 && ((uintptr_t)xq & 15) == 0;
}

hipError_t launch_gemm_skinny_layout(const void *w, const void *xq, float *y, int K, int N, int M, bool split,
                                     hipStream_t stream) {
    if (!gemm_skinny_supported(w, xq, K, M)) return hipErrorInvalidValue;
    if (M <= 16) {
        // 32-row workgroups of 4 K-slice waves while that fills the chip; for short
        // matrices (N < 8192) 16-row workgroups of 8 K-slice waves (twice the
        // workgroups, each CU holding one).
        if ((N + 31) / 32 >= 256) return launch_rcp<kSkinnyRt, 1, kSkinnyP, 4>(w, xq, y, K, N, M, split, stream);
        return launch_rcp<1, 1, kSkinnyP, 8>(w, xq, y, K, N, M, split, stream);
    }
    return launch_rcp<kSkinnyRt, 2, kSkinnyP, 4>(w, xq, y, K, N, M, split, stream);
}

hipError_t launch_gemm_skinny(const void *w, const void *xq, float *y, int K, int N, int M, hipStream_t stream) {
    return launch_gemm_skinny_layout(w, xq, y, K, N, M, false, stream);
}

}  // namespace jjo
