// Prefill / MoE-expert GEMM of Q4_0 weights x Q8_1 activations on gfx950
// int8 matrix cores.
//
// Math is the reference's per-block epilogue (src/cuda/mm_q4_0_q8_1.cu:71-93,
// summed over K at :256-269):
//     y[m][n] = sum_b d_w[n,b] * (sumi[n,m,b] * d_x[m,b] - 8 * s_x[m,b])
// with sumi the exact unsigned-nibble x int8 dot of one 32-block.
//
// MI355X design
//   * One v_mfma_i32_32x32x32_i8 covers exactly one 32-wide K block, so each
//     MFMA result is the exact int32 `sumi` tile of one block.
//   * The MFMA accumulator is seeded with the integer 0x4B400000 (the bits of
//     the float 1.5*2^23): after the MFMA adds sumi (|sumi| < 2^16) the register
//     read as fp32 is exactly 1.5*2^23 + sumi.  The epilogue is then two fp32
//     ops per element and block, with no int->float conversion:
//         t   = fma(D_as_float, d_x/8, -1.5*2^23 * d_x/8)   (= round(sumi*d_x)/8)
//         acc = fma(d_w (fp32, converted once when staged), t, acc)
//   * The "-8 * s_x" term, sum_b d_w[n,b] * s_x[m,b], is itself a contraction
//     over blocks: one v_mfma_f32_32x32x8_f16 per 8 blocks adds
//     sum_b d_w * (-s_x) into the same accumulator (fp16 x fp16 products are
//     exact in fp32).  The result is y = 8 * acc (exact power-of-two scale).
//   * Those two fp32 ops per element-block bound this kernel: 2 VALU lane-ops
//     per 64 int8 MACs+adds.  gfx950 retires plain v_fma_f32 at up to 32 lanes
//     per clock per SIMD (128 per CU) against 8192 int8 ops/clk/CU, i.e. twice
//     the MFMA time: about 50% of int8 peak at best.  A v_fma_mix_f32 (fp16
//     operand) issues at about half the plain rate, hence fp32 scales.
//   * Workgroup tile 128 (weight rows) x 128 (tokens) x 128 (K per stage);
//     four waves in 2x2, each owning 2x2 MFMA tiles of 32x32.
//   * Weights are staged once per workgroup: raw 18-byte blocks (dwordx4
//     loads), nibbles expanded to int8 in K order while writing LDS, scales
//     stored twice (fp16 row-major for the f16 MFMA, and as fp32 permuted so a
//     lane's 16 epilogue rows are one 64-byte run).
//   * Activations use the quantizer's superblock-major layout: for a fixed
//     superblock the 128 tokens of a tile are one contiguous 18 KB run, copied
//     to LDS verbatim with 16-byte loads.
//   * Next stage's global loads are issued into registers before the current
//     stage's MFMA/epilogue work (register double buffering).
#include <hip/hip_fp16.h>

#include <type_traits>

#include "mfma_q4q8_tile.hpp"
#include "q4q8_common.hpp"
#include "q8_1_quant.hpp"

namespace jjo {
namespace {

constexpr int BN = 128;          // weight rows per workgroup
constexpr int BM = 128;          // tokens per workgroup
constexpr int KB = 4;            // 32-blocks per stage (K = 128: one Q8_1 superblock)
constexpr int kThreads = 256;

// LDS carve-up (bytes).  Activation and weight tiles are both double-buffered:
// 78 KB per workgroup, so two workgroups share a CU.
constexpr int kXsBytes = BM * kQ8BlockBytes;             // 18432 per stage: [BM][144]
constexpr int kWqStride = KB * 32 + 16;                  // 144: one row's 4 unpacked blocks + pad
constexpr int kWqBytes = BN * kWqStride;                 // 18432
constexpr int kWdEpiBytes = KB * BN * 4;                 // [KB][BN] fp32, rows permuted
constexpr int kWdRowBytes = BN * KB * 2;                 // [BN][KB] fp16
constexpr int kWBufBytes = kWqBytes + kWdEpiBytes + kWdRowBytes;  // one weight stage
constexpr int kOffW = 2 * kXsBytes;
constexpr int kOffWdEpi = kWqBytes;                      // offsets inside a weight stage
constexpr int kOffWdRow = kWqBytes + kWdEpiBytes;
constexpr int kSmemBytes = kOffW + 2 * kWBufBytes;       // 79872
constexpr int kXUnits = kXsBytes / 16;                   // 1152 16-byte units per stage
constexpr int kXRuns = kXUnits / 64;                     // 18 wave-sized (1 KB) runs


// kSwiglu (grouped, two stacked matrices): the workgroup's 128 rows are rows
// 64x..64x+63 of the gate matrix (tile rows 0..63) and of the up matrix (tile rows
// 64..127), x = blockIdx.x; instead of storing them it writes the Q8_1 bytes of
// silu(gate) * up for those 64 intermediate values of each route to `midq`
// (superblock-major over the M routes, as the quantizer lays out a [M][n_split]
// activation).  n_split is the intermediate size I.
// kSplit: the weights are in the split layout (a nibble plane, then an fp16 scale
// plane, over all rows of the buffer: the stacked experts of a grouped launch, each
// of w and w2 on its own); the staging thread's two blocks are then 32 contiguous
// nibble bytes and one scale dword, the same three loads and nine registers.
template <bool kGrouped, bool kSwiglu = false, bool kSplit = false>
__global__ __launch_bounds__(kThreads, 2) void gemm_q4_0_q8_1_mfma_kernel(
    const uint8_t *__restrict__ w_all, const uint8_t *__restrict__ xq, float *__restrict__ y, int K,
    int N, int M, const int32_t *__restrict__ expert_offsets, int n_experts,
    const int32_t *__restrict__ route_dst, const uint8_t *__restrict__ w2, int n_split,
    uint8_t *__restrict__ midq = nullptr) {
    static_assert(kGrouped || !kSwiglu, "the fused SwiGLU epilogue is for the grouped gate|up launch");
    extern __shared__ __align__(16) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave >> 1;  // row half of the workgroup tile
    const int wm = wave & 1;   // token half
    const int l32 = lane & 31;
    const int hh = lane >> 5;  // K half inside an MFMA operand / row group in the output

    const int n0 = blockIdx.x * BN;
    const size_t row_bytes = (size_t)(K / kQK) * kQ4BlockBytes;
    const int nb = K / kQK;
    const int n_stages = nb / KB;  // K % 128 == 0

    // ---- token range of this workgroup ----
    int m0, m_end;
    const uint8_t *w = w_all;
    int expert = 0;
    if constexpr (kGrouped) {
        // Tile t of the concatenated per-expert tile lists: first every tile with more
        // than 32 tokens (expert by expert), then every short tail tile (at most 32
        // tokens, run narrow below).  The long tiles thus start in the first rounds of
        // the grid and the short ones fill its ragged end.
        // Searched 64 experts per step: lane i takes expert e0 + i, a lane prefix sum of
        // the tile counts and a ballot find the expert that holds tile t (the same
        // enumeration as a walk over the experts, in O(E / 64) steps).
        int t = blockIdx.y;
        int e = 0;
        m0 = -1;
        m_end = 0;
        for (int pass = 0; pass < 2 && m0 < 0; ++pass) {
            for (int e0 = 0; e0 < n_experts && m0 < 0; e0 += 64) {
                const int ei = e0 + lane;
                int beg = 0, end = 0, full = 0, tiles = 0;
                if (ei < n_experts) {
                    // Clamped to [0, M] and to beg <= end: a malformed table yields fewer
                    // tiles, never an access outside the activation and output buffers.
                    beg = min(max(expert_offsets[ei], 0), M);
                    end = min(max(expert_offsets[ei + 1], beg), M);
                    full = (end - beg) / BM;
                    const int rem = (end - beg) % BM;
                    tiles = pass == 0 ? full + (rem > 32) : (rem > 0 && rem <= 32);
                }
                int incl = tiles;
#pragma unroll
                for (int d = 1; d < 64; d <<= 1) {
                    const int o = __shfl_up(incl, d);
                    if (lane >= d) incl += o;
                }
                const int total = __shfl(incl, 63);
                if (t < total) {
                    const int f = __builtin_ctzll(__ballot(incl > t));  // the expert holding tile t
                    const int tf = t - (__shfl(incl, f) - __shfl(tiles, f));
                    m0 = __shfl(beg, f) + (pass == 0 ? tf : __shfl(full, f)) * BM;
                    m_end = __shfl(end, f);
                    e = e0 + f;
                } else {
                    t -= total;
                }
            }
        }
        if (m0 < 0) return;  // uniform over the workgroup
        expert = e;
        w = w_all + (size_t)e * (w2 != nullptr ? n_split : N) * row_bytes;
    } else {
        m0 = blockIdx.y * BM;
        m_end = M;
    }

    // ---- staging: weights through registers, activations by LDS DMA ----
    const int st_row = tid >> 1;    // W: one row, one block pair per thread
    const int st_half = tid & 1;
    // Two stacked matrices (w2 != nullptr): rows [0, n_split) from w, rows
    // [n_split, N) from w2 (expert e's block of each); n_split % BN == 0, so a
    // workgroup's rows come from one of them.
    int n_loc0 = n0, n_mat = N;
    const uint8_t *w_src;
    if constexpr (kSwiglu) {
        // Tile rows 0..63: gate rows 64x.., tile rows 64..127: up rows 64x..
        const int ni0 = blockIdx.x * 64;
        const uint8_t *wm = st_row < 64 ? w : w2 + (size_t)expert * n_split * row_bytes;
        w_src = wm + (size_t)min(ni0 + (st_row & 63), n_split - 1) * row_bytes + (size_t)st_half * 36;
    } else {
        if (w2 != nullptr) {
            if (n0 < n_split) {
                n_mat = n_split;
            } else {
                w = w2 + (size_t)expert * (N - n_split) * row_bytes;
                n_loc0 = n0 - n_split;
                n_mat = N - n_split;
            }
        }
        w_src = w + (size_t)min(n_loc0 + st_row, n_mat - 1) * row_bytes + (size_t)st_half * 36;
    }
    // Split layout: the same rows, as (matrix, row of its buffer, rows of its buffer).
    const uint8_t *wq_s = nullptr, *wd_s = nullptr;
    if constexpr (kSplit) {
        const int nb_ = K / kQK;
        const uint8_t *mat;
        int64_t rows_total, row;
        if constexpr (kSwiglu) {
            const int ni0 = blockIdx.x * 64;
            mat = st_row < 64 ? w_all : w2;
            rows_total = (int64_t)n_experts * n_split;
            row = (int64_t)expert * n_split + min(ni0 + (st_row & 63), n_split - 1);
        } else {
            if (kGrouped && w2 != nullptr) {
                const bool first = n0 < n_split;
                const int rows_e = first ? n_split : N - n_split;
                mat = first ? w_all : w2;
                rows_total = (int64_t)n_experts * rows_e;
                row = (int64_t)expert * rows_e + min((first ? n0 : n0 - n_split) + st_row, rows_e - 1);
            } else {
                mat = w_all;
                rows_total = kGrouped ? (int64_t)n_experts * N : N;
                row = (kGrouped ? (int64_t)expert * N : 0) + min(n0 + st_row, N - 1);
            }
        }
        wq_s = mat + ((size_t)row * nb_ + 2 * st_half) * 16;
        wd_s = mat + (size_t)rows_total * nb_ * 16 + ((size_t)row * nb_ + 2 * st_half) * 2;
    }
    // This thread's 2 raw Q4_0 blocks (36 bytes) of a stage, in two register sets:
    // stage k lands in set k & 1, two compute phases before it is unpacked.
    uint32_t wr0[9], wr1[9];

    // Three vector-memory instructions per call (the explicit waits count on it).
    auto load_w = [&](int c, uint32_t(&wst)[9]) {
        if constexpr (kSplit) {
            const uint8_t *pq = wq_s + (size_t)c * (KB * 16);
            const u32x4 a = *reinterpret_cast<const u32x4 *>(pq);
            const u32x4 b = *reinterpret_cast<const u32x4 *>(pq + 16);
            wst[0] = a.x; wst[1] = a.y; wst[2] = a.z; wst[3] = a.w;
            wst[4] = b.x; wst[5] = b.y; wst[6] = b.z; wst[7] = b.w;
            wst[8] = *reinterpret_cast<const uint32_t *>(wd_s + (size_t)c * (KB * 2));
        } else {
            const uint8_t *p = w_src + (size_t)c * (KB * kQ4BlockBytes);
            const u32x4a4 a = *reinterpret_cast<const u32x4a4 *>(p);
            const u32x4a4 b = *reinterpret_cast<const u32x4a4 *>(p + 16);
            wst[0] = a.x; wst[1] = a.y; wst[2] = a.z; wst[3] = a.w;
            wst[4] = b.x; wst[5] = b.y; wst[6] = b.z; wst[7] = b.w;
            wst[8] = *reinterpret_cast<const uint32_t *>(p + 32);
        }
    };

    // Activation tile of stage c = superblock c: tokens m0.. of one contiguous run.
    // Wave `wave` moves 1 KB runs r = wave, wave+4, ... (< 18); lane l moves 16 bytes.
    // Units past the last valid token re-read unit 0 (their LDS bytes are never used
    // with a nonzero scale).
    const size_t x_stride = (size_t)M * kQ8BlockBytes;  // bytes per superblock
    const uint8_t *x_base = xq + (size_t)m0 * kQ8BlockBytes;
    const int x_valid_units = min(BM, m_end - m0) * (kQ8BlockBytes / 16);
    uint32_t x_off[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int unit = min(wave + 4 * i, kXRuns - 1) * 64 + lane;
        x_off[i] = unit < x_valid_units ? unit * 16 : 0;
    }
    // Up to five DMA instructions per wave and call (waves 2 and 3 have four runs;
    // their fifth rewrites run 17 with the same bytes as wave 1).
    // Issued through inline asm: the compiler's wait insertion cannot tell that the
    // DMA target (an activation buffer) is disjoint from the weight buffers that the
    // same iteration writes and reads, and would wait for every load in flight
    // (vmcnt(0)) before the next LDS access, collapsing the weight prefetch.  Their
    // completion is waited for explicitly (the vmcnt(3) before each unpack and the
    // vmcnt(0) after the K loop); the hardware counter counts them like any load.
    auto load_x = [&](int c) {
        const uint32_t xs = (uint32_t)(uintptr_t)(smem + (c & 1) * kXsBytes);
        const uint8_t *src = x_base + (size_t)c * x_stride;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int run = min(wave + 4 * i, kXRuns - 1);
            // Runs past the tile's last token hold nothing a nonzero scale reads
            // (grouped tails): skipped.  Wave-uniform.
            if (run * 64 >= x_valid_units) continue;
            const uint32_t m0v = __builtin_amdgcn_readfirstlane(xs + run * 1024);
            asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src + x_off[i]), "{m0}"(m0v) : "memory");
        }
    };

    auto store_w = [&](int buf, const uint32_t(&wst)[9]) {
        uint8_t *wq = smem + kOffW + buf * kWBufBytes;
        float *wd_epi = reinterpret_cast<float *>(wq + kOffWdEpi);
        _Float16 *wd_row = reinterpret_cast<_Float16 *>(wq + kOffWdRow);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // Even block: scale in the low half of dword 0, nibbles from byte 2 on
            // (re-aligned); odd block: scale in the high half of dword 4, nibbles in
            // dwords 5..8.
            uint32_t q[4];
            uint32_t dbits;
            if constexpr (kSplit) {  // nibbles of block i in dwords 4i..4i+3, both scales in dword 8
                dbits = i == 0 ? (wst[8] & 0xffffu) : (wst[8] >> 16);
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = wst[4 * i + k];
            } else if (i == 0) {
                dbits = wst[0] & 0xffffu;
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = __builtin_amdgcn_alignbyte(wst[k + 1], wst[k], 2);
            } else {
                dbits = wst[4] >> 16;
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = wst[5 + k];
            }
            const int b = st_half * 2 + i;
            u32x4 lo, hi;
            lo.x = q[0] & 0x0f0f0f0fu; lo.y = q[1] & 0x0f0f0f0fu;
            lo.z = q[2] & 0x0f0f0f0fu; lo.w = q[3] & 0x0f0f0f0fu;
            hi.x = (q[0] >> 4) & 0x0f0f0f0fu; hi.y = (q[1] >> 4) & 0x0f0f0f0fu;
            hi.z = (q[2] >> 4) & 0x0f0f0f0fu; hi.w = (q[3] >> 4) & 0x0f0f0f0fu;
            uint8_t *dst = wq + st_row * kWqStride + b * 32;
            *reinterpret_cast<u32x4 *>(dst) = lo;
            *reinterpret_cast<u32x4 *>(dst + 16) = hi;
            const unsigned short dh = (unsigned short)dbits;
            wd_epi[b * BN + (st_row & ~31) + epi_perm(st_row & 31)] = __half2float(__ushort_as_half(dh));
            reinterpret_cast<unsigned short *>(wd_row)[st_row * KB + b] = dh;
        }
    };

    // ---- accumulators ----
    f32x16 acc[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[rt][ct][v] = 0.0f;

    // Paired narrow tiles (grouped, <= 8 tokens): wave w, rows 32w + 16rg + (lane & 15).
    f32x4 acc_p[2];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg) acc_p[rg] = f32x4{0.f, 0.f, 0.f, 0.f};

    i32x16 bias;
#pragma unroll
    for (int v = 0; v < 16; ++v) bias[v] = (int32_t)kBiasBits;
    // Opaque to the optimizer: the 16 bias registers stay resident instead of being
    // re-materialized (16 v_mov) before every MFMA whose result reuses them.
    asm volatile("" : "+v"(bias));

    // Tokens past m_end (a tail tile) hold stale LDS bytes: once an activation tile has
    // landed, their (d, s) headers are zeroed, so every product with them is zero.
    const int x_valid_tokens = min(BM, m_end - m0);
    // At most 8 valid tokens (grouped): the paired narrow layout below masks every
    // other token in its operands, so no headers need zeroing.
    const bool pnarrow = kGrouped && x_valid_tokens <= 8;  // uniform over the workgroup
    auto zero_tail_headers = [&](int buf) {
        if (x_valid_tokens < BM && !pnarrow) {  // uniform over the workgroup
            if (tid >= x_valid_tokens && tid < BM) {
                // Zeros made here (opaque to the optimizer): a zero vector kept from the
                // kernel start was spilled and reloaded with vmcnt(0) in every stage.
                u32x4 z = {0u, 0u, 0u, 0u};
                asm volatile("" : "+v"(z));
                *reinterpret_cast<u32x4 *>(smem + buf * kXsBytes + tid * kQ8BlockBytes) = z;
            }
            __syncthreads();
        }
    };
    // 32-token sub-tiles of this wave that hold valid tokens (grouped tails have 0 or
    // 1): a compile-time parameter of the stage loop below, chosen once per wave.
    // A tile with at most 32 valid tokens (a short tail: an expert's last few routes)
    // runs narrow instead (LIVE = 3, grouped launches only): wave w takes weight rows
    // 32w..32w+31 against tokens 0..31, so the four waves share the tile's one token
    // column evenly.
    const bool narrow = kGrouped && x_valid_tokens <= 32;  // uniform over the workgroup
    const int n_live = pnarrow ? 4 : narrow ? 3 : (m0 + wm * 64 < m_end) + (m0 + wm * 64 + 32 < m_end);

    // Pipeline, one barrier per stage.  While stage c is computed from buffers c&1,
    // X(c+1) (LDS DMA) and the weights of stages c+1 and c+2 (register sets
    // (c+1)&1 and c&1) are in flight.  After the compute, W(c+1) is unpacked into
    // the other weight buffer, one barrier publishes X(c+1) and W(c+1) and retires
    // the reads of buffers c&1, and then X(c+2) (into buffer c&1) and W(c+3) (into
    // the set just unpacked) are issued.  Weight loads thus have two compute phases
    // to land: a grouped GEMM's weight tile is read by one or two workgroups only,
    // so it comes from HBM, not L2.  The explicit vmcnt(3) before each unpack
    // covers X(c+1), which was issued after W(c+1): only W(c+2)'s three loads may
    // still be in flight.
    load_x(0);
    load_w(0, wr0);
    load_w(min(1, n_stages - 1), wr1);
    JJO_GEMM_VMCNT(3);
    store_w(0, wr0);
    __syncthreads();
    zero_tail_headers(0);
    load_x(min(1, n_stages - 1));
    load_w(min(2, n_stages - 1), wr0);

    auto stage_loop = [&](auto live_tag) {
        constexpr int LIVE = decltype(live_tag)::value;
        // One stage; PAR = c & 1 names the register set statically.
        auto stage = [&](int c, auto par_tag) {
            constexpr int PAR = decltype(par_tag)::value;
            uint32_t(&w_next)[9] = *[&]() { if constexpr (PAR) return &wr0; else return &wr1; }();

            uint8_t *wq = smem + kOffW + (c & 1) * kWBufBytes;
            const float *wd_epi = reinterpret_cast<const float *>(wq + kOffWdEpi);
            const _Float16 *wd_row = reinterpret_cast<const _Float16 *>(wq + kOffWdRow);
            const uint8_t *xs = smem + (c & 1) * kXsBytes;

            // Activation headers (d, s) of this lane's two columns (narrow: column l32).
            uint32_t hdr[2][4];
    #pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int col = LIVE == 3 ? l32 : wm * 64 + ct * 32 + l32;
                const u32x4 h = *reinterpret_cast<const u32x4 *>(xs + col * kQ8BlockBytes);
                hdr[ct][0] = h.x; hdr[ct][1] = h.y; hdr[ct][2] = h.z; hdr[ct][3] = h.w;
            }

            if constexpr (LIVE == 4) {
            // Paired narrow tile (at most 8 tokens): v_mfma_i32_16x16x64_i8 with MFMA row
            // r = token r & 7 of block parity r >> 3 and K = the pair of blocks (2p, 2p+1),
            // each row's other block zeroed, so every output is one block's exact sumi;
            // all 16 output rows are useful instead of 8 of 32 columns.  Lane (l16, g4):
            // A row l16, B column = weight row 32*wave + 16*rg + l16, K chunk
            // 16*(g4 & 1) of block 2p + (g4 >> 1); outputs are tokens 4(g4 & 1)..+3 of
            // block parity g4 >> 1 (the parities meet at the store).
            const int t16 = lane & 15, g4 = lane >> 4;
            const int ta = t16 & 7, pa = t16 >> 3;
            const bool a_on = (g4 >> 1) == pa && ta < x_valid_tokens;
            i32x4 p_aop[2];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const i32x4 v = *reinterpret_cast<const i32x4 *>(xs + ta * kQ8BlockBytes + 16 + 32 * (2 * p + pa) +
                                                                 16 * (g4 & 1));
                p_aop[p] = a_on ? v : i32x4{0, 0, 0, 0};
            }
            float p_dx8[2][4], p_nb8[2][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = min(4 * (g4 & 1) + i, x_valid_tokens - 1);
                const u32x4 h = *reinterpret_cast<const u32x4 *>(xs + m * kQ8BlockBytes);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const uint32_t hb = (g4 >> 1) ? (p ? h.w : h.y) : (p ? h.z : h.x);
                    x_scales(hb, p_dx8[p][i], p_nb8[p][i]);
                }
            }
            // -s_x of the stage's 4 blocks on rows of parity 0 (K group 0 only; zero
            // elsewhere, and the d_w side is finite everywhere).
            f16x4 p_sx;
            {
                const u32x4 h = *reinterpret_cast<const u32x4 *>(xs + min(ta, x_valid_tokens - 1) * kQ8BlockBytes);
                const uint32_t keep = (g4 == 0 && pa == 0 && ta < x_valid_tokens) ? 0xffffffffu : 0u;
                const uint32_t lo = (((h.x >> 16) | (h.y & 0xffff0000u)) ^ 0x80008000u) & keep;
                const uint32_t hi = (((h.z >> 16) | (h.w & 0xffff0000u)) ^ 0x80008000u) & keep;
                const u32x2 pk = {lo, hi};
                p_sx = __builtin_bit_cast(f16x4, pk);
            }
            const i32x4 bias4 = {bias[0], bias[1], bias[2], bias[3]};
#pragma unroll
            for (int rg = 0; rg < 2; ++rg) {
                const int r = wave * 32 + rg * 16 + t16;  // weight row (MFMA column) of this lane
                f16x4 p_dw = *reinterpret_cast<const f16x4 *>(wd_row + r * KB);
                if (g4 != 0) p_dw = f16x4{0, 0, 0, 0};
                acc_p[rg] = __builtin_amdgcn_mfma_f32_16x16x16f16(p_sx, p_dw, acc_p[rg], 0, 0, 0);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const int bb = 2 * p + (g4 >> 1);
                    const i32x4 bop = *reinterpret_cast<const i32x4 *>(wq + r * kWqStride + bb * 32 + 16 * (g4 & 1));
                    const float dw = wd_epi[bb * BN + (r & ~31) + epi_perm(r & 31)];
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(p_aop[p], bop, bias4, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float tt = fmaf(__int_as_float(d[i]), p_dx8[p][i], p_nb8[p][i]);
                        acc_p[rg][i] = fmaf(dw, tt, acc_p[rg][i]);
                    }
                }
            }
            } else if constexpr (LIVE == 3) {
    #pragma unroll
            for (int b = 0; b < KB; ++b) {
                const i32x4 bop = *reinterpret_cast<const i32x4 *>(xs + l32 * kQ8BlockBytes + 16 + 32 * b + 16 * hh);
                const i32x4 aop =
                    *reinterpret_cast<const i32x4 *>(wq + (wave * 32 + l32) * kWqStride + b * 32 + 16 * hh);
                float dx8, nb8;
                x_scales(hdr[0][b], dx8, nb8);
                float wv[16];
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 w4 = *reinterpret_cast<const f32x4 *>(wd_epi + b * BN + wave * 32 + hh * 16 + 4 * j);
                    wv[4 * j] = w4.x; wv[4 * j + 1] = w4.y; wv[4 * j + 2] = w4.z; wv[4 * j + 3] = w4.w;
                }
                const i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, bias, 0, 0, 0);
                epilogue_f32(acc[0][0], d0, wv, dx8, nb8);
            }
            {
                const f16x4 aop = *reinterpret_cast<const f16x4 *>(wd_row + (wave * 32 + l32) * KB);
                const uint32_t *h = hdr[0];
                uint32_t lo = ((h[0] >> 16) | (h[1] & 0xffff0000u)) ^ 0x80008000u;
                uint32_t hi = ((h[2] >> 16) | (h[3] & 0xffff0000u)) ^ 0x80008000u;
                if (hh) { lo = 0u; hi = 0u; }
                const u32x2 pk = {lo, hi};
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x8f16(aop, __builtin_bit_cast(f16x4, pk), acc[0][0], 0, 0, 0);
            }
            } else if constexpr (LIVE > 0) {
    #pragma unroll
            for (int b = 0; b < KB; ++b) {
                i32x4 bop[2], aop[2];
    #pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    const int col = wm * 64 + ct * 32 + l32;
                    bop[ct] = *reinterpret_cast<const i32x4 *>(xs + col * kQ8BlockBytes + 16 + 32 * b + 16 * hh);
                }
    #pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const int row = wn * 64 + rt * 32 + l32;
                    aop[rt] = *reinterpret_cast<const i32x4 *>(wq + row * kWqStride + b * 32 + 16 * hh);
                }
                float dx8[2], nb8[2];
    #pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    x_scales(hdr[ct][b], dx8[ct], nb8[ct]);
                }
                // fp32 scales: the epilogue is two plain v_fma_f32 per element
                // (v_fma_mix_f32 on fp16 scales issues at about half their rate).
                float wv[2][16];
    #pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const int rbase = (wn * 2 + rt) * 32 + hh * 16;
    #pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x4 w4 = *reinterpret_cast<const f32x4 *>(wd_epi + b * BN + rbase + 4 * j);
                        wv[rt][4 * j] = w4.x; wv[rt][4 * j + 1] = w4.y; wv[rt][4 * j + 2] = w4.z; wv[rt][4 * j + 3] = w4.w;
                    }
                }
                // Two result tiles in flight: the MFMA of the next tile overlaps the
                // VALU epilogue of the previous one.
                if constexpr (LIVE == 2) {
                    i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[0], bop[0], bias, 0, 0, 0);
                    i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[0], bop[1], bias, 0, 0, 0);
                    epilogue_f32(acc[0][0], d0, wv[0], dx8[0], nb8[0]);
                    d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[1], bop[0], bias, 0, 0, 0);
                    epilogue_f32(acc[0][1], d1, wv[0], dx8[1], nb8[1]);
                    d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[1], bop[1], bias, 0, 0, 0);
                    epilogue_f32(acc[1][0], d0, wv[1], dx8[0], nb8[0]);
                    epilogue_f32(acc[1][1], d1, wv[1], dx8[1], nb8[1]);
                } else {
                    const i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[0], bop[0], bias, 0, 0, 0);
                    const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[1], bop[0], bias, 0, 0, 0);
                    epilogue_f32(acc[0][0], d0, wv[0], dx8[0], nb8[0]);
                    epilogue_f32(acc[1][0], d1, wv[1], dx8[0], nb8[0]);
                }
            }

            // sum_b d_w * (-s_x) over this stage's 4 blocks on the f16 MFMA (K = 8:
            // the lanes of the upper K half contribute zeros).
            {
                f16x4 aop[2], bop[2];
    #pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const int row = wn * 64 + rt * 32 + l32;
                    aop[rt] = *reinterpret_cast<const f16x4 *>(wd_row + row * KB);
                }
    #pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    const uint32_t *h = hdr[ct];
                    uint32_t lo = ((h[0] >> 16) | (h[1] & 0xffff0000u)) ^ 0x80008000u;
                    uint32_t hi = ((h[2] >> 16) | (h[3] & 0xffff0000u)) ^ 0x80008000u;
                    // Zero B (not A) in the upper K half: an infinite s_x must not meet 0.
                    if (hh) { lo = 0u; hi = 0u; }
                    const u32x2 pk = {lo, hi};
                    bop[ct] = __builtin_bit_cast(f16x4, pk);
                }
    #pragma unroll
                for (int rt = 0; rt < 2; ++rt)
    #pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        acc[rt][ct] = __builtin_amdgcn_mfma_f32_32x32x8f16(aop[rt], bop[ct], acc[rt][ct], 0, 0, 0);
            }
            }  // LIVE > 0

            // Unconditional, also after the last stage (stage indices clamped to the
            // last one: the extra unpack and loads fill buffers no wave reads any
            // more): the same number of loads on every path keeps the compiler's
            // register waits exact instead of vmcnt(0).
            JJO_GEMM_VMCNT(3);  // all but W(c+2): X(c+1) and W(c+1) have landed
            store_w((c + 1) & 1, w_next);
            __syncthreads();
            zero_tail_headers((c + 1) & 1);
            load_x(min(c + 2, n_stages - 1));          // buffer c&1, freed by the barrier
            load_w(min(c + 3, n_stages - 1), w_next);  // set (c+1)&1, just unpacked
        };
        int c = 0;
        for (; c + 1 < n_stages; c += 2) {
            stage(c, std::integral_constant<int, 0>{});
            stage(c + 1, std::integral_constant<int, 1>{});
        }
        if (c < n_stages) stage(c, std::integral_constant<int, 0>{});
        JJO_GEMM_VMCNT(0);  // the clamped loads of the last stage
    };
    if (kGrouped && n_live == 4)
        stage_loop(std::integral_constant<int, 4>{});
    else if (kGrouped && n_live == 3)
        stage_loop(std::integral_constant<int, 3>{});
    else if (n_live == 2)
        stage_loop(std::integral_constant<int, 2>{});
    else if (n_live == 1)
        stage_loop(std::integral_constant<int, 1>{});
    else
        stage_loop(std::integral_constant<int, 0>{});

    if constexpr (kSwiglu) {
        // ---- fused SwiGLU + Q8_1: 8*acc of the 128 x 128 tile -> LDS res[token][row]
        // (rows 0..63 gate, 64..127 up), then silu(gate) * up quantized per 32-group
        // of intermediate values with the quantizer's exact arithmetic.
        __syncthreads();  // every wave is done with the staging buffers
        float *res = reinterpret_cast<float *>(smem);
        constexpr int kResStride = BN + 4;  // floats per token (padding against bank conflicts)
        if (pnarrow) {
            const int t16 = lane & 15, g4 = lane >> 4;
#pragma unroll
            for (int rg = 0; rg < 2; ++rg) {
                float sum[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) sum[i] = acc_p[rg][i] + __shfl_xor(acc_p[rg][i], 32);
                if (g4 < 2) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        res[(4 * g4 + i) * kResStride + wave * 32 + rg * 16 + t16] = 8.0f * sum[i];
                }
            }
        } else if (narrow) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = {8.0f * acc[0][0][4 * q], 8.0f * acc[0][0][4 * q + 1], 8.0f * acc[0][0][4 * q + 2],
                                 8.0f * acc[0][0][4 * q + 3]};
                *reinterpret_cast<f32x4 *>(res + l32 * kResStride + wave * 32 + 8 * q + 4 * hh) = v;
            }
        } else {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 v = {8.0f * acc[rt][ct][4 * q], 8.0f * acc[rt][ct][4 * q + 1],
                                         8.0f * acc[rt][ct][4 * q + 2], 8.0f * acc[rt][ct][4 * q + 3]};
                        *reinterpret_cast<f32x4 *>(res + (wm * 64 + ct * 32 + l32) * kResStride + wn * 64 + rt * 32 +
                                                   8 * q + 4 * hh) = v;
                    }
        }
        __syncthreads();
        // 8 lanes per (token, 32-group); 16 lanes per token (two groups of 64 values).
        const int ni0 = blockIdx.x * 64;
        const int n_valid = min(BM, m_end - m0);
#pragma unroll 1
        for (int it = 0; it < BM * 16 / kThreads; ++it) {
            const int idx = it * kThreads + tid;
            const int tok = idx >> 4, grp = (idx >> 3) & 1, j = idx & 7;
            const float *rg = res + tok * kResStride + 32 * grp + 4 * j;
            const f32x4 g = *reinterpret_cast<const f32x4 *>(rg);
            const f32x4 u = *reinterpret_cast<const f32x4 *>(rg + 64);
            const float v0 = swiglu(g.x, u.x), v1 = swiglu(g.y, u.y), v2 = swiglu(g.z, u.z), v3 = swiglu(g.w, u.w);
            uint32_t ds;
            const uint32_t qv = quantize_group8(v0, v1, v2, v3, &ds);  // all lanes: the butterfly
            if (tok < n_valid) {
                const int n = ni0 + 32 * grp + 4 * j;  // intermediate index of the lane's first value
                uint8_t *blk = midq + ((size_t)(n / kQSuper) * M + (m0 + tok)) * kQ8BlockBytes;
                const int iqs = n % kQSuper;
                *reinterpret_cast<uint32_t *>(blk + 16 + iqs) = qv;
                if (j == 0) *reinterpret_cast<uint32_t *>(blk + 4 * (iqs / 32)) = ds;
            }
        }
        return;
    }

    // ---- store: y[m][n] = 8 * acc ----
    if (kGrouped && pnarrow) {  // block parities meet across lanes l and l ^ 32
        const int t16 = lane & 15, g4 = lane >> 4;
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
            f32x4 sum;
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] = acc_p[rg][i] + __shfl_xor(acc_p[rg][i], 32);
            const int n = n0 + wave * 32 + rg * 16 + t16;
            if (g4 < 2 && n < N) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = m0 + 4 * g4 + i;
                    if (m < m_end) {
                        int out_row = m;
                        if constexpr (kGrouped) {
                            if (route_dst != nullptr) out_row = route_dst[m];
                        }
                        y[(size_t)out_row * N + n] = 8.0f * sum[i];
                    }
                }
            }
        }
        return;
    }
    if (kGrouped && narrow) {
        const int m = m0 + l32;
        if (m < m_end) {
            int out_row = m;
            if constexpr (kGrouped) {
                if (route_dst != nullptr) out_row = route_dst[m];
            }
            float *yrow = y + (size_t)out_row * N;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wave * 32 + 8 * q + 4 * hh;
                const float v0 = 8.0f * acc[0][0][4 * q + 0];
                const float v1 = 8.0f * acc[0][0][4 * q + 1];
                const float v2 = 8.0f * acc[0][0][4 * q + 2];
                const float v3 = 8.0f * acc[0][0][4 * q + 3];
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
        return;
    }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int m = m0 + wm * 64 + ct * 32 + l32;
        if (m >= m_end) continue;
        int out_row = m;
        if constexpr (kGrouped) {
            if (route_dst != nullptr) out_row = route_dst[m];
        }
        float *yrow = y + (size_t)out_row * N;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * 64 + rt * 32 + 8 * q + 4 * hh;
                const float v0 = 8.0f * acc[rt][ct][4 * q + 0];
                const float v1 = 8.0f * acc[rt][ct][4 * q + 1];
                const float v2 = 8.0f * acc[rt][ct][4 * q + 2];
                const float v3 = 8.0f * acc[rt][ct][4 * q + 3];
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
}

template <bool kGrouped, bool kSwiglu = false, bool kSplit = false>
hipError_t set_smem_attr() {
    return ensure_dynamic_lds((const void *)gemm_q4_0_q8_1_mfma_kernel<kGrouped, kSwiglu, kSplit>, kSmemBytes);
}
static_assert(BM * (BN + 4) * 4 <= kSmemBytes, "fused SwiGLU result tile fits the staging LDS");

}  // namespace

hipError_t launch_gemm_mfma(const void *w, const void *xq, float *y, int K, int N, int M,
                            hipStream_t stream) {
    hipError_t e = set_smem_attr<false>();
    if (e != hipSuccess) return e;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(gemm_q4_0_q8_1_mfma_kernel<false>, grid, dim3(kThreads), kSmemBytes, stream,
                       (const uint8_t *)w, (const uint8_t *)xq, y, K, N, M, nullptr, 0, nullptr,
                       (const uint8_t *)nullptr, 0);
    return hipGetLastError();
}

hipError_t launch_gemm_mfma_grouped(const void *w, const void *xq, const int32_t *expert_offsets,
                                    int n_experts, const int32_t *route_dst, float *y, int K,
                                    int N, int n_routes, hipStream_t stream, const void *w2, int n_split,
                                    bool split) {
    hipError_t e = split ? set_smem_attr<true, false, true>() : set_smem_attr<true>();
    if (e != hipSuccess) return e;
    // Upper bound on the number of token tiles over all experts.
    const int max_tiles = (n_routes + BM - 1) / BM + n_experts;
    const dim3 grid((N + BN - 1) / BN, max_tiles);
    if (split)
        hipLaunchKernelGGL((gemm_q4_0_q8_1_mfma_kernel<true, false, true>), grid, dim3(kThreads), kSmemBytes,
                           stream, (const uint8_t *)w, (const uint8_t *)xq, y, K, N, n_routes, expert_offsets,
                           n_experts, route_dst, (const uint8_t *)w2, n_split, (uint8_t *)nullptr);
    else
        hipLaunchKernelGGL(gemm_q4_0_q8_1_mfma_kernel<true>, grid, dim3(kThreads), kSmemBytes, stream,
                           (const uint8_t *)w, (const uint8_t *)xq, y, K, N, n_routes, expert_offsets,
                           n_experts, route_dst, (const uint8_t *)w2, n_split);
    return hipGetLastError();
}

hipError_t launch_gemm_gate_up_swiglu_q8_1(const void *w_gate, const void *w_up, const void *xq,
                                           const int32_t *expert_offsets, int n_experts, void *mid_q8_1, int K,
                                           int I, int n_routes, hipStream_t stream, bool split) {
    hipError_t e = split ? set_smem_attr<true, true, true>() : set_smem_attr<true, true>();
    if (e != hipSuccess) return e;
    const int max_tiles = (n_routes + BM - 1) / BM + n_experts;
    const dim3 grid(I / 64, max_tiles);
    if (split)
        hipLaunchKernelGGL((gemm_q4_0_q8_1_mfma_kernel<true, true, true>), grid, dim3(kThreads), kSmemBytes, stream,
                           (const uint8_t *)w_gate, (const uint8_t *)xq, (float *)nullptr, K, 2 * I, n_routes,
                           expert_offsets, n_experts, (const int32_t *)nullptr, (const uint8_t *)w_up, I,
                           (uint8_t *)mid_q8_1);
    else
        hipLaunchKernelGGL((gemm_q4_0_q8_1_mfma_kernel<true, true>), grid, dim3(kThreads), kSmemBytes, stream,
                           (const uint8_t *)w_gate, (const uint8_t *)xq, (float *)nullptr, K, 2 * I, n_routes,
                           expert_offsets, n_experts, (const int32_t *)nullptr, (const uint8_t *)w_up, I,
                           (uint8_t *)mid_q8_1);
    return hipGetLastError();
}

}  // namespace jjo
