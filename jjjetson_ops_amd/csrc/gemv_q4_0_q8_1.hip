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
//     fetched with dwordx4 + dwordx4 + dword.  A wave owns U rows of one slice and
//     issues all its weight loads before anything else.
//   * Integer dot without unpacking nibbles: with u = q + 128 = 16*hi + lo
//     (hi, lo in 0..15) the activation is split once into two 4-bit planes laid
//     out in the weight's own nibble order (element j in the low nibble of byte
//     j, element j+16 in the high nibble), so a raw Q4_0 nibble dword feeds
//     v_dot8_u32_u4 directly:
//        sumi = 16*dot8(w, HI) + dot8(w, LO) - 128*dot8(w, 0x11111111)
//     (the last term depends on the weights only and is shared by all tokens).
//   * While the weight loads are in flight, the workgroup builds those planes
//     plus (d_x, -8*s_x) for every block of its K range in LDS: from the Q8_1
//     blocks, or -- fused variant, M = 1 -- straight from the fp32 activation
//     with the reference quantizer's arithmetic (exact sum tree, IEEE divides,
//     roundf), optionally writing the Q8_1 bytes too.  One 80-byte LDS record
//     per (token, block pair): conflict-free ds_read_b128 for consecutive lanes.
//   * Lane partials: one transposed butterfly for all of a wave's row x token
//     sums (ds_bpermute rounds, then DPP within the lanes that share a sum); the JS
//     K-slices of a row group (JS waves of one workgroup) are added in LDS in
//     slice order.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "q4q8_common.hpp"

namespace jjo {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a8 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRec = 80;  // LDS bytes per (token, block pair): HI a|LO a|HI b|LO b|dx a,c a,dx b,c b

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

// Planes of one block from its 8 activation dwords (int8 q, element 4i+k in byte k
// of dword i).  u = q ^ 0x80 per byte = q + 128.  Output dword i pairs element
// 4i+k (low nibble of byte k) with element 16+4i+k (high nibble).
__device__ __forceinline__ void make_planes(const uint32_t q[8], uint32_t hi[4], uint32_t lo[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = q[i] ^ 0x80808080u;
        const uint32_t b = q[i + 4] ^ 0x80808080u;
        lo[i] = (a & 0x0f0f0f0fu) | ((b & 0x0f0f0f0fu) << 4);
        hi[i] = ((a >> 4) & 0x0f0f0f0fu) | (b & 0xf0f0f0f0u);
    }
}

// Integer sum of one Q4_0 block: w = its 4 raw nibble dwords, n128 = 128 * sum(nib).
__device__ __forceinline__ int32_t block_sumi(const uint32_t w[4], const uint32_t hi[4], const uint32_t lo[4],
                                              int32_t n128) {
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_udot8(w[i], hi[i], s, false);
    s <<= 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_udot8(w[i], lo[i], s, false);
    return (int32_t)s - n128;
}

__device__ __forceinline__ int32_t nib_sum128(const uint32_t w[4]) {
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) n = __builtin_amdgcn_udot8(w[i], 0x11111111u, n, false);
    return (int32_t)(n << 7);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// NV independent 64-lane sums at once (NV a power of two, <= 32).  Transposed
// butterfly: in round r (distance 32 >> r) each lane keeps one of every pair of its
// values, adds its partner's copy of it and sends the other, so the values per lane
// halve while the lanes per partial double.  After log2(NV) rounds every lane holds
// one partial, for value sum_r bit(5 - r of lane) << r; a plain reduction over the
// remaining 64 / NV lanes that share it finishes the sum.  Returns the lane's sum.
template <int NV>
__device__ __forceinline__ float multi_sum(float (&v)[NV], int lane) {
    static_assert(NV == 1 || NV == 2 || NV == 4 || NV == 8 || NV == 16 || NV == 32, "NV");
    constexpr int R = NV == 1 ? 0 : NV == 2 ? 1 : NV == 4 ? 2 : NV == 8 ? 3 : NV == 16 ? 4 : 5;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int dist = 32 >> r;
        const bool bit = lane & dist;
#pragma unroll
        for (int j = 0; j < (NV >> r) / 2; ++j) {
            const float keep = bit ? v[2 * j + 1] : v[2 * j];
            const float send = bit ? v[2 * j] : v[2 * j + 1];
            v[j] = keep + __shfl_xor(send, dist);
        }
    }
    constexpr int G = 64 >> R;  // lanes that share a value
    float t = v[0];
    if constexpr (G >= 2) t += dpp<0xB1>(t);   // quad_perm [1,0,3,2]
    if constexpr (G >= 4) t += dpp<0x4E>(t);   // quad_perm [2,3,0,1]
    if constexpr (G == 8) t += dpp<0x141>(t);  // row_half_mirror: the other quad of 8
    if constexpr (G >= 16) {
        t += dpp<0x124>(t);  // row_ror:4
        t += dpp<0x128>(t);  // row_ror:8
    }
    if constexpr (G >= 32) t += __shfl_xor(t, 16);
    if constexpr (G == 64) t += __shfl_xor(t, 32);
    return t;
}

// Value index whose sum multi_sum<NV> leaves in `lane`.
template <int NV>
__device__ __forceinline__ int multi_sum_index(int lane) {
    constexpr int R = NV == 1 ? 0 : NV == 2 ? 1 : NV == 4 ? 2 : NV == 8 ? 3 : NV == 16 ? 4 : 5;
    int idx = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) idx |= ((lane >> (5 - r)) & 1) << r;
    return idx;
}

constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }

// Write one block's planes and constants into its half of the pair record.
__device__ __forceinline__ void put_block(uint8_t *rec, int half, const uint32_t hi[4], const uint32_t lo[4],
                                          float dx, float c) {
    *reinterpret_cast<u32x4a16 *>(rec + 32 * half) = u32x4a16{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<u32x4a16 *>(rec + 32 * half + 16) = u32x4a16{lo[0], lo[1], lo[2], lo[3]};
    reinterpret_cast<float *>(rec + 64)[2 * half] = dx;
    reinterpret_cast<float *>(rec + 64)[2 * half + 1] = c;
}

// ---- activation staging from Q8_1 blocks (quantizer layout) ----
// Item = (token m, block b).  Loads are issued first (issue_q8), the planes are
// built once the data is there (finish_q8), so the weight requests can leave in
// between.
struct ItemQ8 {
    uint32_t ds;
    uint32_t q[8];
};

template <int M>
__device__ __forceinline__ void issue_q8(ItemQ8 &it, const uint8_t *__restrict__ xq, int item, int nb) {
    item = min(item, M * nb - 1);  // idle lanes re-read a valid item (no branch around the load)
    const int m = item / nb, b = item - m * nb;
    const uint8_t *blk = xq + ((size_t)(b >> 2) * M + m) * kQ8BlockBytes;
    const int g = b & 3;
    it.ds = *reinterpret_cast<const uint32_t *>(blk + 4 * g);
    const u32x4a16 v0 = *reinterpret_cast<const u32x4a16 *>(blk + 16 + 32 * g);
    const u32x4a16 v1 = *reinterpret_cast<const u32x4a16 *>(blk + 32 + 32 * g);
    it.q[0] = v0.x; it.q[1] = v0.y; it.q[2] = v0.z; it.q[3] = v0.w;
    it.q[4] = v1.x; it.q[5] = v1.y; it.q[6] = v1.z; it.q[7] = v1.w;
}

// Unconditional (no branch for the loads to sink into): items past the end write
// the spare record `spare` after the M * nb/2 real ones.
__device__ __forceinline__ void finish_q8(uint8_t *xs, const ItemQ8 &it, int item, int nb, int n_items) {
    const int m = item / nb, b = item - m * nb;
    uint32_t hi[4], lo[4];
    make_planes(it.q, hi, lo);
    const size_t rec = item < n_items ? (size_t)m * (nb >> 1) + (b >> 1) : (size_t)(n_items >> 1);
    put_block(xs + rec * kRec, b & 1, hi, lo, half_lo(it.ds), -8.0f * half_hi(it.ds));
}

// ---- fused staging (M = 1): quantize fp32 x exactly as quantize_q8_1_kernel
// (src/cuda/q8_1.cu:40-103).  Item = half of a 32-group; the two halves of a group
// are adjacent lanes: h = 0 holds elements 0..7 and 16..23 (the reference's
// virtual lanes t0, t1, t4, t5), h = 1 holds 8..15 and 24..31 (t2, t3, t6, t7).
// The xor-4 partners are inside a lane, the xor-2 partners are exchanged with one
// DPP quad_perm, and the group sum is ((t0+t4)+(t2+t6)) + ((t1+t5)+(t3+t7))
// exactly as the reference's butterfly.
struct ItemF32 {
    f32x4 v[4];  // v[0], v[1]: elements 8h..8h+7; v[2], v[3]: 16+8h..16+8h+7
};

__device__ __forceinline__ void issue_f32(ItemF32 &it, const float *__restrict__ x, int item, int nb) {
    const int b = min(item >> 1, nb - 1), h = item & 1;
    const float *gx = x + (size_t)b * 32;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        it.v[i] = *reinterpret_cast<const f32x4 *>(gx + 8 * h + 4 * i);
        it.v[2 + i] = *reinterpret_cast<const f32x4 *>(gx + 16 + 8 * h + 4 * i);
    }
}

// roundf (ties away from zero) for |v| < 2^23 in three ops: adding 0.5 - 2^-25
// with v's sign and truncating gives the same integer as roundf for every such
// float (checked exhaustively over all 2^30 non-negative floats below 2^23 in
// the test suite; the sign makes it symmetric).  `v` must be the rounded fp32
// product: contraction of the caller's multiply into this add (an fma) would skip
// that rounding and move products just below a .5 tie that round up onto it.
__device__ __forceinline__ int32_t round_away(float v) {
#pragma clang fp contract(off)
    return __float2int_rz(v + copysignf(0.49999997f, v));
}

// All lanes of the wave must call this together (DPP partner exchange); `live`
// masks the stores of items past the end.
__device__ __forceinline__ void finish_f32(uint8_t *xs, uint8_t *__restrict__ xq_out, const ItemF32 &it, int item,
                                           int nb, bool live) {
    const int b = min(item >> 1, nb - 1), h = item & 1;
    const f32x4 *v = it.v;
    float am[4], su[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        am[i] = fmaxf(fabsf(v[i].x), fmaxf(fabsf(v[i].y), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        float s = v[i].x + v[i].y;
        s = s + v[i].z;
        su[i] = s + v[i].w;
    }
    // xor-4 step (inside the lane): (t0+t4), (t1+t5) for h = 0; (t2+t6), (t3+t7) for h = 1
    const float s0 = su[0] + su[2], s1 = su[1] + su[3];
    const float m0 = fmaxf(am[0], am[2]), m1 = fmaxf(am[1], am[3]);
    // xor-2 step: partner lane
    const float s0o = dpp<0xB1>(s0), s1o = dpp<0xB1>(s1);
    const float m0o = dpp<0xB1>(m0), m1o = dpp<0xB1>(m1);
    // xor-1 step; additions are commutative, so both lanes get identical bits
    const float sum = (s0 + s0o) + (s1 + s1o);
    const float amax = fmaxf(fmaxf(m0, m0o), fmaxf(m1, m1o));
    const float d_inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
    uint32_t q[4];  // bytes of elements 8h..8h+7 (q[0], q[1]) and 16+8h.. (q[2], q[3])
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)
        const int32_t a = round_away(v[i].x * d_inv), bb = round_away(v[i].y * d_inv);
        const int32_t c = round_away(v[i].z * d_inv), d = round_away(v[i].w * d_inv);
        q[i] = (uint32_t)(a & 0xff) | ((uint32_t)(bb & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
               ((uint32_t)(d & 0xff) << 24);
    }
    if (!live) return;
    // planes for weight dwords i = 2h, 2h+1 of block b
    uint8_t *rec = xs + (size_t)(b >> 1) * kRec + 32 * (b & 1);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t a = q[i] ^ 0x80808080u;
        const uint32_t bq = q[2 + i] ^ 0x80808080u;
        reinterpret_cast<uint32_t *>(rec + 16)[2 * h + i] = (a & 0x0f0f0f0fu) | ((bq & 0x0f0f0f0fu) << 4);
        reinterpret_cast<uint32_t *>(rec)[2 * h + i] = ((a >> 4) & 0x0f0f0f0fu) | (bq & 0xf0f0f0f0u);
    }
    const __half hd = __float2half_rn(1.0f / d_inv);
    const __half hs = __float2half_rn(sum);
    if (h == 0) {
        float *cst = reinterpret_cast<float *>(xs + (size_t)(b >> 1) * kRec + 64) + 2 * (b & 1);
        cst[0] = __half2float(hd);
        cst[1] = -8.0f * __half2float(hs);
    }
    if (xq_out != nullptr) {
        uint8_t *blk = xq_out + (size_t)(b >> 2) * kQ8BlockBytes;
        const int g = b & 3;
        *reinterpret_cast<u32x2a8 *>(blk + 16 + 32 * g + 8 * h) = u32x2a8{q[0], q[1]};
        *reinterpret_cast<u32x2a8 *>(blk + 16 + 32 * g + 16 + 8 * h) = u32x2a8{q[2], q[3]};
        if (h == 0)
            *reinterpret_cast<uint32_t *>(blk + 4 * g) =
                (uint32_t)__half_as_ushort(hd) | ((uint32_t)__half_as_ushort(hs) << 16);
    }
}

// ---- routed (MoE decode) launches ----
// The weights are E stacked [N][K] expert matrices and the activation is the
// expert-sorted Q8_1 route rows (superblock-major over n_routes rows); routes
// offsets[e]..offsets[e+1]-1 use expert e.  blockIdx.y = which * slots + slot
// selects the slot-th expert that has routes (which = 1: the second stacked
// matrix w2, written N columns further along each output row).  The workgroup
// keeps its weight rows in registers and takes the expert's routes M at a time
// (each chunk re-stages only activation rows), so every weight byte of an active
// expert is read once whatever its route count.  Output row p (a sorted route
// position) starts at y + p * ldy, or at y + route_dst[p] * ldy.
struct RouteArgs {
    const int32_t *offsets;    // [n_experts + 1]
    const uint8_t *w2;         // second stacked matrix, or null
    const int32_t *route_dst;  // output row of sorted route p (null: p)
    int n_experts, n_routes, slots, ldy;
};

__device__ __forceinline__ size_t routed_row(const RouteArgs &ra, int p) {
    return ra.route_dst != nullptr ? (size_t)ra.route_dst[p] : (size_t)p;
}

struct RouteTile {
    int expert, which, m0, mc, end;  // first chunk: routes m0 .. m0 + mc - 1; the expert's end
};

// Clamped route range of expert e (a malformed table gives fewer routes, never
// an access outside the activation or output rows).
__device__ __forceinline__ void expert_range(const RouteArgs &ra, int e, int &beg, int &end) {
    beg = min(max(ra.offsets[e], 0), ra.n_routes);
    end = min(max(ra.offsets[e + 1], beg), ra.n_routes);
}

// false: this workgroup has no routes (the same for all its waves).
__device__ __forceinline__ bool route_tile(const RouteArgs &ra, int mt, RouteTile &t) {
    const int which = (int)blockIdx.y >= ra.slots;
    int slot = (int)blockIdx.y - which * ra.slots;
    const int lane = threadIdx.x & 63;
    int e = -1;
    for (int e0 = 0; e0 < ra.n_experts; e0 += 64) {
        bool nonempty = false;
        if (e0 + lane < ra.n_experts) {
            int b, en;
            expert_range(ra, e0 + lane, b, en);
            nonempty = en > b;
        }
        uint64_t bal = __ballot(nonempty);
        const int c = __popcll(bal);
        if (slot < c) {
            for (int i = 0; i < slot; ++i) bal &= bal - 1;
            e = e0 + __builtin_ctzll(bal);
            break;
        }
        slot -= c;
    }
    if (e < 0) return false;
    int beg, end;
    expert_range(ra, e, beg, end);
    if (beg >= end) return false;
    t.expert = e;
    t.which = which;
    t.m0 = beg;
    t.mc = min(mt, end - beg);
    t.end = end;
    return true;
}

// issue_q8 for routed launches: token m of the chunk reads route row
// m0 + min(m, mc - 1) of the n_routes-row activation (tokens past the chunk's
// routes re-read its last one; their sums are never stored).
template <int M>
__device__ __forceinline__ void issue_q8_routed(ItemQ8 &it, const uint8_t *__restrict__ xq, int item, int nb,
                                                int n_routes, int m0, int mc) {
    item = min(item, M * nb - 1);
    const int m = item / nb, b = item - m * nb;
    const int row = m0 + min(m, mc - 1);
    const uint8_t *blk = xq + ((size_t)(b >> 2) * n_routes + row) * kQ8BlockBytes;
    const int g = b & 3;
    it.ds = *reinterpret_cast<const uint32_t *>(blk + 4 * g);
    const u32x4a16 v0 = *reinterpret_cast<const u32x4a16 *>(blk + 16 + 32 * g);
    const u32x4a16 v1 = *reinterpret_cast<const u32x4a16 *>(blk + 32 + 32 * g);
    it.q[0] = v0.x; it.q[1] = v0.y; it.q[2] = v0.z; it.q[3] = v0.w;
    it.q[4] = v1.x; it.q[5] = v1.y; it.q[6] = v1.z; it.q[7] = v1.w;
}

__device__ __forceinline__ int opaque_int(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Workgroup = RG row groups x JS K-slices (one wave each).  JS = ceil(K / 4096).
// FUSED: `xin` is the fp32 activation [K] (M = 1) instead of Q8_1 blocks and
// `xq_out` (optional) receives its Q8_1 bytes (written by workgroup 0).
// ROUTED: a routed launch (RouteArgs), M routes per workgroup, Q8_1 input.
// R2 (K <= 2048, one K slice): rows hold at most 32 block pairs, so lanes 32..63 take
// the rows U further on: a wave covers 2U rows (each lane's sums for the other half's
// rows are zero in the wave reduction).
template <int M, int U, int JS, int RG, bool FUSED, int EARLY, bool ROUTED = false, bool R2 = false>
__global__ __launch_bounds__(64 * JS * RG) void gemv_q4_0_q8_1_kernel(const uint8_t *__restrict__ w,
                                                                      const void *__restrict__ xin,
                                                                      uint8_t *__restrict__ xq_out,
                                                                      float *__restrict__ y, int K, int N,
                                                                      RouteArgs ra) {
    static_assert(!(ROUTED && FUSED), "routed launches take Q8_1 route rows");
    static_assert(!R2 || JS == 1, "paired rows: one K slice");
    constexpr int kRowsW = R2 ? 2 * U : U;  // rows per wave
    extern __shared__ __align__(16) uint8_t xs[];  // M * K/64 records of kRec bytes + 1 spare
    __shared__ float part[JS > 1 ? RG * JS * U * M : 1];

    constexpr int kThreadsWG = 64 * JS * RG;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int js = wave % JS;              // K-slice of this wave
    const int rg = wave / JS;              // row group inside the workgroup
    const int nb = K / kQK;
    const int P = nb >> 1;                 // block pairs per row
    const int p = R2 ? (lane & 31) : lane + 64 * js;  // this lane's pair
    const int hrow = R2 ? (lane >> 5) * U : 0;         // R2: lanes 32..63 on rows U further
    const bool live = p < P;
    const size_t row_bytes = (size_t)nb * kQ4BlockBytes;
    const int r0 = (blockIdx.x * RG + rg) * kRowsW;
    const int n_items = FUSED ? 2 * nb : M * nb;
    const int rounds = (n_items + kThreadsWG - 1) / kThreadsWG;
    RouteTile rt{0, 0, 0, M, M};
    if constexpr (ROUTED) {
        if (!route_tile(ra, M, rt)) return;
        w = (rt.which ? ra.w2 : w) + (size_t)rt.expert * N * row_bytes;
        y += (size_t)rt.which * N;
    }
    const int ldy = ROUTED ? ra.ldy : N;
    int m0c = rt.m0, mcc = rt.mc;  // the current chunk of routes (routed launches)
    bool again = false;            // a later chunk: all its items are loaded in the pass

    // All global loads below are unconditional (clamped addresses), so the
    // compiler can count them and wait for exactly the ones each step needs.
    // 1) activation requests (L2-resident): EARLY items per thread, ahead of the weights
    using Item = typename std::conditional<FUSED, ItemF32, ItemQ8>::type;
    Item early[EARLY];
#pragma unroll
    for (int r = 0; r < EARLY; ++r) {
        const int item = threadIdx.x + r * kThreadsWG;
        if constexpr (FUSED) {
            issue_f32(early[r], reinterpret_cast<const float *>(xin), item, nb);
        } else {
            if constexpr (ROUTED)
                issue_q8_routed<M>(early[r], reinterpret_cast<const uint8_t *>(xin), item, nb, ra.n_routes, m0c, mcc);
            else
                issue_q8<M>(early[r], reinterpret_cast<const uint8_t *>(xin), item, nb);
        }
    }
    // Keep the instruction scheduler from hoisting the weight loads above them.
    __builtin_amdgcn_sched_barrier(0);
    // 2) weight requests for all U rows, in row order
    PairW wb[U];
    {
        const int pl = min(p, P - 1);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int rr = min(r0 + hrow + u, N - 1);
            load_pair(wb[u], w + (size_t)rr * row_bytes + (size_t)pl * 36);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3) the early items (routed launches: before the chunk loop, so that they are not
    //    held across it; later chunks load every item in their pass)
    uint8_t *xq_w = (FUSED && blockIdx.x == 0) ? xq_out : nullptr;
#pragma unroll
    for (int r = 0; r < EARLY; ++r) {
        const int item = threadIdx.x + r * kThreadsWG;
        if constexpr (FUSED) {
            finish_f32(xs, xq_w, early[r], item, nb, item < n_items);
        } else {
            finish_q8(xs, early[r], item, nb, n_items);
        }
    }
    const int lane_o = lane, js_o = js, rg_o = rg, p_o = p, r0_o = r0;  // (see the pass)
    for (;;) {  // one pass; routed launches: one per chunk of routes
        // Routed launches recompute the lane values of each pass from an opaque
        // thread index instead of holding them (and what derives from them) across
        // passes, which would cost the 1- and 2-route kernels half their occupancy.
        const int tid = ROUTED ? opaque_int(threadIdx.x) : (int)threadIdx.x;
        const int lane = ROUTED ? (tid & 63) : lane_o;
        const int js = ROUTED ? (tid >> 6) % JS : js_o;
        const int rg = ROUTED ? (tid >> 6) / JS : rg_o;
        const int p = ROUTED ? (R2 ? (lane & 31) : lane + 64 * js) : p_o;
        const bool live = p < P;
        const int r0 = ROUTED ? (int)(blockIdx.x * RG + rg) * kRowsW : r0_o;
        // 3) activation planes of the whole K range in LDS, once per workgroup (routed:
        //    per chunk of routes)
        for (int r = (ROUTED && again) ? 0 : EARLY; r < rounds; ++r) {  // the rest, load-then-use
            const int item = tid + r * kThreadsWG;
            Item it;
            if constexpr (FUSED) {
                issue_f32(it, reinterpret_cast<const float *>(xin), item, nb);
                finish_f32(xs, xq_w, it, item, nb, item < n_items);
            } else {
                if constexpr (ROUTED)
                    issue_q8_routed<M>(it, reinterpret_cast<const uint8_t *>(xin), item, nb, ra.n_routes, m0c, mcc);
                else
                    issue_q8<M>(it, reinterpret_cast<const uint8_t *>(xin), item, nb);
                finish_q8(xs, it, item, nb, n_items);
            }
        }
        __syncthreads();

        // 4) rows in load order: the wait for row u covers only rows 0..u
        float acc[U][M];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[u][m] = 0.0f;

        if (ROUTED && live) {
            // Token-outer: tokens past this expert's routes (mc <= M, uniform over the
            // workgroup) cost no dot products; each (row, token) sum is the same
            // expression as below.
            // Per row: the nibble sums and scales; the nibble dwords themselves are
            // taken from wb per token (block b's are 2-byte shifted: one alignbyte
            // each), which keeps the pass under the 1024-thread register budget.
            int32_t na[U], nbs[U];
            float dwa[U], dwb[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // Opaque per pass: the weight terms below stay after the activation
                // staging instead of being hoisted ahead of it (which would wait on
                // every weight load before the first LDS write).
#pragma unroll
                for (int i = 0; i < 9; ++i) asm volatile("" : "+v"(wb[u].d[i]));
                uint32_t qa[4], qb[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    qa[i] = __builtin_amdgcn_alignbyte(wb[u].d[i + 1], wb[u].d[i], 2);
                    qb[i] = wb[u].d[i + 5];
                }
                na[u] = nib_sum128(qa);
                nbs[u] = nib_sum128(qb);
                dwa[u] = half_lo(wb[u].d[0]);
                dwb[u] = half_hi(wb[u].d[4]);
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (m < mcc) {
                    const uint8_t *rec = xs + ((size_t)m * P + p) * kRec;
                    const u32x4a16 ha = *reinterpret_cast<const u32x4a16 *>(rec);
                    const u32x4a16 la = *reinterpret_cast<const u32x4a16 *>(rec + 16);
                    const u32x4a16 hb = *reinterpret_cast<const u32x4a16 *>(rec + 32);
                    const u32x4a16 lb = *reinterpret_cast<const u32x4a16 *>(rec + 48);
                    const f32x4 cst = *reinterpret_cast<const f32x4 *>(rec + 64);
                    const uint32_t hia[4] = {ha.x, ha.y, ha.z, ha.w}, loa[4] = {la.x, la.y, la.z, la.w};
                    const uint32_t hib[4] = {hb.x, hb.y, hb.z, hb.w}, lob[4] = {lb.x, lb.y, lb.z, lb.w};
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        uint32_t qa[4], qb[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            qa[i] = __builtin_amdgcn_alignbyte(wb[u].d[i + 1], wb[u].d[i], 2);
                            qb[i] = wb[u].d[i + 5];
                        }
                        const int32_t sa = block_sumi(qa, hia, loa, na[u]);
                        const int32_t sb = block_sumi(qb, hib, lob, nbs[u]);
                        float a = dwa[u] * fmaf((float)sa, cst.x, cst.y);
                        a = fmaf(dwb[u], fmaf((float)sb, cst.z, cst.w), a);
                        acc[u][m] = a;
                    }
                }
            }
        } else if (live) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                uint32_t qa[4], qb[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    qa[i] = __builtin_amdgcn_alignbyte(wb[u].d[i + 1], wb[u].d[i], 2);
                    qb[i] = wb[u].d[i + 5];
                }
                const int32_t na = nib_sum128(qa), nbs = nib_sum128(qb);
                const float dwa = half_lo(wb[u].d[0]);
                const float dwb = half_hi(wb[u].d[4]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint8_t *rec = xs + ((size_t)m * P + p) * kRec;
                    const u32x4a16 ha = *reinterpret_cast<const u32x4a16 *>(rec);
                    const u32x4a16 la = *reinterpret_cast<const u32x4a16 *>(rec + 16);
                    const u32x4a16 hb = *reinterpret_cast<const u32x4a16 *>(rec + 32);
                    const u32x4a16 lb = *reinterpret_cast<const u32x4a16 *>(rec + 48);
                    const f32x4 cst = *reinterpret_cast<const f32x4 *>(rec + 64);
                    const uint32_t hia[4] = {ha.x, ha.y, ha.z, ha.w}, loa[4] = {la.x, la.y, la.z, la.w};
                    const uint32_t hib[4] = {hb.x, hb.y, hb.z, hb.w}, lob[4] = {lb.x, lb.y, lb.z, lb.w};
                    const int32_t sa = block_sumi(qa, hia, loa, na);
                    const int32_t sb = block_sumi(qb, hib, lob, nbs);
                    float a = dwa * fmaf((float)sa, cst.x, cst.y);
                    a = fmaf(dwb, fmaf((float)sb, cst.z, cst.w), a);
                    acc[u][m] = a;
                }
            }
        }

        // All U * M sums of the wave in one transposed reduction; lane `owner` of each
        // group that shares a value holds its sum.
        constexpr int NV = pow2_at_least(kRowsW * M);
        float v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            // (R2: values U*M.. are the rows U further on, held by lanes 32..63)
            const int ii = i % (U * M);
            const bool mine = !R2 || ((i >= U * M) == (lane >= 32));
            v[i] = i < kRowsW * M && mine ? acc[ii / M][ii % M] : 0.0f;
        }
        const float s = multi_sum<NV>(v, lane);
        const int idx = multi_sum_index<NV>(lane);
        const int u = idx / M, m = idx % M;
        const bool owner = (lane & (64 / NV - 1)) == 0 && idx < kRowsW * M;
        if constexpr (JS == 1) {
            if (owner && r0 + u < N && m < mcc) y[(ROUTED ? routed_row(ra, m0c + m) : (size_t)m) * ldy + r0 + u] = s;
        } else {
            if (owner) part[((rg * U + u) * M + m) * JS + js] = s;
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
                            if (m < mcc) y[(ROUTED ? routed_row(ra, m0c + m) : (size_t)m) * ldy + r0 + u] = s;
                        }
                    }
            }
        }
        if constexpr (!ROUTED) {
            break;
        } else {
            // the expert's next chunk of routes: the same weight rows, new activation rows
            m0c += M;
            if (m0c >= rt.end) break;
            mcc = min(M, rt.end - m0c);
            again = true;
            __syncthreads();  // every wave is done with the records and partial sums
            if constexpr (M <= 2) {
                // Re-request the weight rows (L2) rather than keep them live through
                // the pass: held, they cost the 1- and 2-route kernels half their
                // occupancy, for a loop that only a tie-broken top-k repeat reaches.
                const int pl = min(p, P - 1);
                for (int u = 0; u < U; ++u)
                    load_pair(wb[u], w + (size_t)min(r0 + (R2 ? (lane >> 5) * U : 0) + u, N - 1) * row_bytes +
                                         (size_t)pl * 36);
            }
        }
    }
}

// ---- split weight layout (nibble plane + fp16 scale plane) ----
// Row n's block b: 16 nibble bytes at qs + (n*nb + b)*16 (the block_q4_0 qs bytes,
// unchanged) and its fp16 scale at d + (n*nb + b)*2, with d = qs + N*nb*16.  Every
// block is 16-byte aligned, so lane l of a wave reads block base + l of a row with
// one 16-byte load: each load instruction of a wave covers one contiguous 1 KB run.
// The activation record per (token, block) is 48 bytes in LDS: HI planes (16), LO
// planes (16), d_x and -8*s_x (8), 8 bytes of padding so that consecutive lanes'
// 16-byte reads hit disjoint banks.
constexpr int kRecS = 48;

__device__ __forceinline__ void put_block_s(uint8_t *rec, const uint32_t hi[4], const uint32_t lo[4], float dx,
                                            float c) {
    *reinterpret_cast<u32x4a16 *>(rec) = u32x4a16{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<u32x4a16 *>(rec + 16) = u32x4a16{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<u32x2a8 *>(rec + 32) = u32x2a8{__float_as_uint(dx), __float_as_uint(c)};
}

// Q8_1 item (token m, block b) -> record m*nb + b (items past the end: the spare).
__device__ __forceinline__ void finish_q8_s(uint8_t *xs, const ItemQ8 &it, int item, int nb, int n_items) {
    uint32_t hi[4], lo[4];
    make_planes(it.q, hi, lo);
    const size_t rec = item < n_items ? (size_t)item : (size_t)n_items;
    put_block_s(xs + rec * kRecS, hi, lo, half_lo(it.ds), -8.0f * half_hi(it.ds));
}

// Fused staging for the split layout: the arithmetic of finish_f32 (the reference
// quantizer's), written as per-block records.
__device__ __forceinline__ void finish_f32_s(uint8_t *xs, uint8_t *__restrict__ xq_out, const ItemF32 &it,
                                             int item, int nb, bool live) {
    const int b = min(item >> 1, nb - 1), h = item & 1;
    const f32x4 *v = it.v;
    float am[4], su[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        am[i] = fmaxf(fabsf(v[i].x), fmaxf(fabsf(v[i].y), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        float s = v[i].x + v[i].y;
        s = s + v[i].z;
        su[i] = s + v[i].w;
    }
    const float s0 = su[0] + su[2], s1 = su[1] + su[3];
    const float m0 = fmaxf(am[0], am[2]), m1 = fmaxf(am[1], am[3]);
    const float s0o = dpp<0xB1>(s0), s1o = dpp<0xB1>(s1);
    const float m0o = dpp<0xB1>(m0), m1o = dpp<0xB1>(m1);
    const float sum = (s0 + s0o) + (s1 + s1o);
    const float amax = fmaxf(fmaxf(m0, m0o), fmaxf(m1, m1o));
    const float d_inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)
        const int32_t a = round_away(v[i].x * d_inv), bb = round_away(v[i].y * d_inv);
        const int32_t c = round_away(v[i].z * d_inv), d = round_away(v[i].w * d_inv);
        q[i] = (uint32_t)(a & 0xff) | ((uint32_t)(bb & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
               ((uint32_t)(d & 0xff) << 24);
    }
    if (!live) return;
    uint8_t *rec = xs + (size_t)b * kRecS;
    uint32_t hw[2], lw[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t a = q[i] ^ 0x80808080u;
        const uint32_t bq = q[2 + i] ^ 0x80808080u;
        lw[i] = (a & 0x0f0f0f0fu) | ((bq & 0x0f0f0f0fu) << 4);
        hw[i] = ((a >> 4) & 0x0f0f0f0fu) | (bq & 0xf0f0f0f0u);
    }
    *reinterpret_cast<u32x2a8 *>(rec + 8 * h) = u32x2a8{hw[0], hw[1]};
    *reinterpret_cast<u32x2a8 *>(rec + 16 + 8 * h) = u32x2a8{lw[0], lw[1]};
    const __half hd = __float2half_rn(1.0f / d_inv);
    const __half hs = __float2half_rn(sum);
    if (h == 0)
        *reinterpret_cast<u32x2a8 *>(rec + 32) =
            u32x2a8{__float_as_uint(__half2float(hd)), __float_as_uint(-8.0f * __half2float(hs))};
    if (xq_out != nullptr) {
        uint8_t *blk = xq_out + (size_t)(b >> 2) * kQ8BlockBytes;
        const int g = b & 3;
        *reinterpret_cast<u32x2a8 *>(blk + 16 + 32 * g + 8 * h) = u32x2a8{q[0], q[1]};
        *reinterpret_cast<u32x2a8 *>(blk + 16 + 32 * g + 16 + 8 * h) = u32x2a8{q[2], q[3]};
        if (h == 0)
            *reinterpret_cast<uint32_t *>(blk + 4 * g) =
                (uint32_t)__half_as_ushort(hd) | ((uint32_t)__half_as_ushort(hs) << 16);
    }
}

// Split-layout GEMV.  Workgroup = RG row groups x JS K-slices of 128 blocks (one
// wave each, JS = ceil(K / 4096)); lane l of slice js owns blocks 128*js + l and
// 128*js + 64 + l of its wave's U rows.  Each of those blocks is one nontemporal
// 16-byte load (plus a 2-byte scale load); the integer dot is the dot8 plane form
// of gemv_q4_0_q8_1_kernel.
// ROUTED: a routed launch (RouteArgs) over E stacked split-layout experts (one
// nibble plane over all E * N rows, then one scale plane), Q8_1 input.
// R2 (K <= 2048, one K slice): a lane's second block slot, otherwise past the row
// end, takes the same block of the row U further on: a wave covers 2U rows.
template <int M, int U, int JS, int RG, bool FUSED, int EARLY, bool ROUTED = false, bool R2 = false>
__global__ __launch_bounds__(64 * JS * RG) void gemv_q4s_kernel(const uint8_t *__restrict__ w,
                                                                const void *__restrict__ xin,
                                                                uint8_t *__restrict__ xq_out,
                                                                float *__restrict__ y, int K, int N,
                                                                RouteArgs ra) {
    static_assert(!(ROUTED && FUSED), "routed launches take Q8_1 route rows");
    static_assert(!R2 || JS == 1, "paired rows: one K slice");
    constexpr int kRowsW = R2 ? 2 * U : U;  // rows per wave
    extern __shared__ __align__(16) uint8_t xs[];  // M * K/32 records of kRecS bytes + 1 spare
    __shared__ float part[JS > 1 ? RG * JS * U * M : 1];

    constexpr int kThreadsWG = 64 * JS * RG;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int js = wave % JS;
    const int rg = wave / JS;
    const int nb = K / kQK;
    const int bk0 = 128 * js + lane;       // this lane's two blocks
    const int bk1 = bk0 + 64;
    const int c0 = min(bk0, nb - 1), c1 = min(bk1, nb - 1);
    const int r0 = (blockIdx.x * RG + rg) * kRowsW;
    const int n_items = FUSED ? 2 * nb : M * nb;
    const int rounds = (n_items + kThreadsWG - 1) / kThreadsWG;
    RouteTile rt{0, 0, 0, M, M};
    size_t plane_rows = N, row0 = 0;  // rows of the buffer's planes, first row of this matrix
    if constexpr (ROUTED) {
        if (!route_tile(ra, M, rt)) return;
        if (rt.which) w = ra.w2;
        plane_rows = (size_t)ra.n_experts * N;
        row0 = (size_t)rt.expert * N;
        y += (size_t)rt.which * N;
    }
    const int ldy = ROUTED ? ra.ldy : N;
    int m0c = rt.m0, mcc = rt.mc;  // the current chunk of routes (routed launches)
    bool again = false;            // a later chunk: all its items are loaded in the pass
    const uint16_t *__restrict__ dpl = reinterpret_cast<const uint16_t *>(w + plane_rows * nb * 16);

    // 1) activation requests (L2-resident), ahead of the weights
    using Item = typename std::conditional<FUSED, ItemF32, ItemQ8>::type;
    Item early[EARLY];
#pragma unroll
    for (int r = 0; r < EARLY; ++r) {
        const int item = threadIdx.x + r * kThreadsWG;
        if constexpr (FUSED) {
            issue_f32(early[r], reinterpret_cast<const float *>(xin), item, nb);
        } else {
            if constexpr (ROUTED)
                issue_q8_routed<M>(early[r], reinterpret_cast<const uint8_t *>(xin), item, nb, ra.n_routes, m0c, mcc);
            else
                issue_q8<M>(early[r], reinterpret_cast<const uint8_t *>(xin), item, nb);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2) weight requests: per row, two coalesced 16-byte nibble loads and two scales
    u32x4a16 wq[U][2];
    uint32_t wd[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t base = (row0 + (size_t)min(r0 + u, N - 1)) * nb;
        const size_t base1 = R2 ? (row0 + (size_t)min(r0 + U + u, N - 1)) * nb : base;  // slot 1's row
        const int cs1 = R2 ? c0 : c1;                                                       // slot 1's block
        wq[u][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a16 *>(w + (base + c0) * 16));
        wq[u][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a16 *>(w + (base1 + cs1) * 16));
        wd[u][0] = dpl[base + c0];
        wd[u][1] = dpl[base1 + cs1];
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3) the early items (routed launches: before the chunk loop, so that they are not
    //    held across it; later chunks load every item in their pass)
    uint8_t *xq_w = (FUSED && blockIdx.x == 0) ? xq_out : nullptr;
#pragma unroll
    for (int r = 0; r < EARLY; ++r) {
        const int item = threadIdx.x + r * kThreadsWG;
        if constexpr (FUSED) {
            finish_f32_s(xs, xq_w, early[r], item, nb, item < n_items);
        } else {
            finish_q8_s(xs, early[r], item, nb, n_items);
        }
    }
    const int lane_o = lane, js_o = js, rg_o = rg, bk0_o = bk0, r0_o = r0;  // (see the pass)
    for (;;) {  // one pass; routed launches: one per chunk of routes
        // (lane values per pass: as in gemv_q4_0_q8_1_kernel)
        const int tid = ROUTED ? opaque_int(threadIdx.x) : (int)threadIdx.x;
        const int lane = ROUTED ? (tid & 63) : lane_o;
        const int js = ROUTED ? (tid >> 6) % JS : js_o;
        const int rg = ROUTED ? (tid >> 6) / JS : rg_o;
        const int bk0 = ROUTED ? 128 * js + lane : bk0_o;
        const int bk1 = bk0 + 64;
        const int c0 = min(bk0, nb - 1), c1 = min(bk1, nb - 1);
        const int r0 = ROUTED ? (int)(blockIdx.x * RG + rg) * kRowsW : r0_o;
        // 3) activation records of the whole K range in LDS, once per workgroup (routed:
        //    per chunk of routes)
        for (int r = (ROUTED && again) ? 0 : EARLY; r < rounds; ++r) {  // the rest, load-then-use
            const int item = tid + r * kThreadsWG;
            Item it;
            if constexpr (FUSED) {
                issue_f32(it, reinterpret_cast<const float *>(xin), item, nb);
                finish_f32_s(xs, xq_w, it, item, nb, item < n_items);
            } else {
                if constexpr (ROUTED)
                    issue_q8_routed<M>(it, reinterpret_cast<const uint8_t *>(xin), item, nb, ra.n_routes, m0c, mcc);
                else
                    issue_q8<M>(it, reinterpret_cast<const uint8_t *>(xin), item, nb);
                finish_q8_s(xs, it, item, nb, n_items);
            }
        }
        __syncthreads();

        // 4) rows in load order
        float acc[kRowsW][M];
#pragma unroll
        for (int u = 0; u < kRowsW; ++u)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[u][m] = 0.0f;

        if constexpr (ROUTED) {
            // Token-outer (as in gemv_q4_0_q8_1_kernel): tokens past the expert's routes
            // cost no dot products; every sum adds block k = 0, then k = 1, as below.
            int32_t ns[U][2];
            float dw[U][2];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    // opaque per pass: keeps the weight terms after the staging (as in
                    // gemv_q4_0_q8_1_kernel)
                    asm volatile("" : "+v"(wq[u][k]), "+v"(wd[u][k]));
                    const uint32_t q[4] = {wq[u][k].x, wq[u][k].y, wq[u][k].z, wq[u][k].w};
                    ns[u][k] = nib_sum128(q);
                    dw[u][k] = __half2float(__ushort_as_half((unsigned short)wd[u][k]));
                }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (m < mcc) {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const bool live = ((k && !R2) ? bk1 : bk0) < nb;
                        const uint8_t *rec = xs + ((size_t)m * nb + ((k && !R2) ? c1 : c0)) * kRecS;
                        const u32x4a16 h4 = *reinterpret_cast<const u32x4a16 *>(rec);
                        const u32x4a16 l4 = *reinterpret_cast<const u32x4a16 *>(rec + 16);
                        const u32x2a8 c2 = *reinterpret_cast<const u32x2a8 *>(rec + 32);
                        const uint32_t hi[4] = {h4.x, h4.y, h4.z, h4.w}, lo[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const uint32_t q[4] = {wq[u][k].x, wq[u][k].y, wq[u][k].z, wq[u][k].w};
                            const int32_t sv = block_sumi(q, hi, lo, ns[u][k]);
                            const float v = dw[u][k] * fmaf((float)sv, __uint_as_float(c2.x), __uint_as_float(c2.y));
                            acc[u + (R2 ? k * U : 0)][m] += live ? v : 0.0f;
                        }
                    }
                }
            }
        } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const bool live = ((k && !R2) ? bk1 : bk0) < nb;
                const int cb = (k && !R2) ? c1 : c0;
                const uint32_t q[4] = {wq[u][k].x, wq[u][k].y, wq[u][k].z, wq[u][k].w};
                const int32_t ns = nib_sum128(q);
                const float dw = __half2float(__ushort_as_half((unsigned short)wd[u][k]));
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint8_t *rec = xs + ((size_t)m * nb + cb) * kRecS;
                    const u32x4a16 h4 = *reinterpret_cast<const u32x4a16 *>(rec);
                    const u32x4a16 l4 = *reinterpret_cast<const u32x4a16 *>(rec + 16);
                    const u32x2a8 c2 = *reinterpret_cast<const u32x2a8 *>(rec + 32);
                    const uint32_t hi[4] = {h4.x, h4.y, h4.z, h4.w}, lo[4] = {l4.x, l4.y, l4.z, l4.w};
                    const int32_t sv = block_sumi(q, hi, lo, ns);
                    const float v = dw * fmaf((float)sv, __uint_as_float(c2.x), __uint_as_float(c2.y));
                    acc[u + (R2 ? k * U : 0)][m] += live ? v : 0.0f;
                }
            }
        }
        }

        constexpr int NV = pow2_at_least(kRowsW * M);
        float v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = i < kRowsW * M ? acc[i / M][i % M] : 0.0f;
        const float s = multi_sum<NV>(v, lane);
        const int idx = multi_sum_index<NV>(lane);
        const int u = idx / M, m = idx % M;
        const bool owner = (lane & (64 / NV - 1)) == 0 && idx < kRowsW * M;
        if constexpr (JS == 1) {
            if (owner && r0 + u < N && m < mcc) y[(ROUTED ? routed_row(ra, m0c + m) : (size_t)m) * ldy + r0 + u] = s;
        } else {
            if (owner) part[((rg * U + u) * M + m) * JS + js] = s;
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
                            if (m < mcc) y[(ROUTED ? routed_row(ra, m0c + m) : (size_t)m) * ldy + r0 + u] = s;
                        }
                    }
            }
        }
        if constexpr (!ROUTED) {
            break;
        } else {
            // the expert's next chunk of routes: the same weight rows, new activation rows
            m0c += M;
            if (m0c >= rt.end) break;
            mcc = min(M, rt.end - m0c);
            again = true;
            __syncthreads();  // every wave is done with the records and partial sums
            if constexpr (M <= 2) {  // (as in gemv_q4_0_q8_1_kernel)
                for (int u = 0; u < U; ++u) {
                    const size_t base = (row0 + (size_t)min(r0 + u, N - 1)) * nb;
                    const size_t base1 = R2 ? (row0 + (size_t)min(r0 + U + u, N - 1)) * nb : base;
                    const int cs1 = R2 ? c0 : c1;
                    wq[u][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a16 *>(w + (base + c0) * 16));
                    wq[u][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a16 *>(w + (base1 + cs1) * 16));
                    wd[u][0] = dpl[base + c0];
                    wd[u][1] = dpl[base1 + cs1];
                }
            }
        }
    }
}

// Row groups per workgroup (the activation staging of a workgroup is shared by
// its RG row groups of U rows).  Single-token decode favours wide workgroups of
// short row groups; multi-token batches favour four row groups of four rows.
constexpr int kRg1 = 8;    // row groups per workgroup, Q8_1-input decode (M=1, one K slice)
constexpr int kU1 = 2;     // rows per wave, Q8_1-input decode
constexpr int kRg1Js3 = 4; // row groups at M=1 with three K slices
constexpr int kRgM = 4;    // row groups, batches 2..8 (one K slice)
constexpr int kU4 = 4;     // rows per wave at batch 4
// The fused decode step (fp32 x quantized in every workgroup) prefers fewer,
// deeper workgroups: four rows per wave, four row groups (K <= 4096), which halves
// the workgroups that re-read and re-quantize x (7.22 against 7.44 us at K=4096,
// N=11008 on one box; the Q8_1-input kernel is faster with two rows per wave).
constexpr int kU1F = 4;
constexpr int kRg1F = 4;
template <int M, int JS, bool FUSED = false>
constexpr int rg_for() {
    if (M == 1 && FUSED && JS == 1) return kRg1F;
    if (M == 1) return JS == 1 ? kRg1 : JS == 2 ? 4 : JS == 3 ? kRg1Js3 : 2;
    return JS == 1 ? kRgM : JS == 2 ? 2 : 1;
}

// Split layout: row groups per workgroup.
#ifndef JJO_Q4S_RG1F
#define JJO_Q4S_RG1F 4
#endif
#ifndef JJO_Q4S_RG1
#define JJO_Q4S_RG1 4
#endif
template <int M, int JS, bool FUSED = false>
constexpr int rg_for_s() {
    if (M == 1 && FUSED && JS == 1) return JJO_Q4S_RG1F;
    // Three K slices (K 8193..12288): the Q8_1-input kernel prefers twice the
    // workgroups of half the rows (K=11008, N=4096: 6.25-6.59 against 6.65-6.88 us,
    // with two rows per wave); the fused step keeps four row groups, since every
    // workgroup re-stages the fp32 x (44 KB at K=11008).
    if (M == 1) return JS == 1 ? JJO_Q4S_RG1 : JS == 2 ? 4 : JS == 3 ? (FUSED ? 4 : 2) : 2;
    return JS == 1 ? kRgM : JS == 2 ? 2 : 1;
}

// Routed launches: every workgroup stages its routes' whole activation rows, so
// long rows (the down projection's K = I) want more row groups per workgroup to
// spread that staging over more weight rows.
#ifndef JJO_RT_RG2
#define JJO_RT_RG2 4
#endif
#ifndef JJO_RT_RG3
#define JJO_RT_RG3 4
#endif
#ifndef JJO_RT_RG4
#define JJO_RT_RG4 4
#endif
#ifndef JJO_RT_RG4_BLK_M4
#define JJO_RT_RG4_BLK_M4 4
#endif
#ifndef JJO_RT_RG1_M1
#define JJO_RT_RG1_M1 0  // one K slice, one route per chunk: 0 = the dense kernel's choice
#endif
#ifndef JJO_RT_RG1_M2
#define JJO_RT_RG1_M2 0  // one K slice, two-route chunks: 0 = JJO_RT_RG1_MX
#endif
#ifndef JJO_RT_RG1_MX
#define JJO_RT_RG1_MX 0  // one K slice, 2- and 4-route chunks: 0 = the dense kernel's choice
#endif
// One route per chunk (at most one route per active expert, e.g. E=8 top-2 at 1-4
// tokens) at three or four K slices: only the weight stream is left to hide, and
// twice as many 2-row-group workgroups hide it better (E=8 down projection, T=1..4:
// I=14336 2-6%, I=11008 1-3% per FFN step; 2- and 4-route chunks lose 1-15% at 2).
#ifndef JJO_RT_RG2_M1
#define JJO_RT_RG2_M1 0  // two K slices, one route per chunk: 0 = JJO_RT_RG2
#endif
#ifndef JJO_RT_RG3_M1
#define JJO_RT_RG3_M1 2
#endif
#ifndef JJO_RT_RG4_M1
#define JJO_RT_RG4_M1 2
#endif
#ifndef JJO_RT_RG4_M2
#define JJO_RT_RG4_M2 2  // four K slices, two-route chunks (E=8 top-2 T=8: 2-3%)
#endif
template <bool SPLIT, int M, int JS, bool FUSED, bool ROUTED>
constexpr int rg_pick() {
    if (ROUTED && JS == 2 && M == 1 && JJO_RT_RG2_M1 > 0) return JJO_RT_RG2_M1;
    if (ROUTED && JS == 2) return JJO_RT_RG2;
    if (ROUTED && JS == 3 && M == 1 && JJO_RT_RG3_M1 > 0) return JJO_RT_RG3_M1;
    if (ROUTED && JS == 3) return JJO_RT_RG3;
    if (ROUTED && JS == 4 && M == 1) return JJO_RT_RG4_M1;
    if (ROUTED && JS == 4 && M == 2) return JJO_RT_RG4_M2;
    if (ROUTED && JS == 1 && M == 1 && JJO_RT_RG1_M1 > 0) return JJO_RT_RG1_M1;
    if (ROUTED && JS == 1 && M == 2 && JJO_RT_RG1_M2 > 0) return JJO_RT_RG1_M2;
    if (ROUTED && JS == 1 && M > 1 && JJO_RT_RG1_MX > 0) return JJO_RT_RG1_MX;
    if (ROUTED && JS == 4) return (!SPLIT && M == 4) ? JJO_RT_RG4_BLK_M4 : JJO_RT_RG4;
    return SPLIT ? rg_for_s<M, JS, FUSED>() : rg_for<M, JS, FUSED>();
}

// Routed launches (ROUTED) run over the gy expert slots of `ra`.
template <bool SPLIT, int M, int U, int JS, bool FUSED, int EARLY, bool ROUTED = false, bool R2 = false>
hipError_t launch_cfg(const void *w, const void *xin, uint8_t *xq_out, float *y, int K, int N, hipStream_t stream,
                      const RouteArgs &ra = RouteArgs{}, int gy = 1) {
    constexpr int RG = rg_pick<SPLIT, M, JS, FUSED, ROUTED>();
    constexpr int kRowsW = R2 ? 2 * U : U;
    const int groups = (N + kRowsW - 1) / kRowsW;
    const int blocks = (groups + RG - 1) / RG;
    const size_t smem = SPLIT ? ((size_t)M * (K / 32) + 1) * kRecS : ((size_t)M * (K / 64) + 1) * kRec;
    const void *kern = SPLIT ? (const void *)gemv_q4s_kernel<M, U, JS, RG, FUSED, EARLY, ROUTED, R2>
                             : (const void *)gemv_q4_0_q8_1_kernel<M, U, JS, RG, FUSED, EARLY, ROUTED, R2>;
    if (smem > 64 * 1024) {
        // Raise this instantiation's dynamic-LDS limit to what the call needs.
        hipError_t e = ensure_dynamic_lds(kern, smem);
        if (e != hipSuccess) return e;
    }
    if constexpr (SPLIT) {
        hipLaunchKernelGGL((gemv_q4s_kernel<M, U, JS, RG, FUSED, EARLY, ROUTED, R2>), dim3(blocks, gy),
                           dim3(64 * JS * RG), smem, stream, (const uint8_t *)w, xin, xq_out, y, K, N, ra);
    } else {
        hipLaunchKernelGGL((gemv_q4_0_q8_1_kernel<M, U, JS, RG, FUSED, EARLY, ROUTED, R2>), dim3(blocks, gy),
                           dim3(64 * JS * RG), smem, stream, (const uint8_t *)w, xin, xq_out, y, K, N, ra);
    }
    return hipGetLastError();
}

template <bool SPLIT, int M, int U, int JS, bool FUSED, bool ROUTED = false, bool R2 = false>
hipError_t launch_js(const void *w, const void *xin, uint8_t *xq_out, float *y, int K, int N, hipStream_t stream,
                     const RouteArgs &ra = RouteArgs{}, int gy = 1) {
    constexpr int RG = rg_pick<SPLIT, M, JS, FUSED, ROUTED>();
    const int n_items = FUSED ? 2 * (K / kQK) : M * (K / kQK);
    const int rounds = (n_items + 64 * JS * RG - 1) / (64 * JS * RG);
    // Routed block_q4_0 at 4 routes and four K slices: only the first round ahead of
    // the weights (its chunk loop keeps the 36 raw weight dwords of four rows live;
    // two early rounds spill at 1024 threads' 128 registers).
    if constexpr (ROUTED && !SPLIT && M == 4 && JS == 4 && RG == 4)
        return launch_cfg<SPLIT, M, U, JS, FUSED, 1, ROUTED, R2>(w, xin, xq_out, y, K, N, stream, ra, gy);
    if (rounds <= 1) return launch_cfg<SPLIT, M, U, JS, FUSED, 1, ROUTED, R2>(w, xin, xq_out, y, K, N, stream, ra, gy);
    if (rounds <= 2) return launch_cfg<SPLIT, M, U, JS, FUSED, 2, ROUTED, R2>(w, xin, xq_out, y, K, N, stream, ra, gy);
    return launch_cfg<SPLIT, M, U, JS, FUSED, 4, ROUTED, R2>(w, xin, xq_out, y, K, N, stream, ra, gy);
}

#ifndef JJO_GEMV_R2
#define JJO_GEMV_R2 1
#endif
template <bool SPLIT, int M, int U, bool FUSED, bool ROUTED = false>
hipError_t launch_m(const void *w, const void *xin, uint8_t *xq_out, float *y, int K, int N, hipStream_t stream,
                    const RouteArgs &ra = RouteArgs{}, int gy = 1) {
    const int js = (K / 64 + 63) / 64;
    switch (js) {
        case 1:
            // Rows of at most 64 blocks: two rows per wave instruction (R2), unless that
            // leaves fewer workgroups than CUs (N=2048 at batch 4: 6.12 against 5.76 us).
            if (K <= 2048 && JJO_GEMV_R2) {
                constexpr int kRowsWG = 2 * U * rg_pick<SPLIT, M, 1, FUSED, ROUTED>();
                if ((int64_t)((N + kRowsWG - 1) / kRowsWG) * gy >= device_cu_count())
                    return launch_js<SPLIT, M, U, 1, FUSED, ROUTED, true>(w, xin, xq_out, y, K, N, stream, ra, gy);
            }
            return launch_js<SPLIT, M, U, 1, FUSED, ROUTED>(w, xin, xq_out, y, K, N, stream, ra, gy);
        case 2: return launch_js<SPLIT, M, U, 2, FUSED, ROUTED>(w, xin, xq_out, y, K, N, stream, ra, gy);
        case 3:
            return launch_js<SPLIT, M, (SPLIT && M == 1 && !FUSED) ? 2 : U, 3, FUSED, ROUTED>(w, xin, xq_out, y, K, N,
                                                                                           stream, ra, gy);
        case 4: return launch_js<SPLIT, M, U, 4, FUSED, ROUTED>(w, xin, xq_out, y, K, N, stream, ra, gy);
        default: return hipErrorInvalidValue;  // K > 16384: the C ABI routes these to the MFMA GEMM
    }
}


}  // namespace

hipError_t launch_gemv_dot4(const void *w, const void *xq, float *y, int K, int N, int M,
                            hipStream_t stream) {
    switch (M) {
        case 1: return launch_m<false, 1, kU1, false>(w, xq, nullptr, y, K, N, stream);
        case 2: return launch_m<false, 2, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 3: return launch_m<false, 3, 4, false>(w, xq, nullptr, y, K, N, stream);
        case 4: return launch_m<false, 4, kU4, false>(w, xq, nullptr, y, K, N, stream);
        case 5: return launch_m<false, 5, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 6: return launch_m<false, 6, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 7: return launch_m<false, 7, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 8: return launch_m<false, 8, 2, false>(w, xq, nullptr, y, K, N, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_fused(const void *w, const float *x, void *xq_out, float *y, int K, int N,
                             hipStream_t stream) {
    return launch_m<false, 1, kU1F, true>(w, x, (uint8_t *)xq_out, y, K, N, stream);
}

#ifndef JJO_Q4S_U1
#define JJO_Q4S_U1 4
#endif
#ifndef JJO_Q4S_U1F
#define JJO_Q4S_U1F 4
#endif

hipError_t launch_gemv_q4s(const void *w, const void *xq, float *y, int K, int N, int M, hipStream_t stream) {
    switch (M) {
        case 1: return launch_m<true, 1, JJO_Q4S_U1, false>(w, xq, nullptr, y, K, N, stream);
        case 2: return launch_m<true, 2, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 3: return launch_m<true, 3, 4, false>(w, xq, nullptr, y, K, N, stream);
        case 4: return launch_m<true, 4, 4, false>(w, xq, nullptr, y, K, N, stream);
        case 5: return launch_m<true, 5, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 6: return launch_m<true, 6, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 7: return launch_m<true, 7, 2, false>(w, xq, nullptr, y, K, N, stream);
        case 8: return launch_m<true, 8, 2, false>(w, xq, nullptr, y, K, N, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_q4s_fused(const void *w, const float *x, void *xq_out, float *y, int K, int N,
                                 hipStream_t stream) {
    return launch_m<true, 1, JJO_Q4S_U1F, true>(w, x, (uint8_t *)xq_out, y, K, N, stream);
}

#ifndef JJO_RT_MT4_MAXK_SPLIT
#define JJO_RT_MT4_MAXK_SPLIT 16384
#endif
// Rows per wave of the one-route routed instances: split as the dense decode
// kernel; block_q4_0 at 4 instead of 2 (E=8 top-2 FFN T=4: 142.9 -> 138.7 us; split
// at 2 or 8 and block_q4_0 at 1 were slower).
#ifndef JJO_RT_U1_SPLIT
#define JJO_RT_U1_SPLIT JJO_Q4S_U1
#endif
#ifndef JJO_RT_U1_BLOCK
#define JJO_RT_U1_BLOCK 4
#endif
// Rows per wave of the 2- and 4-route instances: 2-route chunks at 4 rows (E=8 top-2
// FFN T=8: 210.9 -> 197.0 us block, 202.0 -> 193.3 split; 1 row 252-254); 4-route
// chunks at 2 rows were slower (T=16 250.8 -> 294.8).
#ifndef JJO_RT_U2_SPLIT
#define JJO_RT_U2_SPLIT 4
#endif
#ifndef JJO_RT_U2_BLOCK
#define JJO_RT_U2_BLOCK 4
#endif
#ifndef JJO_RT_U4_SPLIT
#define JJO_RT_U4_SPLIT 4
#endif
#ifndef JJO_RT_U4_BLOCK
#define JJO_RT_U4_BLOCK kU4
#endif
int gemv_routed_chunk(int max_routes_per_expert, int K, bool split) {
    const int cap = split && K > JJO_RT_MT4_MAXK_SPLIT ? 2 : 4;
    const int mt = max_routes_per_expert <= 1 ? 1 : max_routes_per_expert <= 2 ? 2 : 4;
    return mt < cap ? mt : cap;
}

hipError_t launch_gemv_routed(const void *w, const void *w2, const void *xq, const int32_t *expert_offsets,
                              int n_experts, int n_routes, int max_routes_per_expert, float *y, int ldy, int K, int N,
                              bool split, hipStream_t stream, const int32_t *route_dst) {
    if (K > 16384 || max_routes_per_expert < 1) return hipErrorInvalidValue;
    const int mt = gemv_routed_chunk(max_routes_per_expert, K, split);
    const int slots = n_experts < n_routes ? n_experts : n_routes;
    const RouteArgs ra{expert_offsets, (const uint8_t *)w2, route_dst, n_experts, n_routes, slots, ldy};
    const int gy = slots * (w2 != nullptr ? 2 : 1);
    if (split) {
        switch (mt) {
            case 1: return launch_m<true, 1, JJO_RT_U1_SPLIT, false, true>(w, xq, nullptr, y, K, N, stream, ra, gy);
            case 2: return launch_m<true, 2, JJO_RT_U2_SPLIT, false, true>(w, xq, nullptr, y, K, N, stream, ra, gy);
            default: return launch_m<true, 4, JJO_RT_U4_SPLIT, false, true>(w, xq, nullptr, y, K, N, stream, ra, gy);
        }
    }
    switch (mt) {
        case 1: return launch_m<false, 1, JJO_RT_U1_BLOCK, false, true>(w, xq, nullptr, y, K, N, stream, ra, gy);
        case 2: return launch_m<false, 2, JJO_RT_U2_BLOCK, false, true>(w, xq, nullptr, y, K, N, stream, ra, gy);
        default: return launch_m<false, 4, JJO_RT_U4_BLOCK, false, true>(w, xq, nullptr, y, K, N, stream, ra, gy);
    }
}

}  // namespace jjo
