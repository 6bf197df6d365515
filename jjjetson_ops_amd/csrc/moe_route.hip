// MoE routing around the Q4_0 expert GEMMs on gfx950: top-k gating, dispatch
// (stable sort of routes by expert plus the permuted Q8_1 activation rows) and
// combine.  Semantics follow the reference's moe_top_k / moe_dispatch_sota /
// moe_combine_sota kernels; the data movement is redesigned for this path:
//   * dispatch gathers Q8_1 blocks (1.125 B per value) instead of fp32 rows: the
//     activation is quantized once per token, before the permutation, which gives
//     the same bytes as quantizing the permuted rows (quantization is per row);
//   * the route sort is a counting sort in one workgroup (16 waves, each owning a
//     contiguous range of routes; ranks inside a wave come from ballots), which is
//     stable exactly like the reference's radix sort.
#include <hip/hip_runtime.h>

#include "q4q8_common.hpp"
#include "q8_1_quant.hpp"

namespace jjo {
namespace {

// ---------------------------------------------------------------- top-k
// One wave per token (num_experts <= 1024, top_k <= 32).
// Selection: moe_top_k.cu:120-176 -- top_k rounds; round k scans e = 0..E-1 with
// v(e) = -inf for an expert taken in an earlier round, else the logit, keeps e = 0's
// value first and takes a later e only when strictly greater; ids[k] in selection
// order.  That keeps the smallest id of the largest non-NaN value, or expert 0 when
// v(0) is NaN (nothing compares greater than NaN), and it re-selects a taken expert
// once only -inf values are left; the wave computes exactly that: each lane holds
// experts lane + 64j in registers with a taken bit each, and a lane-local best
// (value, id) over its non-NaN values is reduced over the wave (larger value, then
// smaller id).
// Weights: softmax over the selected logits (delayed_softmax, moe_top_k.cu:12-55,
// 190-195): max = the first selected value, e_i = expf(v_i - max), and the sum is
// the 32-lane xor butterfly of warp_reduce_xor_sum (include/cuda_utils.cuh:37-43)
// over e_0..e_{top_k-1} held by lanes 0..top_k-1 (zeros elsewhere), run on the
// lanes themselves, so the association order is the reference's; w_i = e_i * (1 / sum).
constexpr int kTopKPerLane = 16;  // 1024 experts / 64 lanes

// All 64 lanes of the wave call this for one token; lanes 0..top_k-1 write
// weights[lane] and ids[lane].
__device__ __forceinline__ void top_k_token(const float *__restrict__ row, int num_experts, int top_k,
                                            float *__restrict__ weights, int *__restrict__ ids, int lane) {
    float v[kTopKPerLane];
#pragma unroll
    for (int j = 0; j < kTopKPerLane; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < num_experts ? row[e] : 0.0f;
    }
    const float v0 = __shfl(v[0], 0);  // expert 0's logit
    uint32_t taken = 0;                // bit j: expert lane + 64j
    bool taken0 = false;
    float my_v = 0.0f, mx = 0.0f;
    int my_id = 0;
    for (int k = 0; k < top_k; ++k) {
        float bv = -INFINITY;
        int bid = 0x7fffffff;
        bool ok = false;
#pragma unroll
        for (int j = 0; j < kTopKPerLane; ++j) {
            const int e = lane + 64 * j;
            const float x = ((taken >> j) & 1u) ? -INFINITY : v[j];
            if (e < num_experts && x == x && (!ok || x > bv)) {  // ids ascend with j
                bv = x;
                bid = e;
                ok = true;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oid = __shfl_xor(bid, off);
            const bool ook = __shfl_xor((int)ok, off) != 0;
            if (ook && (!ok || ov > bv || (ov == bv && oid < bid))) {
                bv = ov;
                bid = oid;
                ok = true;
            }
        }
        const float v0k = taken0 ? -INFINITY : v0;
        if (v0k != v0k) {  // v(0) NaN: the scan never leaves expert 0
            bv = v0k;
            bid = 0;
        }
        if (lane == (bid & 63)) taken |= 1u << (bid >> 6);
        taken0 |= bid == 0;
        if (k == 0) mx = bv;
        if (lane == k) {
            my_v = bv;
            my_id = bid;
        }
    }
    const float ex = lane < top_k ? expf(my_v - mx) : 0.0f;
    float t = ex;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) t = t + __shfl_xor(t, off);
    const float inv_sum = 1.0f / __shfl(t, 0);
    if (lane < top_k) {
        weights[lane] = ex * inv_sum;
        ids[lane] = my_id;
    }
}

constexpr int kTopKWaves = 4;  // tokens per workgroup

__global__ __launch_bounds__(64 * kTopKWaves) void moe_top_k_kernel(const float *__restrict__ logits,
                                                                    float *__restrict__ weights,
                                                                    int *__restrict__ ids, int num_tokens,
                                                                    int num_experts, int top_k) {
    const int t = blockIdx.x * kTopKWaves + (threadIdx.x >> 6);
    if (t >= num_tokens) return;  // whole waves
    top_k_token(logits + (size_t)t * num_experts, num_experts, top_k, weights + (size_t)t * top_k,
                ids + (size_t)t * top_k, threadIdx.x & 63);
}

// ---------------------------------------------------------------- dispatch
// Route r = t*top_k + k has expert ids[r].  Output position of r:
//   pos(r) = #{routes with a smaller expert} + #{r' < r with the same expert}
// (a stable sort by expert, as cub::DeviceRadixSort::SortPairs over the arange in
// moe_dispatch_sota.cu:127-136), and expert_offsets[e] = #{routes with expert < e}
// (the lower-bound search of moe_dispatch_sota.cu:45-71).
constexpr int kDispatchWaves = 16;

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

__global__ __launch_bounds__(64 * kDispatchWaves) void moe_dispatch_kernel(
    const int *__restrict__ ids, int num_routes, int num_experts, int32_t *__restrict__ expert_offsets,
    int32_t *__restrict__ src_route, int32_t *__restrict__ dst_of_route) {
    extern __shared__ int32_t cnt[];  // [kDispatchWaves][num_experts]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int per = (num_routes + kDispatchWaves - 1) / kDispatchWaves;
    const int r_beg = min(num_routes, wave * per);
    const int r_end = min(num_routes, r_beg + per);
    int32_t *my = cnt + wave * num_experts;

    for (int e = threadIdx.x; e < kDispatchWaves * num_experts; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    // per-wave histogram of its route range
    // (out-of-range ids are clamped to a valid expert: memory safety, not semantics)
    for (int r = r_beg + lane; r < r_end; r += 64) atomicAdd(&my[min(max(ids[r], 0), num_experts - 1)], 1);
    __syncthreads();
    // exclusive scan over (expert, wave): base of wave w for expert e.  Thread e
    // (num_experts <= 1024 = the workgroup) totals its expert's wave counts; a scan
    // of those totals (within each wave, then over the waves' sums) gives the
    // expert's base, then its waves' bases follow in wave order.
    __shared__ int wave_sum[kDispatchWaves];
    const int e_own = threadIdx.x;
    int tot = 0;
    if (e_own < num_experts)
        for (int w = 0; w < kDispatchWaves; ++w) tot += cnt[w * num_experts + e_own];
    int incl = tot;  // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
    }
    if (lane == 63) wave_sum[wave] = incl;
    __syncthreads();
    int base = incl - tot;
    for (int w = 0; w < wave; ++w) base += wave_sum[w];
    if (e_own < num_experts) {
        expert_offsets[e_own] = base;
        for (int w = 0; w < kDispatchWaves; ++w) {
            const int c = cnt[w * num_experts + e_own];
            cnt[w * num_experts + e_own] = base;
            base += c;
        }
        if (e_own == num_experts - 1) expert_offsets[num_experts] = base;
    }
    __syncthreads();
    // stable placement: 64 routes per step in route order; lanes with equal experts
    // are ranked by lane index through a ballot per distinct expert of the step
    for (int r0 = r_beg; r0 < r_end; r0 += 64) {
        const int r = r0 + lane;
        const bool live = r < r_end;
        const int e = live ? min(max(ids[r], 0), num_experts - 1) : -1;
        uint64_t todo = ballot64(live);
        int pos = 0;
        while (todo != 0) {
            const int leader = __builtin_ctzll(todo);
            const int el = __shfl(e, leader);
            const uint64_t grp = ballot64(live && e == el);
            if (e == el && live) pos = my[el] + __builtin_popcountll(grp & ((1ull << lane) - 1ull));
            if (lane == leader) my[el] += __builtin_popcountll(grp);
            todo &= ~grp;
        }
        if (live) {
            src_route[pos] = r;
            dst_of_route[r] = pos;
        }
    }
}

// Permuted Q8_1 activation: block (s * n_routes + p) <- block (s * num_tokens + token(p))
// with token(p) = src_route[p] / top_k (moe_dispatch_sota.cu:73-95 on Q8_1 blocks).
__global__ __launch_bounds__(256) void moe_gather_q8_1_kernel(const uint8_t *__restrict__ xq,
                                                              const int32_t *__restrict__ src_route,
                                                              uint8_t *__restrict__ xp, int num_tokens,
                                                              int n_routes, int top_k, int n_super) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte piece
    const int64_t total = (int64_t)n_super * n_routes * (kQ8BlockBytes / 16);
    if (i >= total) return;
    const int piece = (int)(i % (kQ8BlockBytes / 16));
    const int64_t blk = i / (kQ8BlockBytes / 16);
    const int p = (int)(blk % n_routes);
    const int64_t s = blk / n_routes;
    const int t = min(src_route[p] / top_k, num_tokens - 1);
    const uint4 v = *reinterpret_cast<const uint4 *>(xq + (s * num_tokens + t) * kQ8BlockBytes + 16 * piece);
    *reinterpret_cast<uint4 *>(xp + blk * kQ8BlockBytes + 16 * piece) = v;
}

// ---------------------------------------------------------------- decode routing
// Decode batches (at most kMoeDecodeRoutes routes): quantize, top-k, dispatch and
// gather in one launch.  Workgroup r owns route r = t * top_k + k: it issues the
// loads of token t's fp32 row first, then recomputes the top-k of every token
// (top_k_token, a wave per token: the same bits as moe_top_k_kernel) and
// the stable position of each route
//   pos(r) = #{r' : e(r') < e(r)} + #{r' < r : e(r') = e(r)}
// (moe_dispatch_kernel's order), and quantizes the row into Q8_1 row pos(r) of xp
// with the quantizer's group arithmetic (quantize_group8: the bytes of
// launch_quantize_q8_1 + moe_gather_q8_1).  Workgroup 0 also writes the tables.
constexpr int kDecodeRowRegs = 4;       // float4 per thread loaded up front (1024 threads' worth per step)

__device__ __forceinline__ void quantize_store_q8_1(float4 v, int i0, uint8_t *__restrict__ xp, int R, int pos) {
    uint32_t ds;
    const uint32_t q = quantize_group8(v.x, v.y, v.z, v.w, &ds);
    uint8_t *out = xp + ((size_t)(i0 / kQSuper) * R + pos) * kQ8BlockBytes;
    const int iqs = i0 % kQSuper;
    *reinterpret_cast<uint32_t *>(out + 16 + iqs) = q;
    if ((iqs & 31) == 0) *reinterpret_cast<uint32_t *>(out + 4 * (iqs / 32)) = ds;
}

__global__ __launch_bounds__(256) void moe_route_decode_kernel(
    const float *__restrict__ x, const float *__restrict__ logits, int num_tokens, int hidden, int num_experts,
    int top_k, float *__restrict__ route_w, int *__restrict__ ids, int32_t *__restrict__ expert_offsets,
    int32_t *__restrict__ src_route, int32_t *__restrict__ dst_of_route, uint8_t *__restrict__ xp) {
    __shared__ int s_ids[kMoeDecodeRoutes];
    __shared__ float s_w[kMoeDecodeRoutes];
    __shared__ int s_pos[kMoeDecodeRoutes];
    const int R = num_tokens * top_k;
    const int r_own = blockIdx.x;
    const bool lead = blockIdx.x == 0;
    // 1) this route's token row: the first 1024 * kDecodeRowRegs values in flight now
    //    (hidden % 128 == 0: every 32-lane half-wave is live or idle as a whole)
    const float *row = x + (size_t)(r_own / top_k) * hidden;
    float4 xv[kDecodeRowRegs];
#pragma unroll
    for (int i = 0; i < kDecodeRowRegs; ++i) {
        const int i0 = (threadIdx.x + i * 256) * 4;
        xv[i] = i0 < hidden ? *reinterpret_cast<const float4 *>(row + i0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // 2) top-k of every token, one wave per token
    for (int t = threadIdx.x >> 6; t < num_tokens; t += blockDim.x >> 6)
        top_k_token(logits + (size_t)t * num_experts, num_experts, top_k, s_w + t * top_k, s_ids + t * top_k,
                    threadIdx.x & 63);
    __syncthreads();
    // 3) stable positions (ids clamped to a valid expert, as in moe_dispatch_kernel)
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        const int e = min(max(s_ids[r], 0), num_experts - 1);
        int pos = 0;
        for (int j = 0; j < R; ++j) {
            const int ej = min(max(s_ids[j], 0), num_experts - 1);
            pos += (ej < e) | ((ej == e) & (j < r));
        }
        s_pos[r] = pos;
        if (lead) {
            dst_of_route[r] = pos;
            src_route[pos] = r;
            route_w[r] = s_w[r];
            ids[r] = s_ids[r];
        }
    }
    if (lead) {
        for (int e = threadIdx.x; e <= num_experts; e += blockDim.x) {
            int c = 0;
            for (int j = 0; j < R; ++j) c += min(max(s_ids[j], 0), num_experts - 1) < e;
            expert_offsets[e] = c;
        }
    }
    __syncthreads();
    // 4) Q8_1 row pos(r_own) of xp
    const int pos = s_pos[r_own];
#pragma unroll
    for (int i = 0; i < kDecodeRowRegs; ++i) {
        const int i0 = (threadIdx.x + i * 256) * 4;
        if (i0 < hidden) quantize_store_q8_1(xv[i], i0, xp, R, pos);
    }
    for (int i0 = (threadIdx.x + kDecodeRowRegs * 256) * 4; i0 < hidden; i0 += 1024)
        quantize_store_q8_1(*reinterpret_cast<const float4 *>(row + i0), i0, xp, R, pos);
}

// ---------------------------------------------------------------- combine
// y[t][h] = sum over k in order of w[t,k] * expert_out[dst(t,k)][h], acc from 0
// (moe_combine_sota.cu:21-41).  Four consecutive h per thread.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *__restrict__ expert_out,
                                                          const int32_t *__restrict__ dst_of_route,
                                                          const float *__restrict__ route_weights,
                                                          float *__restrict__ y, int hidden, int top_k) {
    const int t = blockIdx.y;
    const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (h >= hidden) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < top_k; ++k) {
        const int r = t * top_k + k;
        const float w = route_weights[r];
        const float4 v = *reinterpret_cast<const float4 *>(expert_out + (size_t)dst_of_route[r] * hidden + h);
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
    }
    *reinterpret_cast<float4 *>(y + (size_t)t * hidden + h) = acc;
}

}  // namespace

hipError_t launch_moe_top_k(const float *logits, float *weights, int *ids, int num_tokens, int num_experts,
                            int top_k, hipStream_t stream) {
    hipLaunchKernelGGL(moe_top_k_kernel, dim3((num_tokens + kTopKWaves - 1) / kTopKWaves), dim3(64 * kTopKWaves), 0,
                       stream, logits, weights, ids, num_tokens, num_experts, top_k);
    return hipGetLastError();
}

hipError_t launch_moe_dispatch(const int *ids, int num_routes, int num_experts, int32_t *expert_offsets,
                               int32_t *src_route, int32_t *dst_of_route, hipStream_t stream) {
    const size_t smem = (size_t)kDispatchWaves * num_experts * sizeof(int32_t);
    hipLaunchKernelGGL(moe_dispatch_kernel, dim3(1), dim3(64 * kDispatchWaves), smem, stream, ids, num_routes,
                       num_experts, expert_offsets, src_route, dst_of_route);
    return hipGetLastError();
}

hipError_t launch_moe_gather_q8_1(const void *xq, const int32_t *src_route, void *xp, int num_tokens, int n_routes,
                                  int top_k, int K, hipStream_t stream) {
    const int n_super = K / kQSuper;
    const int64_t total = (int64_t)n_super * n_routes * (kQ8BlockBytes / 16);
    hipLaunchKernelGGL(moe_gather_q8_1_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       (const uint8_t *)xq, src_route, (uint8_t *)xp, num_tokens, n_routes, top_k, n_super);
    return hipGetLastError();
}

hipError_t launch_moe_route_decode(const float *x, const float *logits, int num_tokens, int hidden, int num_experts,
                                  int top_k, float *route_w, int *ids, int32_t *expert_offsets, int32_t *src_route,
                                  int32_t *dst_of_route, void *xp, hipStream_t stream) {
    if (num_tokens * top_k > kMoeDecodeRoutes || hidden % kQSuper != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_route_decode_kernel, dim3((unsigned)(num_tokens * top_k)), dim3(256), 0, stream, x,
                       logits, num_tokens, hidden, num_experts, top_k, route_w, ids, expert_offsets, src_route,
                       dst_of_route, (uint8_t *)xp);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float *expert_out, const int32_t *dst_of_route, const float *route_weights,
                              float *y, int num_tokens, int hidden, int top_k, hipStream_t stream) {
    const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)num_tokens);
    hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, stream, expert_out, dst_of_route, route_weights, y,
                       hidden, top_k);
    return hipGetLastError();
}

}  // namespace jjo
