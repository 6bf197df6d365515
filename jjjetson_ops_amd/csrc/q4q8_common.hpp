// Shared definitions of the gfx950 Q4_0 x Q8_1 path: wire formats, error
// plumbing and the kernel launchers each translation unit provides.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jjjetson_ops_amd.h"

namespace jjo {

constexpr int kQK = 32;             // values per Q4_0 block and per Q8_1 group
constexpr int kQSuper = 128;        // values per block_q8_1_mmq
constexpr int kQ8BlockBytes = 144;  // sizeof(block_q8_1_mmq)
constexpr int kQ4BlockBytes = 18;   // sizeof(block_q4_0)

// Set the calling thread's error text (printf-style).  Returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the calling thread's error text.
void clear_error();
// Map a HIP status to JJO_ERR_HIP with a message naming `what`.
int hip_fail(hipError_t e, const char *what);

#define JJO_HIP_TRY(expr)                                  \
    do {                                                   \
        hipError_t jjo_e_ = (expr);                        \
        if (jjo_e_ != hipSuccess) return ::jjo::hip_fail(jjo_e_, #expr); \
    } while (0)

// Raises `kernel`'s dynamic-LDS limit to at least `bytes` on the current device
// (hipFuncAttributeMaxDynamicSharedMemorySize), once per (kernel, device) and
// thread-safely; later calls with the same or a smaller size cost a lookup.
hipError_t ensure_dynamic_lds(const void *kernel, size_t bytes);

// Compute units of the current device (256 on MI355X; the value found when the
// C ABI checked the device).
int device_cu_count();

// Kernel launchers (asynchronous on `stream`).  Shapes are validated by the
// C-ABI layer before these are called.
hipError_t launch_quantize_q8_1(const float *x, void *y, int64_t K, int64_t ne1, int64_t nz,
                                hipStream_t stream);
hipError_t launch_gemv_dot4(const void *w, const void *xq, float *y, int K, int N, int M,
                            hipStream_t stream);
// M = 1 GEMV straight from the fp32 activation (quantized in-kernel, bit-exact with
// launch_quantize_q8_1); xq_out (nullable) receives the Q8_1 bytes.
hipError_t launch_gemv_fused(const void *w, const float *x, void *xq_out, float *y, int K, int N,
                             hipStream_t stream);
// Split weight layout (nibble plane + fp16 scale plane): GEMV at batch <= 8 from
// Q8_1 input, and the fused quantize + GEMV at batch 1.
hipError_t launch_gemv_q4s(const void *w, const void *xq, float *y, int K, int N, int M, hipStream_t stream);
hipError_t launch_gemv_q4s_fused(const void *w, const float *x, void *xq_out, float *y, int K, int N,
                                 hipStream_t stream);
// Routed GEMV over E stacked [N][K] experts (MoE decode): routes sorted by expert,
// expert_offsets[E+1], Q8_1 route rows superblock-major over n_routes rows; each
// active expert's weights are read once, its routes taken in chunks sized for
// max_routes_per_expert (routes per active expert expected; more take more chunks).
// Sorted route p's output row starts at y + p * ldy, or at y + route_dst[p] * ldy
// (route_dst nullable, entries unchecked).  w2 (nullable): a second stacked matrix of the same shape,
// computed in the same launch into columns N..2N-1 of each output row.  K <= 16384;
// split: both matrices in the split layout (planes over all E * N rows).
hipError_t launch_gemv_routed(const void *w, const void *w2, const void *xq, const int32_t *expert_offsets,
                              int n_experts, int n_routes, int max_routes_per_expert, float *y, int ldy, int K, int N,
                              bool split, hipStream_t stream, const int32_t *route_dst = nullptr);
// Routes per chunk of launch_gemv_routed (1, 2 or 4): its LDS holds that many
// activation rows of K values (48 B per 32 values split, 40 B block_q4_0).
int gemv_routed_chunk(int max_routes_per_expert, int K, bool split);
// Int8-MFMA GEMM, one wave per 32 rows x 128 tokens; weights in the split layout
// (split = true, 16-byte aligned) or block_q4_0 rows (4-byte aligned).
hipError_t launch_gemm_q4s_mfma(const void *w, const void *xq, float *y, int K, int N, int M, bool split,
                                hipStream_t stream);
// block_q4_0 rows -> split layout (n_blocks blocks; out must not alias w).
hipError_t launch_q4_0_to_split(const void *w, void *out, int64_t n_blocks, hipStream_t stream);
// Batch <= 32: int8 MFMA 16x16 tiles, weights streamed per wave, K split over 4 waves.
bool gemm_skinny_supported(const void *w, const void *xq, int K, int M);
hipError_t launch_gemm_skinny(const void *w, const void *xq, float *y, int K, int N, int M,
                              hipStream_t stream);
// The same kernel on split-layout weights (split = true).
hipError_t launch_gemm_skinny_layout(const void *w, const void *xq, float *y, int K, int N, int M, bool split,
                                     hipStream_t stream);
// Batch <= 16: activation resident in LDS, up to 4 weight tiles per workgroup.
bool gemm_skinny_persist_supported(const void *w, const void *xq, int K, int M);
hipError_t launch_gemm_skinny_persist(const void *w, const void *xq, float *y, int K, int N, int M,
                                      hipStream_t stream);
// The same kernel with the weights in either layout (split: nibble + scale planes).
hipError_t launch_gemm_skinny_persist_layout(const void *w, const void *xq, float *y, int K, int N, int M, bool split,
                                             hipStream_t stream);
// tile_rows: 64, or 32 (the stage's blocks split between wave pairs).
// split: the weights are in the split layout (16-byte aligned).
hipError_t launch_gemm_mfma64(const void *w, const void *xq, float *y, int K, int N, int M,
                              hipStream_t stream, int tile_rows, bool split = false);
hipError_t launch_gemm_mfma(const void *w, const void *xq, float *y, int K, int N, int M,
                            hipStream_t stream);
hipError_t launch_gemm_mfma_grouped(const void *w, const void *xq, const int32_t *expert_offsets,
                                    int n_experts, const int32_t *route_dst, float *y, int K,
                                    int N, int n_routes, hipStream_t stream, const void *w2 = nullptr,
                                    int n_split = 0, bool split = false);
// gate|up grouped GEMM with the SwiGLU + Q8_1 quantize epilogue: writes the Q8_1
// bytes of silu(x.W_gate) * (x.W_up) per route (I % 128 == 0) and nothing else.
hipError_t launch_gemm_gate_up_swiglu_q8_1(const void *w_gate, const void *w_up, const void *xq,
                                           const int32_t *expert_offsets, int n_experts, void *mid_q8_1, int K,
                                           int I, int n_routes, hipStream_t stream, bool split = false);
hipError_t launch_swiglu_quantize_q8_1(const float *gate_up, void *y, float *mid_out, int64_t K, int64_t rows,
                                       hipStream_t stream);
hipError_t launch_moe_top_k(const float *logits, float *weights, int *ids, int num_tokens, int num_experts,
                            int top_k, hipStream_t stream);
hipError_t launch_moe_dispatch(const int *ids, int num_routes, int num_experts, int32_t *expert_offsets,
                               int32_t *src_route, int32_t *dst_of_route, hipStream_t stream);
hipError_t launch_moe_gather_q8_1(const void *xq, const int32_t *src_route, void *xp, int num_tokens, int n_routes,
                                  int top_k, int K, hipStream_t stream);
// Decode batches (num_tokens * top_k <= kMoeDecodeRoutes, hidden % 128 == 0):
// quantize x, top-k, dispatch and the Q8_1 gather in one launch; the outputs are
// those of launch_quantize_q8_1 + launch_moe_top_k + launch_moe_dispatch +
// launch_moe_gather_q8_1 (except the unpermuted Q8_1 x, not written).
constexpr int kMoeDecodeRoutes = 384;
hipError_t launch_moe_route_decode(const float *x, const float *logits, int num_tokens, int hidden, int num_experts,
                                  int top_k, float *route_w, int *ids, int32_t *expert_offsets, int32_t *src_route,
                                  int32_t *dst_of_route, void *xp, hipStream_t stream);
hipError_t launch_moe_combine(const float *expert_out, const int32_t *dst_of_route, const float *route_weights,
                              float *y, int num_tokens, int hidden, int top_k, hipStream_t stream);
// fp32 -> Q4_0 over a flat run of n_blocks 32-value blocks.
hipError_t launch_quantize_q4_0(const float *w, void *out, int64_t n_blocks, hipStream_t stream);
hipError_t launch_block_sums(const void *w, const void *xq, int32_t *sumi, int K, int N, int M,
                             hipStream_t stream);

// Largest batch / reduction length the dot4 GEMV kernel is instantiated for
// (K is cut into at most 4 slices of 4096 values).
constexpr int kGemvMaxBatch = 8;
constexpr int kGemvMaxK = 4 * 4096;
constexpr int kSkinnyMaxBatch = 32;
// AUTO dispatch: the GEMV up to this batch, the skinny MFMA kernel above it (up to
// kSkinnyMaxBatch), the tiled MFMA GEMM beyond (measured crossovers at K=4096).
constexpr int kGemvPreferredBatch = 4;

}  // namespace jjo
