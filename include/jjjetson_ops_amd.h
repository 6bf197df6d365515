/*
 * jjjetson_ops_amd.h — C ABI of the MI355X (gfx950) Q4_0 x Q8_1 quantized matmul path.
 *
 * Every entry point is plain C: pointers, sizes, an int status. No C++ or torch
 * types cross this boundary.  `stream` arguments are `hipStream_t` passed as
 * `void*` (NULL = the legacy default stream).
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the AshburnLee/JJJetson_Ops tree).
 *
 * Wire formats (identical to the reference's structs):
 *   block_q8_1_mmq (144 B): half2 ds4[4] {d, s} then int8 qs[128]
 *       (src/cuda/q8_1.cu:14-18, src/cuda/mm_q4_0_q8_1.cu:41-46)
 *       Superblock (k/128) of token t lives at block index (k/128)*T + t
 *       (src/cuda/q8_1.cu:84-87).
 *   block_q4_0 (18 B): half d then uint8 qs[16]; byte j holds element j in its
 *       low nibble and element j+16 in its high nibble; value = d*(nib-8).
 *       Row-major [N][K/32] (src/cuda/mm_q4_0_q8_1.cu:35-38,119).
 *   output y: fp32, y[m*N + n] (src/cuda/mm_q4_0_q8_1.cu:286).
 */
#ifndef JJJETSON_OPS_AMD_H
#define JJJETSON_OPS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every int-returning entry point. */
#define JJO_OK 0
#define JJO_ERR_INVALID_ARG 1 /* shape / pointer / alignment validation failed */
#define JJO_ERR_HIP 2         /* a HIP runtime call failed */
#define JJO_ERR_NO_DEVICE 3   /* no usable gfx950 device */

#define JJO_QK4_0 32
#define JJO_QK8_1 32
#define JJO_QK8_1_MMQ 128
#define JJO_BLOCK_Q4_0_BYTES 18
#define JJO_BLOCK_Q8_1_MMQ_BYTES 144

/* Text of the last error raised on the calling thread ("" if none). */
const char *jjo_last_error(void);

/* Library version string. */
const char *jjo_version(void);

/*
 * Bytes the Q8_1 output of an activation with dims [K, ne1, ne2, ne3] occupies.
 * Matches the block indexing of quantize_q8_1_kernel (src/cuda/q8_1.cu:84-86),
 * including the per-slice stride ne1*4*ceil(K/512) blocks used when ne2*ne3 > 1.
 * Returns -1 on invalid dims.
 */
int64_t q8_1_output_bytes(const int64_t *dims, int ndims);

/*
 * Host-buffer quantizer.  Replaces `extern "C" void q8_1(float*, uint8_t*,
 * std::vector<int>&)` at src/cuda/q8_1.cu:148.  `input` is fp32, dim0 fastest,
 * dims = [K, ne1, ne2, ne3] (ndims 1..4, missing dims are 1).  K must be a
 * multiple of 32.  Writes q8_1_output_bytes(dims) bytes to `output`.
 * Synchronous (H2D, kernel, D2H on an internal stream).
 */
int q8_1(const float *input, uint8_t *output, const int64_t *dims, int ndims);

/*
 * Device-pointer quantizer on the caller's stream, no allocation, no copies.
 * Has no counterpart in the reference (its quantizer only has the host entry
 * above); it is the device-side quantize that mat_mul_q4_0_q8_1_device's
 * contract (src/cuda/mm_q4_0_q8_1.cu:384-392) presupposes.  `d_input` must be
 * 16-byte aligned.
 */
int q8_1_device(const float *d_input, void *d_output, const int64_t *dims, int ndims, void *stream);

/*
 * Host-side unpacking of Q8_1 blocks.  Replaces parse_q8_1_output at
 * src/cuda/q8_1.cu:197.  qs_out[n*128], scale_out[n*4] = fp32(d),
 * sum_out[n*4] = fp32(s).  Pure CPU, no device needed.
 */
void parse_q8_1_output(const uint8_t *input, int8_t *qs_out, float *scale_out, float *sum_out,
                       int64_t n_blocks);

/*
 * Host-buffer matmul.  Replaces `extern "C" void mat_mul_q4_0_q8_1(const void*,
 * float*, uint8_t*, float*, std::vector<int>&, int, int)` at
 * src/cuda/mm_q4_0_q8_1.cu:318.  Quantizes `input` ([K, T] fp32, dims as for
 * q8_1 with T = ne1*ne2*ne3) into `quant_workspace` (host, T*K/128*144 bytes),
 * then y[T][N] = dequant(W) . dequant(Xq).  Validation as the reference
 * (dims[0] == ncols_k, ncols_k % 128 == 0), but failures return
 * JJO_ERR_INVALID_ARG instead of printing.  Synchronous.
 */
int mat_mul_q4_0_q8_1(const void *weight_q4_0, const float *input, uint8_t *quant_workspace,
                      float *output, const int64_t *dims, int ndims, int nrows_out, int ncols_k);

/*
 * Device-pointer matmul on the caller's stream.  Replaces
 * mat_mul_q4_0_q8_1_device at src/cuda/mm_q4_0_q8_1.cu:394 (same argument
 * order: ncols_k, nrows_out, batch).  d_x_q8_1 is in the quantizer's layout
 * (superblock-major, see above).  Picks the decode GEMV (small batch) or the
 * int8-MFMA GEMM.  No allocation, asynchronous.
 */
int mat_mul_q4_0_q8_1_device(const void *d_w_q4_0, const void *d_x_q8_1, float *d_y, int ncols_k,
                             int nrows_out, int batch, void *stream);

/*
 * Device-pointer form of the reference's host mat_mul_q4_0_q8_1
 * (src/cuda/mm_q4_0_q8_1.cu:318-380): quantizes the fp32 activation d_x
 * ([ncols_k, batch], dim0 fastest, 16-byte aligned) into d_quant_workspace
 * (batch*ncols_k/128*144 bytes, quantizer layout; may be NULL when batch == 1
 * and the caller does not need the Q8_1 bytes) and writes
 * d_y[batch][nrows_out].  At batch == 1 both happen in one fused kernel.  No
 * allocation, asynchronous on `stream`.
 */
int mat_mul_q4_0_q8_1_f32_device(const void *d_w_q4_0, const float *d_x, void *d_quant_workspace,
                                 float *d_y, int ncols_k, int nrows_out, int batch, void *stream);

/* ------------------------------------------------------------ split weight layout
 * The offline repack of a Q4_0 matrix for the GPU (the "repacker to the
 * GPU-friendly split layout" beside the Q4_0 WeightDtype of
 * src/model/weight_loader.h:12-14).  block_q4_0 (18 B) is only 2-byte aligned
 * (src/cuda/mm_q4_0_q8_1.cu:35-38, read with 16-bit gathers at :50-62); the split
 * layout of an nrows x (ncols_k/32) block matrix keeps every byte but moves the
 * scales out, so every block's nibbles are one aligned 16-byte load:
 *     qs plane: block (n, b)'s 16 nibble bytes at (n*nb + b)*16
 *     d plane : its fp16 scale at nrows*nb*16 + (n*nb + b)*2      (nb = ncols_k/32)
 * Same size as the Q4_0 matrix.  Nibble order and values are block_q4_0's.
 * The reference layout stays the interface of every entry above; the split
 * layout is an extra, load-time format for callers that repack once.
 */

/* Bytes of a matrix in either layout (nrows*ncols_k/32*18); -1 if invalid. */
int64_t q4_0_split_bytes(int64_t nrows, int64_t ncols_k);

/* Host repackers (pure CPU, no device): block_q4_0 rows <-> split layout.
 * Buffers must not alias. */
int q4_0_to_split(const void *w_q4_0, void *w_split, int64_t nrows, int64_t ncols_k);
int q4_0_from_split(const void *w_split, void *w_q4_0, int64_t nrows, int64_t ncols_k);

/* Device repacker on `stream` (source 2-byte, destination 16-byte aligned, no
 * aliasing).  Stacked expert matrices repack as one matrix of E*nrows rows. */
int q4_0_to_split_device(const void *d_w_q4_0, void *d_w_split, int nrows, int ncols_k, void *stream);

/*
 * mat_mul_q4_0_q8_1_device (src/cuda/mm_q4_0_q8_1.cu:394, same arguments and
 * results) on a split-layout weight (16-byte aligned): the GEMV up to batch 8
 * (ncols_k <= 16384, batch*ncols_k/32*48 <= 150 KiB), the int8-MFMA GEMM
 * otherwise.
 */
int mat_mul_q4_0s_q8_1_device(const void *d_w_split, const void *d_x_q8_1, float *d_y, int ncols_k,
                              int nrows_out, int batch, void *stream);

/*
 * mat_mul_q4_0_q8_1_f32_device on a split-layout weight: quantize d_x into
 * d_quant_workspace and multiply.  At batch == 1 (ncols_k <= 16384) one fused
 * kernel does both, and d_quant_workspace may be NULL.
 */
int mat_mul_q4_0s_q8_1_f32_device(const void *d_w_split, const float *d_x, void *d_quant_workspace,
                                  float *d_y, int ncols_k, int nrows_out, int batch, void *stream);

/* Kernel selector for mat_mul_q4_0_q8_1_device_algo. */
#define JJO_ALGO_AUTO 0
#define JJO_ALGO_GEMV 1 /* streaming GEMV (v_dot8 on 4-bit planes), batch <= 8 */
#define JJO_ALGO_MFMA 2      /* int8 MFMA tile GEMM, any batch */
#define JJO_ALGO_SKINNY 3    /* int8 MFMA 16x16 tiles streaming weights per wave, batch <= 32 */
#define JJO_ALGO_SKINNY_LDS 4 /* int8 MFMA 16x16 tiles, activation resident in LDS, batch <= 16 */
#define JJO_ALGO_MFMA64 5     /* int8 MFMA GEMM with 64x64 workgroup tiles, any batch */
#define JJO_ALGO_MFMA32 6     /* int8 MFMA GEMM with 32-row x 64-token workgroup tiles, any batch */
#define JJO_ALGO_MFMA_W32 7   /* int8 MFMA GEMM, 128 x 128 tiles, one wave per 32 rows x 128 tokens */

/*
 * As mat_mul_q4_0_q8_1_device with an explicit kernel choice.  Has no
 * counterpart in the reference; it exists for parity tests and crossover
 * tuning of the one entry above.
 */
int mat_mul_q4_0_q8_1_device_algo(const void *d_w_q4_0, const void *d_x_q8_1, float *d_y,
                                  int ncols_k, int nrows_out, int batch, int algo, void *stream);

/*
 * Test-only: per-block integer dot sums sumi[(m*N + n)*(K/32) + b] =
 * sum_{j<32} nib_j * q_j with unsigned nibbles (the `sumi` of
 * q4_0_q8_1_vec_dot_impl, src/cuda/mm_q4_0_q8_1.cu:71-90).  No counterpart
 * entry in the reference; it exposes the integer stage for bit-exact checks.
 */
int mat_mul_q4_0_q8_1_block_sums_device(const void *d_w_q4_0, const void *d_x_q8_1,
                                        int32_t *d_sumi, int ncols_k, int nrows_out, int batch,
                                        void *stream);

/*
 * DIAGNOSTIC ONLY (a measurement probe, not part of the drop-in path; no
 * counterpart in the reference): one plain coalesced read of `bytes`
 * (a multiple of 16) from d_src, the HBM read floor of a single launch that the
 * decode GEMV's bandwidth is reported against.  d_out (4 bytes) is written only
 * when the data's checksum hits a sentinel.
 */
int jjo_read_floor_device(const void *d_src, int64_t bytes, uint32_t *d_out, void *stream);

/*
 * Grouped (MoE expert) matmul in one launch.  Replaces the per-expert fp32
 * moe_grouped_gemm_nt calls (src/cuda/moe/moe_pipeline_sota.cu:47-76,181-189)
 * for the Q4_0 up-projection.  Routes are sorted by expert;
 * expert_offsets[e]..expert_offsets[e+1] are expert e's routes
 * (src/cuda/moe/moe_dispatch_sota.cu:63-72).  d_x_q8_1 holds the quantized
 * routed activations, superblock-major over n_routes "tokens".  Expert e's
 * weight is d_w_q4_0 + e*nrows_out*(ncols_k/32)*18.  Route r's output row goes
 * to d_y[route_dst[r]*nrows_out ...] (route_dst may be NULL: identity).
 * expert_offsets (device, E+1 entries) must be non-decreasing with
 * expert_offsets[0] == 0 and expert_offsets[E] == n_routes; the kernel clamps
 * every range to [0, n_routes], so a malformed offset table drops routes instead
 * of reading or writing outside the buffers.  route_dst is not checked: each of
 * its entries must lie in [0, rows of d_y), or the store writes outside d_y.  (n_routes+127)/128 + n_experts must
 * not exceed 65535.  Up to 48 routes (ncols_k <= 16384) the launch is a GEMV over
 * the experts that have routes, each weight byte read once (decode batches: 2 to
 * 2.3x faster than 128-route MFMA tiles); above, the grouped MFMA GEMM.
 */
int mat_mul_q4_0_q8_1_grouped_device(const void *d_w_q4_0, const void *d_x_q8_1,
                                     const int32_t *d_expert_offsets, int n_experts,
                                     const int32_t *d_route_dst, float *d_y, int ncols_k,
                                     int nrows_out, int n_routes, void *stream);

/*
 * mat_mul_q4_0_q8_1_grouped_device on expert weights repacked into the split layout
 * (the stacked [E * nrows_out] rows repacked as one matrix, 16-byte aligned).  Same
 * arguments and rules; above 48 routes the results equal the block_q4_0 entry's bit
 * for bit (the same kernel, another weight load); up to 48 both are within fp32
 * rounding of the oracle (the two layouts' GEMVs sum a row in different orders).
 * No counterpart beyond the reference's
 * "offline repacker to the GPU-friendly split layout" (weight_loader.h:12-14).
 */
int mat_mul_q4_0s_q8_1_grouped_device(const void *d_w_split, const void *d_x_q8_1,
                                      const int32_t *d_expert_offsets, int n_experts,
                                      const int32_t *d_route_dst, float *d_y, int ncols_k,
                                      int nrows_out, int n_routes, void *stream);

/*
 * Engine linear layer with Q4_0 weights: the slot beside linear_forward_device
 * (src/cuda/linear.h:7-9, called from src/engine/transformer_runner.cpp:214-216,294,
 * 319-327).  Same argument order as the reference with the cuBLAS handle slot
 * replaced by the Q8_1 workspace:
 *   input   fp32 [num_tokens][in_features] (features fastest, the engine's layout)
 *   weight  Q4_0 [out_features][in_features/32] blocks
 *   output  fp32 [num_tokens][out_features]
 *   quant_workspace  linear_q4_0_workspace_bytes(in_features, num_tokens) bytes of
 *            device memory (may be NULL when num_tokens == 1: the decode step runs
 *            as one fused quantize+GEMV launch).
 * in_features must be a multiple of 128.  No allocation, asynchronous on `stream`.
 */
int64_t linear_q4_0_workspace_bytes(int in_features, int num_tokens);
int linear_q4_0_forward_device(void *stream, void *quant_workspace, const float *input,
                               const void *weight_q4_0, float *output, int in_features,
                               int out_features, int num_tokens);

/*
 * linear_q4_0_forward_device on weights repacked once into the split layout
 * (q4_0_to_split / q4_0_to_split_device; 16-byte aligned): the engine's fast path
 * when it repacks at load time, beside the same linear_forward_device slot.  Same
 * arguments, workspace and rules; results follow mat_mul_q4_0s_q8_1_f32_device
 * (oracle tolerance, not bit-identical to the block_q4_0 entry: other kernels).
 */
int linear_q4_0s_forward_device(void *stream, void *quant_workspace, const float *input,
                                const void *weight_split, float *output, int in_features,
                                int out_features, int num_tokens);

/*
 * Allocation-free variant of linear_q4_0_forward_device.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The Q8_1
 * activation goes to a static device buffer of linear_q4_0_noalloc_max_bytes()
 * bytes (16 MiB: e.g. 3640 tokens at in_features 4096) that the library holds on
 * every device it runs on until the process ends; larger batches are rejected with
 * JJO_ERR_INVALID_ARG.  The call allocates nothing and frees nothing.  All calls
 * on one device share that buffer: calls that overlap on one GPU (other streams,
 * other threads) race and must be serialized by the caller.  num_tokens == 1 with
 * in_features <= 16384 does not touch the buffer (the fused quantize+GEMV); any
 * other call quantizes into it.  Results equal
 * linear_q4_0_forward_device's bit for bit.
 */
int64_t linear_q4_0_noalloc_max_bytes(void);
int linear_q4_0_forward_device_noalloc(void *stream, const float *input, const void *weight_q4_0, float *output,
                                       int in_features, int out_features, int num_tokens);

/*
 * Host-buffer test wrapper around linear_q4_0_forward_device, in the argument order
 * of linear_forward_host (src/cuda/linear.h:12-13).  Synchronous.
 */
int linear_q4_0_forward_host(float *input, const void *weight_q4_0, float *output, int in_features,
                             int num_tokens, int out_features);

/* ------------------------------------------------------------------ MoE FFN
 * The Q4_0 replacement of the reference's MoE pipeline
 * (moe_pipeline_sota_forward_device, src/cuda/moe/moe_pipeline_sota.cu:163-198):
 * top-k -> dispatch -> grouped gate/up -> SwiGLU -> grouped down -> combine,
 * with Q4_0 expert weights and Q8_1 activations.  Routes are r = t*top_k + k.
 * Expert weights: w_gate, w_up Q4_0 [E][I][H/32]; w_down Q4_0 [E][H][I/32].
 */

/*
 * Top-k gating.  Replaces moe_top_k_launch_cuda (src/cuda/moe/moe_top_k.cu:218):
 * ids[t*top_k + k] = the k-th largest logit's expert (smaller id on ties),
 * weights = softmax over the top_k selected logits.  logits fp32 [T][E].
 * 1 <= top_k <= min(32, E), E <= 1024.
 */
int moe_top_k_device(void *stream, const float *logits, float *route_weights, int32_t *expert_ids,
                     int num_tokens, int num_experts, int top_k);

/*
 * Dispatch.  Replaces moe_dispatch_sota_launch_cuda
 * (src/cuda/moe/moe_dispatch_sota.cu:113-151): a stable sort of the routes by
 * expert.  expert_offsets[E+1]; src_route[p] = the route at permuted row p
 * (the reference's expanded_src_for_dest_row; token = src_route[p] / top_k);
 * dst_of_route[r] = its permuted row (the reference's inv_permuted_idx,
 * moe_combine_sota.cu:6-19).  Instead of permuting fp32 rows, x_q8_1_permuted
 * receives the Q8_1 blocks of x_q8_1 (quantizer layout over T tokens, hidden_size
 * values) in permuted order (quantizer layout over T*top_k rows).  The two Q8_1
 * pointers may both be NULL (routing tables only).
 */
int moe_dispatch_q8_1_device(void *stream, const int32_t *expert_ids, const void *x_q8_1, int num_tokens,
                             int top_k, int hidden_size, int num_experts, int32_t *expert_offsets,
                             int32_t *src_route, int32_t *dst_of_route, void *x_q8_1_permuted);

/*
 * Grouped gate|up projection of the permuted rows in one launch: gate_up[p][0:I]
 * = w_gate[e(p)] . x_p, gate_up[p][I:2I] = w_up[e(p)] . x_p (fp32 [R][2I]).
 * Replaces the first two moe_grouped_gemm_nt calls
 * (src/cuda/moe/moe_pipeline_sota.cu:181-184).  intermediate_size % 128 == 0.
 * Up to 48 routes (hidden_size <= 16384): one GEMV launch over the active experts.
 */
int moe_q4_0_gate_up_device(void *stream, const void *w_gate, const void *w_up, const void *x_q8_1_permuted,
                            const int32_t *expert_offsets, int num_experts, float *gate_up, int hidden_size,
                            int intermediate_size, int n_routes);

/*
 * The gate|up projection fused with SwiGLU and the Q8_1 quantization of its
 * result, in one grouped launch: mid_q8_1 receives the Q8_1 bytes (quantizer
 * layout over the R = n_routes permuted rows, intermediate_size values each) of
 * silu(gate) * up, bit for bit what moe_q4_0_gate_up_device followed by
 * swiglu_quantize_q8_1_device writes above 48 routes (up to 48 that gate|up runs
 * as a GEMV: each value within one quantization step), with no fp32 [R][2I] buffer.  Replaces the
 * gate/up moe_grouped_gemm_nt calls and swiglu_silu_mul_launch_cuda
 * (src/cuda/moe/moe_pipeline_sota.cu:181-191, src/cuda/swiglu.cu:5-28).
 * intermediate_size % 128 == 0.
 */
int moe_q4_0_gate_up_swiglu_q8_1_device(void *stream, const void *w_gate, const void *w_up,
                                        const void *x_q8_1_permuted, const int32_t *expert_offsets, int num_experts,
                                        void *mid_q8_1, int hidden_size, int intermediate_size, int n_routes);

/*
 * SwiGLU fused with the Q8_1 quantizer: mid = silu(gate) * up
 * (swiglu_silu_mul_launch_device, src/cuda/swiglu.cu:5-28) on gate_up [rows][2I],
 * quantized to Q8_1 (quantizer layout over `rows` tokens, I values) for the down
 * projection.  mid_f32 (optional, may be NULL) receives the fp32 mid values.
 */
int swiglu_quantize_q8_1_device(void *stream, const float *gate_up, void *mid_q8_1, float *mid_f32,
                                int rows, int intermediate_size);

/*
 * Combine.  Replaces moe_combine_sota_launch_cuda
 * (src/cuda/moe/moe_combine_sota.cu:58-66): y[t][h] = sum_k w[t,k] *
 * expert_out[dst_of_route[t*top_k+k]][h], summed in k order.  hidden_size % 4 == 0.
 */
int moe_combine_device(void *stream, const float *expert_out, const int32_t *dst_of_route,
                       const float *route_weights, float *y, int num_tokens, int hidden_size, int top_k);

/*
 * The whole Q4_0 MoE FFN on device pointers: x fp32 [T][H], logits fp32 [T][E],
 * y fp32 [T][H].  `workspace` (256-byte aligned) holds every intermediate; its
 * size is moe_q4_0_ffn_workspace_bytes(...).  Seven launches (quantize x, top-k,
 * dispatch, gather, gate|up with SwiGLU and Q8_1, down, combine); at 16 tokens or
 * fewer, or at most two routes per active expert on average (H, I <= 16384), five
 * (routing in one launch -- four above 384 routes --, gate|up over the active experts
 * into an fp32 [R][2I] part of the workspace, SwiGLU + Q8_1, down, combine).  No
 * allocation, asynchronous on `stream`.  H % 128 == 0, I % 128 == 0.
 */
int64_t moe_q4_0_ffn_workspace_bytes(int num_tokens, int hidden_size, int intermediate_size, int num_experts,
                                     int top_k);
int moe_q4_0_ffn_forward_device(void *stream, const float *x, const float *logits, const void *w_gate,
                                const void *w_up, const void *w_down, float *y, int num_tokens, int hidden_size,
                                int intermediate_size, int num_experts, int top_k, void *workspace,
                                int64_t workspace_bytes);
/* The same FFN on expert weights repacked into the split layout (each of gate, up
 * and down as one [E * rows] matrix, 16-byte aligned); y equals the block_q4_0
 * entry's bit for bit where both run the MFMA tiles (on the routed-GEMV path, both are
 * within fp32 rounding of the oracle: the two layouts' GEMVs sum a row in different
 * orders). */
int moe_q4_0s_ffn_forward_device(void *stream, const float *x, const float *logits, const void *w_gate_split,
                                 const void *w_up_split, const void *w_down_split, float *y, int num_tokens,
                                 int hidden_size, int intermediate_size, int num_experts, int top_k, void *workspace,
                                 int64_t workspace_bytes);

/* ------------------------------------------------------------------ Q4_0 weights on disk
 * The reference's loader holds F32 tensors only (WeightDtype, src/model/weight_loader.h:12-14;
 * HostTensor, :17-23).  These entries add Q4_0: a tensor of logical shape
 * [rows, cols] (rows = out_features, cols = in_features, as the engine's weights,
 * src/cuda/linear.cu:19) stored in a .safetensors file as dtype "U8", shape
 * [rows, cols/32, 18] (block_q4_0, row-major: the layout every kernel above reads),
 * marked by the header metadata entry "q4_0:<name>": "Q4_0".
 * Quantization rule (ggml's Q4_0, which the reference's MMQ consumes): per 32 values
 * mx = the value of largest magnitude (first on ties), d = mx / -8 stored fp16,
 * id = d != 0 ? 1/d : 0, nib = clamp((int)(v*id + 8.5), 0, 15).
 */
#define JJO_WEIGHT_DTYPE_F32 0  /* WEIGHT_DTYPE_F32 (weight_loader.h:13) */
#define JJO_WEIGHT_DTYPE_Q4_0 1 /* new: block_q4_0 bytes */

typedef struct jjo_host_tensor {
    char *name;
    void *data;      /* F32: float[numel]; Q4_0: rows*(cols/32) blocks of 18 bytes */
    int64_t *dims;   /* logical shape; Q4_0 tensors are [rows, cols] */
    int ndim;
    int dtype;       /* JJO_WEIGHT_DTYPE_* */
    int64_t nbytes;  /* bytes at data */
} jjo_host_tensor;

/* Bytes of a [rows, cols] Q4_0 matrix; -1 unless rows > 0 and cols is a positive multiple of 32. */
int64_t q4_0_bytes(int64_t rows, int64_t cols);

/*
 * Host fp32 [rows][cols] -> Q4_0 (num_threads <= 0: one per hardware thread).
 * No counterpart in the reference (it ships no Q4_0 quantizer); the repacker's kernel.
 */
int quantize_q4_0_host(const float *w, void *out, int64_t rows, int64_t cols, int num_threads);

/*
 * The same quantizer on device pointers (one launch, asynchronous on `stream`,
 * bit-identical to quantize_q4_0_host).  w 16-byte aligned.
 */
int quantize_q4_0_device(void *stream, const float *d_w, void *d_out, int64_t rows, int64_t cols);

/*
 * Reads every tensor of a .safetensors file: F32 tensors and Q4_0 tensors (marked
 * as above); any other dtype is an error.  Replaces safetensors_read_file
 * (src/model/safetensors_reader.h:10, safetensors_reader.cpp:369-494).  The caller
 * frees the array with jjo_host_tensors_free (weight_load_result_destroy,
 * weight_loader.h:34).  Returns 0 or a JJO_ERR_* code (nothing allocated on error).
 */
int safetensors_read_file_q4_0(const char *path, jjo_host_tensor **out_tensors, int *out_num_tensors);
void jjo_host_tensors_free(jjo_host_tensor *tensors, int num_tensors);
/* weight_load_result_find (weight_loader.h:36): the tensor named `name`, or NULL. */
const jjo_host_tensor *jjo_host_tensors_find(const jjo_host_tensor *tensors, int num_tensors, const char *name);

/*
 * Writes tensors (F32 or Q4_0, in the given order) as a standard .safetensors file.
 * No counterpart in the reference (its loader only reads).
 */
int safetensors_write_file_q4_0(const char *path, const jjo_host_tensor *tensors, int num_tensors);

/*
 * Offline repacker: copies in_path to out_path with the named 2-D F32 tensors
 * (cols % 32 == 0) quantized to Q4_0, or every such tensor when num_names < 0.
 * Streams one tensor at a time.  No counterpart in the reference.
 */
int safetensors_quantize_q4_0(const char *in_path, const char *out_path, const char *const *names, int num_names,
                              int num_threads);

#ifdef __cplusplus
}
#endif

#endif /* JJJETSON_OPS_AMD_H */
