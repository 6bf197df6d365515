// C ABI of the gfx950 Q4_0 x Q8_1 path (declared in include/jjjetson_ops_amd.h).
//
// Host-buffer entries reproduce the reference host functions' data flow
// (src/cuda/q8_1.cu:148-193, src/cuda/mm_q4_0_q8_1.cu:318-380): per-call
// non-blocking stream, device temporaries, H2D, kernels, D2H, synchronize.
// Device entries only launch on the caller's stream.  Every entry validates its
// arguments and returns a status code instead of exiting the process.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "q4q8_common.hpp"

namespace jjo {

static thread_local std::string g_last_error;

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

int hip_fail(hipError_t e, const char *what) {
    return set_error(JJO_ERR_HIP, "%s failed: %s", what, hipGetErrorString(e));
}

namespace {

// The current device must be a gfx950 (MI355X-class) part: every kernel here is
// built for that ISA only.  Checked once per device and cached.
int require_gfx950() {
    static std::mutex mu;
    static std::vector<int> state;  // 0 unknown, 1 ok, 2 bad
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(JJO_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(mu);
    if ((int)state.size() <= dev) state.resize(dev + 1, 0);
    if (state[dev] == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        state[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
        if (state[dev] == 2)
            return set_error(JJO_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only",
                             dev, prop.gcnArchName);
    }
    if (state[dev] != 1) return set_error(JJO_ERR_NO_DEVICE, "device %d is not gfx950", dev);
    return JJO_OK;
}

struct Dims {
    int64_t K, ne1, ne2, ne3;
};

int parse_dims(const int64_t *dims, int ndims, Dims &d) {
    if (dims == nullptr || ndims < 1 || ndims > 4)
        return set_error(JJO_ERR_INVALID_ARG, "dims must hold 1..4 entries (got %d)", ndims);
    int64_t v[4] = {1, 1, 1, 1};
    for (int i = 0; i < ndims; ++i) v[i] = dims[i];
    for (int i = 0; i < 4; ++i)
        if (v[i] <= 0) return set_error(JJO_ERR_INVALID_ARG, "dims[%d] = %lld must be positive", i, (long long)v[i]);
    d = Dims{v[0], v[1], v[2], v[3]};
    if (d.K % kQK != 0)
        return set_error(JJO_ERR_INVALID_ARG, "dims[0] = %lld must be a multiple of 32", (long long)d.K);
    if (d.ne1 > 0x7fffffffLL || d.ne2 * d.ne3 > 65535 || d.K > (1LL << 30))
        return set_error(JJO_ERR_INVALID_ARG, "dims out of the supported range");
    return JJO_OK;
}

int64_t q8_bytes(const Dims &d) {
    const int64_t nz = d.ne2 * d.ne3;
    const int64_t blocks = nz <= 1 ? d.ne1 * ((d.K + 127) / 128) : nz * d.ne1 * 4 * ((d.K + 511) / 512);
    return blocks * kQ8BlockBytes;
}

// IEEE binary16 bits -> fp32 on the host (exact).
float half_bits_to_float(unsigned short h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-08f;  // m * 2^-24, exact
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int validate_mm(const void *w, const void *xq, const void *y, int K, int N, int M) {
    if (w == nullptr || xq == nullptr || y == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    if (K <= 0 || N <= 0 || M <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "ncols_k=%d nrows_out=%d batch=%d must be positive", K, N, M);
    if (K % kQSuper != 0)
        return set_error(JJO_ERR_INVALID_ARG, "ncols_k=%d must be a multiple of %d for block_q8_1_mmq", K, kQSuper);
    if (!aligned(w, 4)) return set_error(JJO_ERR_INVALID_ARG, "weight pointer must be 4-byte aligned");
    if (!aligned(xq, 16)) return set_error(JJO_ERR_INVALID_ARG, "Q8_1 pointer must be 16-byte aligned");
    if (!aligned(y, 16)) return set_error(JJO_ERR_INVALID_ARG, "output pointer must be 16-byte aligned");
    return JJO_OK;
}

int run_mm(const void *w, const void *xq, float *y, int K, int N, int M, int algo, hipStream_t s) {
    if (algo == JJO_ALGO_AUTO) {
        const bool gemv_ok = M <= kGemvMaxBatch && K <= kGemvMaxK && (int64_t)M * (K / 64) * 80 <= 150 * 1024;
        if (gemv_ok && M <= kGemvPreferredBatch)
            algo = JJO_ALGO_GEMV;
        else if (gemm_skinny_supported(w, xq, K, M))
            algo = JJO_ALGO_SKINNY;
        else
            algo = gemv_ok ? JJO_ALGO_GEMV : JJO_ALGO_MFMA;
    }
    hipError_t e;
    if (algo == JJO_ALGO_GEMV) {
        if (M > kGemvMaxBatch)
            return set_error(JJO_ERR_INVALID_ARG, "GEMV supports batch <= %d (got %d)", kGemvMaxBatch, M);
        if (K > kGemvMaxK)
            return set_error(JJO_ERR_INVALID_ARG, "GEMV supports ncols_k <= %d (got %d)", kGemvMaxK, K);
        if ((int64_t)M * (K / 64) * 80 > 150 * 1024)
            return set_error(JJO_ERR_INVALID_ARG, "GEMV: batch*ncols_k too large for LDS staging (batch=%d K=%d)", M, K);
        e = launch_gemv_dot4(w, xq, y, K, N, M, s);
        if (e != hipSuccess) return hip_fail(e, "gemv_q4_0_q8_1 launch");
    } else if (algo == JJO_ALGO_SKINNY) {
        if (!gemm_skinny_supported(w, xq, K, M))
            return set_error(JJO_ERR_INVALID_ARG,
                             "skinny GEMM needs batch <= %d, ncols_k %% 256 == 0 and 16-byte aligned weights "
                             "(batch=%d K=%d)", kSkinnyMaxBatch, M, K);
        e = launch_gemm_skinny(w, xq, y, K, N, M, s);
        if (e != hipSuccess) return hip_fail(e, "gemm_skinny launch");
    } else if (algo == JJO_ALGO_MFMA) {
        if ((M + 127) / 128 > 65535) return set_error(JJO_ERR_INVALID_ARG, "batch too large");
        e = launch_gemm_mfma(w, xq, y, K, N, M, s);
        if (e != hipSuccess) return hip_fail(e, "gemm_q4_0_q8_1_mfma launch");
    } else {
        return set_error(JJO_ERR_INVALID_ARG, "unknown algo %d", algo);
    }
    return JJO_OK;
}

// Test-only integer stage: one thread per (m, n, b).
__global__ void block_sums_kernel(const uint8_t *__restrict__ w, const uint8_t *__restrict__ xq,
                                  int32_t *__restrict__ out, int K, int N, int M) {
    const int nb = K / kQK;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)M * N * nb;
    if (idx >= total) return;
    const int b = (int)(idx % nb);
    const int64_t mn = idx / nb;
    const int n = (int)(mn % N);
    const int m = (int)(mn / N);
    const uint8_t *wb = w + ((size_t)n * nb + b) * kQ4BlockBytes + 2;
    const int8_t *q = (const int8_t *)(xq + ((size_t)(b / 4) * M + m) * kQ8BlockBytes + 16 + 32 * (b % 4));
    int32_t s = 0;
    for (int j = 0; j < 16; ++j) {
        s += (int32_t)(wb[j] & 0x0f) * (int32_t)q[j];
        s += (int32_t)(wb[j] >> 4) * (int32_t)q[j + 16];
    }
    out[idx] = s;
}

}  // namespace

hipError_t launch_block_sums(const void *w, const void *xq, int32_t *sumi, int K, int N, int M,
                             hipStream_t stream) {
    const int64_t total = (int64_t)M * N * (K / kQK);
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(block_sums_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const uint8_t *)w, (const uint8_t *)xq, sumi, K, N, M);
    return hipGetLastError();
}

}  // namespace jjo

using namespace jjo;

extern "C" {

const char *jjo_last_error(void) { return g_last_error.c_str(); }

const char *jjo_version(void) { return "jjjetson_ops_amd 0.1.0 (gfx950)"; }

int64_t q8_1_output_bytes(const int64_t *dims, int ndims) {
    Dims d;
    if (parse_dims(dims, ndims, d) != JJO_OK) return -1;
    return q8_bytes(d);
}

void parse_q8_1_output(const uint8_t *input, int8_t *qs_out, float *scale_out, float *sum_out,
                       int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = input + b * kQ8BlockBytes;
        memcpy(qs_out + b * 128, blk + 16, 128);
        for (int g = 0; g < 4; ++g) {
            unsigned short dh, sh;
            memcpy(&dh, blk + 4 * g, 2);
            memcpy(&sh, blk + 4 * g + 2, 2);
            scale_out[b * 4 + g] = half_bits_to_float(dh);
            sum_out[b * 4 + g] = half_bits_to_float(sh);
        }
    }
}

int q8_1_device(const float *d_input, void *d_output, const int64_t *dims, int ndims, void *stream) {
    clear_error();
    Dims d;
    int rc = parse_dims(dims, ndims, d);
    if (rc != JJO_OK) return rc;
    if (d_input == nullptr || d_output == nullptr) return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    if (!aligned(d_input, 16)) return set_error(JJO_ERR_INVALID_ARG, "input pointer must be 16-byte aligned");
    if (!aligned(d_output, 4)) return set_error(JJO_ERR_INVALID_ARG, "output pointer must be 4-byte aligned");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e = launch_quantize_q8_1(d_input, d_output, d.K, d.ne1, d.ne2 * d.ne3, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quantize_q8_1 launch");
    return JJO_OK;
}

int q8_1(const float *input, uint8_t *output, const int64_t *dims, int ndims) {
    clear_error();
    Dims d;
    int rc = parse_dims(dims, ndims, d);
    if (rc != JJO_OK) return rc;
    if (input == nullptr || output == nullptr) return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    const int64_t n_in = d.K * d.ne1 * d.ne2 * d.ne3;
    const int64_t n_out = q8_bytes(d);
    hipStream_t s = nullptr;
    float *dx = nullptr;
    void *dy = nullptr;
    rc = JJO_OK;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
    do {
        if ((e = hipMalloc((void **)&dx, n_in * sizeof(float))) != hipSuccess) { rc = hip_fail(e, "hipMalloc(x)"); break; }
        if ((e = hipMalloc(&dy, n_out)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(y)"); break; }
        if ((e = hipMemcpyAsync(dx, input, n_in * sizeof(float), hipMemcpyHostToDevice, s)) != hipSuccess) { rc = hip_fail(e, "H2D x"); break; }
        if ((e = launch_quantize_q8_1(dx, dy, d.K, d.ne1, d.ne2 * d.ne3, s)) != hipSuccess) { rc = hip_fail(e, "quantize_q8_1 launch"); break; }
        if ((e = hipMemcpyAsync(output, dy, n_out, hipMemcpyDeviceToHost, s)) != hipSuccess) { rc = hip_fail(e, "D2H y"); break; }
        if ((e = hipStreamSynchronize(s)) != hipSuccess) { rc = hip_fail(e, "hipStreamSynchronize"); break; }
    } while (0);
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    (void)hipStreamDestroy(s);
    return rc;
}

int mat_mul_q4_0_q8_1_device_algo(const void *d_w_q4_0, const void *d_x_q8_1, float *d_y, int ncols_k,
                                  int nrows_out, int batch, int algo, void *stream) {
    clear_error();
    int rc = validate_mm(d_w_q4_0, d_x_q8_1, d_y, ncols_k, nrows_out, batch);
    if (rc != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    return run_mm(d_w_q4_0, d_x_q8_1, d_y, ncols_k, nrows_out, batch, algo, (hipStream_t)stream);
}

int mat_mul_q4_0_q8_1_device(const void *d_w_q4_0, const void *d_x_q8_1, float *d_y, int ncols_k,
                             int nrows_out, int batch, void *stream) {
    return mat_mul_q4_0_q8_1_device_algo(d_w_q4_0, d_x_q8_1, d_y, ncols_k, nrows_out, batch,
                                         JJO_ALGO_AUTO, stream);
}

int mat_mul_q4_0_q8_1_f32_device(const void *d_w_q4_0, const float *d_x, void *d_quant_workspace,
                                 float *d_y, int ncols_k, int nrows_out, int batch, void *stream) {
    clear_error();
    const void *xq_check = d_quant_workspace != nullptr ? d_quant_workspace : (const void *)d_x;
    int rc = validate_mm(d_w_q4_0, xq_check, d_y, ncols_k, nrows_out, batch);
    if (rc != JJO_OK) return rc;
    if (d_x == nullptr || !aligned(d_x, 16)) return set_error(JJO_ERR_INVALID_ARG, "activation pointer must be non-null and 16-byte aligned");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (batch == 1 && ncols_k <= kGemvMaxK) {
        hipError_t e = launch_gemv_fused(d_w_q4_0, d_x, d_quant_workspace, d_y, ncols_k, nrows_out, s);
        if (e != hipSuccess) return hip_fail(e, "fused quantize+GEMV launch");
        return JJO_OK;
    }
    if (d_quant_workspace == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "quant workspace is required when batch > 1");
    hipError_t e = launch_quantize_q8_1(d_x, d_quant_workspace, ncols_k, batch, 1, s);
    if (e != hipSuccess) return hip_fail(e, "quantize_q8_1 launch");
    return run_mm(d_w_q4_0, d_quant_workspace, d_y, ncols_k, nrows_out, batch, JJO_ALGO_AUTO, s);
}

int mat_mul_q4_0_q8_1_block_sums_device(const void *d_w_q4_0, const void *d_x_q8_1, int32_t *d_sumi,
                                        int ncols_k, int nrows_out, int batch, void *stream) {
    clear_error();
    int rc = validate_mm(d_w_q4_0, d_x_q8_1, d_sumi, ncols_k, nrows_out, batch);
    if (rc != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    if ((int64_t)batch * nrows_out * (ncols_k / kQK) > (int64_t)0xffffffffLL * 256 / 2)
        return set_error(JJO_ERR_INVALID_ARG, "problem too large for the block-sum kernel");
    hipError_t e = launch_block_sums(d_w_q4_0, d_x_q8_1, d_sumi, ncols_k, nrows_out, batch, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "block_sums launch");
    return JJO_OK;
}

int mat_mul_q4_0_q8_1_grouped_device(const void *d_w_q4_0, const void *d_x_q8_1,
                                     const int32_t *d_expert_offsets, int n_experts,
                                     const int32_t *d_route_dst, float *d_y, int ncols_k,
                                     int nrows_out, int n_routes, void *stream) {
    clear_error();
    int rc = validate_mm(d_w_q4_0, d_x_q8_1, d_y, ncols_k, nrows_out, n_routes);
    if (rc != JJO_OK) return rc;
    if (d_expert_offsets == nullptr || n_experts <= 0 || n_experts > 4096)
        return set_error(JJO_ERR_INVALID_ARG, "expert_offsets must be non-null and 1 <= n_experts <= 4096");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e = launch_gemm_mfma_grouped(d_w_q4_0, d_x_q8_1, d_expert_offsets, n_experts, d_route_dst,
                                            d_y, ncols_k, nrows_out, n_routes, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "grouped gemm launch");
    return JJO_OK;
}

int mat_mul_q4_0_q8_1(const void *weight_q4_0, const float *input, uint8_t *quant_workspace,
                      float *output, const int64_t *dims, int ndims, int nrows_out, int ncols_k) {
    clear_error();
    Dims d;
    int rc = parse_dims(dims, ndims, d);
    if (rc != JJO_OK) return rc;
    // Validation of src/cuda/mm_q4_0_q8_1.cu:326-340, reported as a status.
    if (d.K != ncols_k)
        return set_error(JJO_ERR_INVALID_ARG, "input_dims[0]=%lld must equal ncols_k=%d", (long long)d.K, ncols_k);
    if (ncols_k % kQK != 0) return set_error(JJO_ERR_INVALID_ARG, "ncols_k must be multiple of %d", kQK);
    if (ncols_k % kQSuper != 0)
        return set_error(JJO_ERR_INVALID_ARG, "ncols_k must be multiple of %d for block_q8_1_mmq", kQSuper);
    if (nrows_out <= 0) return set_error(JJO_ERR_INVALID_ARG, "nrows_out must be positive");
    if (weight_q4_0 == nullptr || input == nullptr || quant_workspace == nullptr || output == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    if ((rc = require_gfx950()) != JJO_OK) return rc;

    // The activation is handled as [K, T] with T = ne1*ne2*ne3 tokens.
    const int64_t T = d.ne1 * d.ne2 * d.ne3;
    if (T > 0x7fffffffLL) return set_error(JJO_ERR_INVALID_ARG, "too many tokens");
    const int64_t n_in = d.K * T;
    const int64_t q_bytes = T * (d.K / kQSuper) * kQ8BlockBytes;
    const int64_t w_bytes = (int64_t)nrows_out * (ncols_k / kQK) * kQ4BlockBytes;
    const int64_t y_elems = (int64_t)nrows_out * T;

    hipStream_t s = nullptr;
    void *dw = nullptr, *dq = nullptr;
    float *dx = nullptr, *dy = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
    rc = JJO_OK;
    do {
        if ((e = hipMalloc((void **)&dx, n_in * sizeof(float))) != hipSuccess) { rc = hip_fail(e, "hipMalloc(x)"); break; }
        if ((e = hipMalloc(&dq, q_bytes)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(xq)"); break; }
        if ((e = hipMalloc(&dw, w_bytes)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(w)"); break; }
        if ((e = hipMalloc((void **)&dy, y_elems * sizeof(float))) != hipSuccess) { rc = hip_fail(e, "hipMalloc(y)"); break; }
        if ((e = hipMemcpyAsync(dx, input, n_in * sizeof(float), hipMemcpyHostToDevice, s)) != hipSuccess) { rc = hip_fail(e, "H2D x"); break; }
        if ((e = hipMemcpyAsync(dw, weight_q4_0, w_bytes, hipMemcpyHostToDevice, s)) != hipSuccess) { rc = hip_fail(e, "H2D w"); break; }
        if ((rc = mat_mul_q4_0_q8_1_f32_device(dw, dx, dq, dy, ncols_k, nrows_out, (int)T, s)) != JJO_OK) break;
        if ((e = hipMemcpyAsync(quant_workspace, dq, q_bytes, hipMemcpyDeviceToHost, s)) != hipSuccess) { rc = hip_fail(e, "D2H xq"); break; }
        if ((e = hipMemcpyAsync(output, dy, y_elems * sizeof(float), hipMemcpyDeviceToHost, s)) != hipSuccess) { rc = hip_fail(e, "D2H y"); break; }
        if ((e = hipStreamSynchronize(s)) != hipSuccess) { rc = hip_fail(e, "hipStreamSynchronize"); break; }
    } while (0);
    if (dx) (void)hipFree(dx);
    if (dq) (void)hipFree(dq);
    if (dw) (void)hipFree(dw);
    if (dy) (void)hipFree(dy);
    (void)hipStreamDestroy(s);
    return rc;
}

}  // extern "C"
