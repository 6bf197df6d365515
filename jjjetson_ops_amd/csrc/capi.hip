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

hipError_t ensure_dynamic_lds(const void *kernel, size_t bytes) {
    static std::mutex mu;
    static std::vector<std::pair<std::pair<const void *, int>, size_t>> granted;  // (kernel, device) -> bytes
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(mu);
    for (auto &g : granted)
        if (g.first.first == kernel && g.first.second == dev) {
            if (g.second >= bytes) return hipSuccess;
            e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
            if (e == hipSuccess) g.second = bytes;
            return e;
        }
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) granted.push_back({{kernel, dev}, bytes});
    return e;
}

namespace {

std::mutex g_dev_mu;
std::vector<int> g_dev_cus;  // compute units per device, filled by require_gfx950

// The current device must be a gfx950 (MI355X-class) part: every kernel here is
// built for that ISA only.  Checked once per device and cached.
int require_gfx950() {
    static std::vector<int> state;  // 0 unknown, 1 ok, 2 bad
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(JJO_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if ((int)state.size() <= dev) state.resize(dev + 1, 0);
    if (state[dev] == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        state[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
        if ((int)g_dev_cus.size() <= dev) g_dev_cus.resize(dev + 1, 0);
        g_dev_cus[dev] = prop.multiProcessorCount;
        if (state[dev] == 2)
            return set_error(JJO_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only",
                             dev, prop.gcnArchName);
    }
    if (state[dev] != 1) return set_error(JJO_ERR_NO_DEVICE, "device %d is not gfx950", dev);
    return JJO_OK;
}

// Compute units of the current device (after require_gfx950 succeeded on it).
int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    return dev < (int)g_dev_cus.size() && g_dev_cus[dev] > 0 ? g_dev_cus[dev] : 256;
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

// The grouped GEMM launches one workgroup row per possible token tile.
int check_grouped_grid(int n_routes, int n_experts) {
    if ((int64_t)(n_routes + 127) / 128 + n_experts > 65535)
        return set_error(JJO_ERR_INVALID_ARG, "grouped matmul: %d routes over %d experts exceed one launch's tiles",
                         n_routes, n_experts);
    return JJO_OK;
}

// Rows per workgroup of the small-tile GEMM (64 or 32) when the 128 x 128 GEMM would
// not fill the chip well, else 0.  The 128 x 128 tiles fill the chip only from about
// 1.5 tiles per CU; below that the 64 x 64 kernel runs four times as many workgroups
// and is up to 2x faster (K=4096: N=14336 up to M=384, N=4096 up to M=1024).  Above it
// the 128 x 128 kernel also needs its rounds (two workgroups per CU) well filled: 80%
// over one or two rounds, 70% over more.  N=11008, M=768 is 516 tiles, a second round
// for 4 of them (156 us against 128 us for the 64 x 64 kernel); 896 tiles (N=14336,
// M=1024, 88%) stay on it (198 against 213 us), and so do 1120 (M=1280, three rounds 73%
// full: 238 against 258 us).  Down to 1.5 workgroups of 64 x 64 per CU, 32-row tiles
// (twice the workgroups, each wave half of a stage's blocks) are 7-20% faster still.
int small_tile_rows(int N, int M) {
    const int64_t cus = device_cus();
    const int64_t t128 = (int64_t)((N + 127) / 128) * ((M + 127) / 128);
    const int64_t slots = 2 * cus, rounds = (t128 + slots - 1) / slots;
    const bool under = 2 * t128 < 3 * cus ||
                       (rounds <= 2 ? 5 * t128 < 4 * slots * rounds : 10 * t128 < 7 * slots * rounds);
    if (!under) return 0;
    return 2 * (int64_t)((N + 63) / 64) * ((M + 63) / 64) <= 3 * cus ? 32 : 64;
}

int run_mm(const void *w, const void *xq, float *y, int K, int N, int M, int algo, hipStream_t s) {
    if (algo == JJO_ALGO_AUTO) {
        const bool gemv_ok = M <= kGemvMaxBatch && K <= kGemvMaxK && (int64_t)M * (K / 64) * 80 <= 150 * 1024;
        // The GEMV wins up to batch 4 on rows of one K-slice (K <= 4096); with more
        // slices its per-token cost grows and the skinny kernel wins from batch 3.
        // At K <= 4096 the LDS-resident skinny kernel is 4-30% faster than the
        // per-wave one from batch 5 (N=14336: 11.2-11.6 against 12.0-14.0 us; N=11008:
        // 9.0-9.4 against 11.5-13.4 us); at larger K the per-wave kernel is faster.
        if (gemv_ok && M <= (K <= 4096 ? kGemvPreferredBatch : 2))
            algo = JJO_ALGO_GEMV;
        else if (K <= 4096 && M >= 5 && gemm_skinny_persist_supported(w, xq, K, M))
            algo = JJO_ALGO_SKINNY_LDS;
        else if (gemm_skinny_supported(w, xq, K, M))
            algo = JJO_ALGO_SKINNY;
        else if (gemv_ok)
            algo = JJO_ALGO_GEMV;
        else if (const int tr = small_tile_rows(N, M); tr != 0)
            algo = tr == 32 ? JJO_ALGO_MFMA32 : JJO_ALGO_MFMA64;
        else
            algo = JJO_ALGO_MFMA;
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
    } else if (algo == JJO_ALGO_SKINNY_LDS) {
        if (!gemm_skinny_persist_supported(w, xq, K, M))
            return set_error(JJO_ERR_INVALID_ARG,
                             "LDS-resident skinny GEMM needs batch <= 16, ncols_k %% 256 == 0 and 16-byte aligned "
                             "weights (batch=%d K=%d)", M, K);
        e = launch_gemm_skinny_persist(w, xq, y, K, N, M, s);
        if (e != hipSuccess) return hip_fail(e, "gemm_skinny_persist launch");
    } else if (algo == JJO_ALGO_MFMA64 || algo == JJO_ALGO_MFMA32) {
        if ((M + 63) / 64 > 65535) return set_error(JJO_ERR_INVALID_ARG, "batch too large");
        e = launch_gemm_mfma64(w, xq, y, K, N, M, s, algo == JJO_ALGO_MFMA32 ? 32 : 64);
        if (e != hipSuccess) return hip_fail(e, "gemm_q4_0_q8_1_mfma64 launch");
    } else if (algo == JJO_ALGO_MFMA_W32) {
        if ((M + 127) / 128 > 65535) return set_error(JJO_ERR_INVALID_ARG, "batch too large");
        e = launch_gemm_q4s_mfma(w, xq, y, K, N, M, false, s);
        if (e != hipSuccess) return hip_fail(e, "gemm_q4s_mfma launch");
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

// Diagnostic: a plain coalesced read of `n16` 16-byte units, one per thread, as
// nontemporal loads, folded into one word (written only if it hits a sentinel, so
// the loads cannot be dropped).  The single-launch HBM read floor the GEMV is
// measured against.  Of the read forms timed on this GPU for the GEMV's 25.4 MB
// (1, 2, 4, 8 or 16 loads per thread, plain or nontemporal, persistent grids of
// 256..4096 workgroups), this one is the fastest.
__global__ __launch_bounds__(256) void read_floor_kernel(const uint4 *__restrict__ p, int64_t n16,
                                                         uint32_t *__restrict__ out) {
    typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const u32x4n v = __builtin_nontemporal_load(reinterpret_cast<const u32x4n *>(p + (j < n16 ? j : n16 - 1)));
    const uint32_t acc = v.x ^ v.y ^ v.z ^ v.w;
    if (acc == 0x9e3779b9u) out[0] = acc;
}

}  // namespace

int device_cu_count() { return device_cus(); }

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

int q4_0_to_split_device(const void *d_w_q4_0, void *d_w_split, int nrows, int ncols_k, void *stream) {
    clear_error();
    if (d_w_q4_0 == nullptr || d_w_split == nullptr || d_w_q4_0 == d_w_split)
        return set_error(JJO_ERR_INVALID_ARG, "q4_0_to_split_device: null or aliased buffers");
    if (nrows <= 0 || ncols_k <= 0 || ncols_k % kQK != 0)
        return set_error(JJO_ERR_INVALID_ARG, "q4_0_to_split_device: nrows=%d ncols_k=%d (ncols_k %% 32 == 0)", nrows,
                         ncols_k);
    if (!aligned(d_w_q4_0, 2) || !aligned(d_w_split, 16))
        return set_error(JJO_ERR_INVALID_ARG, "q4_0_to_split_device: source 2-byte, destination 16-byte aligned");
    const int64_t n = (int64_t)nrows * (ncols_k / kQK);
    if ((n + 255) / 256 > 0x7fffffffLL) return set_error(JJO_ERR_INVALID_ARG, "q4_0_to_split_device: too large");
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    hipError_t e = launch_q4_0_to_split(d_w_q4_0, d_w_split, n, (hipStream_t)stream);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "q4_0_to_split launch");
}

namespace {
// Split-layout matmul from Q8_1 blocks (shapes validated by the caller).
int run_mm_split(const void *w, const void *xq, float *y, int K, int N, int M, hipStream_t s) {
    const bool gemv_ok = M <= kGemvMaxBatch && K <= kGemvMaxK && (int64_t)M * (K / kQK) * 48 <= 150 * 1024;
    // The block_q4_0 AUTO dispatch's choices, each kernel reading the split layout: the
    // GEMV up to batch 4 (one K slice) or 2, the LDS-resident skinny kernel for 5..16 at
    // K <= 4096, the per-wave skinny kernel up to 32, then the small-tile GEMM while the
    // 128 x 128 tiles would not fill the chip well, else the 128 x 128 GEMM.
    hipError_t e;
    if (gemv_ok && M <= (K <= 4096 ? kGemvPreferredBatch : 2)) {
        e = launch_gemv_q4s(w, xq, y, K, N, M, s);
        return e == hipSuccess ? JJO_OK : hip_fail(e, "gemv_q4s launch");
    }
    if (K <= 4096 && M >= 5 && M <= 16 && gemm_skinny_persist_supported(w, xq, K, M)) {
        e = launch_gemm_skinny_persist_layout(w, xq, y, K, N, M, true, s);
        return e == hipSuccess ? JJO_OK : hip_fail(e, "gemm_skinny_persist (split layout) launch");
    }
    if (gemm_skinny_supported(w, xq, K, M)) {
        e = launch_gemm_skinny_layout(w, xq, y, K, N, M, true, s);
        return e == hipSuccess ? JJO_OK : hip_fail(e, "gemm_skinny (split layout) launch");
    }
    if (gemv_ok) {
        e = launch_gemv_q4s(w, xq, y, K, N, M, s);
        return e == hipSuccess ? JJO_OK : hip_fail(e, "gemv_q4s launch");
    }
    // K=14336, N=4096, M=48 on the 128 x 128 split GEMM: 126 us (32 workgroups).
    if (const int tr = small_tile_rows(N, M); tr != 0) {
        e = launch_gemm_mfma64(w, xq, y, K, N, M, s, tr, true);
        return e == hipSuccess ? JJO_OK : hip_fail(e, "gemm_mfma64 (split layout) launch");
    }
    e = launch_gemm_q4s_mfma(w, xq, y, K, N, M, true, s);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "gemm_q4s_mfma launch");
}

int validate_split(const void *w, const void *xq, const void *y, int K, int N, int M) {
    int rc = validate_mm(w, xq, y, K, N, M);
    if (rc != JJO_OK) return rc;
    if (!aligned(w, 16)) return set_error(JJO_ERR_INVALID_ARG, "split-layout weight pointer must be 16-byte aligned");
    return JJO_OK;
}
}  // namespace

int mat_mul_q4_0s_q8_1_device(const void *d_w_split, const void *d_x_q8_1, float *d_y, int ncols_k, int nrows_out,
                              int batch, void *stream) {
    clear_error();
    int rc = validate_split(d_w_split, d_x_q8_1, d_y, ncols_k, nrows_out, batch);
    if (rc != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    return run_mm_split(d_w_split, d_x_q8_1, d_y, ncols_k, nrows_out, batch, (hipStream_t)stream);
}

int mat_mul_q4_0s_q8_1_f32_device(const void *d_w_split, const float *d_x, void *d_quant_workspace, float *d_y,
                                  int ncols_k, int nrows_out, int batch, void *stream) {
    clear_error();
    const void *xq_check = d_quant_workspace != nullptr ? d_quant_workspace : (const void *)d_x;
    int rc = validate_split(d_w_split, xq_check, d_y, ncols_k, nrows_out, batch);
    if (rc != JJO_OK) return rc;
    if (d_x == nullptr || !aligned(d_x, 16))
        return set_error(JJO_ERR_INVALID_ARG, "activation pointer must be non-null and 16-byte aligned");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (batch == 1 && ncols_k <= kGemvMaxK) {
        hipError_t e = launch_gemv_q4s_fused(d_w_split, d_x, d_quant_workspace, d_y, ncols_k, nrows_out, s);
        return e == hipSuccess ? JJO_OK : hip_fail(e, "fused quantize+GEMV (split layout) launch");
    }
    if (d_quant_workspace == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "quant workspace is required when batch > 1");
    hipError_t e = launch_quantize_q8_1(d_x, d_quant_workspace, ncols_k, batch, 1, s);
    if (e != hipSuccess) return hip_fail(e, "quantize_q8_1 launch");
    return run_mm_split(d_w_split, d_quant_workspace, d_y, ncols_k, nrows_out, batch, s);
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

int jjo_read_floor_device(const void *d_src, int64_t bytes, uint32_t *d_out, void *stream) {
    clear_error();
    if (d_src == nullptr || d_out == nullptr || bytes < 16 || bytes % 16 != 0 || !aligned(d_src, 16))
        return set_error(JJO_ERR_INVALID_ARG, "read_floor: 16-byte aligned source, bytes a positive multiple of 16");
    const int64_t n16 = bytes / 16, blocks = (n16 + 255) / 256;
    if (blocks > 0x7fffffffLL) return set_error(JJO_ERR_INVALID_ARG, "read_floor: too many bytes");
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    hipLaunchKernelGGL(read_floor_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)d_src, n16, d_out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? JJO_OK : hip_fail(e, "read_floor launch");
}

}  // extern "C"

namespace {
// Grouped launches with few routes (decode batches) run as routed GEMVs over the
// active experts: the 128-route MFMA tiles would leave most of the GPU idle.
#ifndef JJO_GROUPED_GEMV_ROUTES
#define JJO_GROUPED_GEMV_ROUTES 48
#endif
constexpr int kGroupedGemvRoutes = JJO_GROUPED_GEMV_ROUTES;
bool grouped_gemv(int n_routes, int K) { return n_routes <= kGroupedGemvRoutes && K <= kGemvMaxK; }
// Routes per active expert expected: the chunk size of the routed GEMV.
int mean_routes(int n_routes, int n_experts) {
    const int active = n_experts < n_routes ? n_experts : n_routes;
    return (n_routes + active - 1) / active;
}
}  // namespace

extern "C" {

int mat_mul_q4_0_q8_1_grouped_device(const void *d_w_q4_0, const void *d_x_q8_1,
                                     const int32_t *d_expert_offsets, int n_experts,
                                     const int32_t *d_route_dst, float *d_y, int ncols_k,
                                     int nrows_out, int n_routes, void *stream) {
    clear_error();
    int rc = validate_mm(d_w_q4_0, d_x_q8_1, d_y, ncols_k, nrows_out, n_routes);
    if (rc != JJO_OK) return rc;
    if (d_expert_offsets == nullptr || n_experts <= 0 || n_experts > 4096)
        return set_error(JJO_ERR_INVALID_ARG, "expert_offsets must be non-null and 1 <= n_experts <= 4096");
    if ((rc = check_grouped_grid(n_routes, n_experts)) != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e = grouped_gemv(n_routes, ncols_k)
                       ? launch_gemv_routed(d_w_q4_0, nullptr, d_x_q8_1, d_expert_offsets, n_experts, n_routes,
                                            mean_routes(n_routes, n_experts), d_y, nrows_out, ncols_k, nrows_out,
                                            false, (hipStream_t)stream, d_route_dst)
                       : launch_gemm_mfma_grouped(d_w_q4_0, d_x_q8_1, d_expert_offsets, n_experts, d_route_dst,
                                                  d_y, ncols_k, nrows_out, n_routes, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "grouped gemm launch");
    return JJO_OK;
}

int mat_mul_q4_0s_q8_1_grouped_device(const void *d_w_split, const void *d_x_q8_1,
                                      const int32_t *d_expert_offsets, int n_experts,
                                      const int32_t *d_route_dst, float *d_y, int ncols_k,
                                      int nrows_out, int n_routes, void *stream) {
    clear_error();
    int rc = validate_split(d_w_split, d_x_q8_1, d_y, ncols_k, nrows_out, n_routes);
    if (rc != JJO_OK) return rc;
    if (d_expert_offsets == nullptr || n_experts <= 0 || n_experts > 4096)
        return set_error(JJO_ERR_INVALID_ARG, "expert_offsets must be non-null and 1 <= n_experts <= 4096");
    if ((rc = check_grouped_grid(n_routes, n_experts)) != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e = grouped_gemv(n_routes, ncols_k)
                       ? launch_gemv_routed(d_w_split, nullptr, d_x_q8_1, d_expert_offsets, n_experts, n_routes,
                                            mean_routes(n_routes, n_experts), d_y, nrows_out, ncols_k, nrows_out,
                                            true, (hipStream_t)stream, d_route_dst)
                       : launch_gemm_mfma_grouped(d_w_split, d_x_q8_1, d_expert_offsets, n_experts, d_route_dst,
                                                  d_y, ncols_k, nrows_out, n_routes, (hipStream_t)stream, nullptr,
                                                  0, true);
    if (e != hipSuccess) return hip_fail(e, "grouped gemm (split layout) launch");
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

// ---------------------------------------------------------------- Q4_0 weights
int quantize_q4_0_device(void *stream, const float *d_w, void *d_out, int64_t rows, int64_t cols) {
    clear_error();
    if (d_w == nullptr || d_out == nullptr) return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    if (q4_0_bytes(rows, cols) < 0)
        return set_error(JJO_ERR_INVALID_ARG, "rows (%lld) and cols (%lld) must be positive, cols a multiple of 32",
                         (long long)rows, (long long)cols);
    if (!aligned(d_w, 16)) return set_error(JJO_ERR_INVALID_ARG, "weight pointer must be 16-byte aligned");
    if (rows * (cols / JJO_QK4_0) > (int64_t)0x7fffffff * 64)
        return set_error(JJO_ERR_INVALID_ARG, "matrix too large for one launch (%lld blocks)",
                         (long long)(rows * (cols / JJO_QK4_0)));
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    hipError_t e = launch_quantize_q4_0(d_w, d_out, rows * (cols / JJO_QK4_0), (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quantize_q4_0 launch");
    return JJO_OK;
}

// ---------------------------------------------------------------- engine linear
int64_t linear_q4_0_workspace_bytes(int in_features, int num_tokens) {
    if (in_features <= 0 || num_tokens <= 0 || in_features % kQSuper != 0) return -1;
    return (int64_t)num_tokens * (in_features / kQSuper) * kQ8BlockBytes;
}

int linear_q4_0_forward_device(void *stream, void *quant_workspace, const float *input,
                               const void *weight_q4_0, float *output, int in_features,
                               int out_features, int num_tokens) {
    clear_error();
    if (in_features <= 0 || out_features <= 0 || num_tokens <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0: invalid in_features=%d out_features=%d num_tokens=%d",
                         in_features, out_features, num_tokens);
    if (input == nullptr || weight_q4_0 == nullptr || output == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0: null pointer argument");
    return mat_mul_q4_0_q8_1_f32_device(weight_q4_0, input, quant_workspace, output, in_features, out_features,
                                        num_tokens, stream);
}

int linear_q4_0s_forward_device(void *stream, void *quant_workspace, const float *input, const void *weight_split,
                                float *output, int in_features, int out_features, int num_tokens) {
    clear_error();
    if (in_features <= 0 || out_features <= 0 || num_tokens <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0s: invalid in_features=%d out_features=%d num_tokens=%d",
                         in_features, out_features, num_tokens);
    if (input == nullptr || weight_split == nullptr || output == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0s: null pointer argument");
    return mat_mul_q4_0s_q8_1_f32_device(weight_split, input, quant_workspace, output, in_features, out_features,
                                         num_tokens, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free engine linear
// Scratch of linear_q4_0_forward_device_noalloc: the Q8_1 activation of a batch
// (num_tokens * in_features/128 * 144 bytes) lives here instead of in a caller's
// workspace.  Each device holds its own copy for the life of the process.  In host
// code `scratch` is only a symbol handle: the device address comes from
// hipGetSymbolAddress, once per device, and only that address is handed to
// kernels.
constexpr int64_t kNoAllocScratchBytes = 16ll << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void *> g_scratch_ptr;  // per device; nullptr until resolved

// Device address of the current device's scratch, resolved on the first call there.
int scratch_address(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(JJO_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        // The first call may come while the caller's stream is being captured into a
        // graph: the lookup enqueues nothing, so this thread's capture mode is
        // relaxed around it (a global-mode capture would otherwise reject the call).
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return hip_fail(e, "hipThreadExchangeStreamCaptureMode");
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (e2 != hipSuccess) return hip_fail(e2, "hipThreadExchangeStreamCaptureMode");
        if (p == nullptr) return set_error(JJO_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return JJO_OK;
}
}  // namespace

extern "C" {

int64_t linear_q4_0_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

int linear_q4_0_forward_device_noalloc(void *stream, const float *input, const void *weight_q4_0, float *output,
                                       int in_features, int out_features, int num_tokens) {
    clear_error();
    if (in_features <= 0 || out_features <= 0 || num_tokens <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0_noalloc: invalid in_features=%d out_features=%d num_tokens=%d",
                         in_features, out_features, num_tokens);
    if (input == nullptr || weight_q4_0 == nullptr || output == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0_noalloc: null pointer argument");
    const int64_t need = linear_q4_0_workspace_bytes(in_features, num_tokens);
    if (need < 0)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0_noalloc: in_features=%d must be a multiple of %d",
                         in_features, kQSuper);
    if (need > kNoAllocScratchBytes)
        return set_error(JJO_ERR_INVALID_ARG,
                         "linear_q4_0_noalloc: num_tokens=%d x in_features=%d needs %lld bytes of Q8_1 scratch, more "
                         "than the %lld-byte static buffer; use linear_q4_0_forward_device with a workspace",
                         num_tokens, in_features, (long long)need, (long long)kNoAllocScratchBytes);
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    // A one-token step with in_features <= kGemvMaxK quantizes inside its GEMV and
    // needs no scratch; every other call (a batch, or one token over a longer row)
    // quantizes into the static buffer first.
    void *ws = nullptr;
    if ((num_tokens > 1 || in_features > kGemvMaxK) && (rc = scratch_address(&ws)) != JJO_OK) return rc;
    return mat_mul_q4_0_q8_1_f32_device(weight_q4_0, input, ws, output, in_features, out_features, num_tokens,
                                        stream);
}

int linear_q4_0_forward_host(float *input, const void *weight_q4_0, float *output, int in_features,
                             int num_tokens, int out_features) {
    clear_error();
    const int64_t ws_bytes = linear_q4_0_workspace_bytes(in_features, num_tokens);
    if (ws_bytes < 0 || out_features <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0: invalid in_features=%d out_features=%d num_tokens=%d",
                         in_features, out_features, num_tokens);
    if (input == nullptr || weight_q4_0 == nullptr || output == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "linear_q4_0: null pointer argument");
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    const int64_t n_in = (int64_t)in_features * num_tokens;
    const int64_t w_bytes = (int64_t)out_features * (in_features / kQK) * kQ4BlockBytes;
    const int64_t y_elems = (int64_t)out_features * num_tokens;
    hipStream_t s = nullptr;
    void *dw = nullptr, *dq = nullptr;
    float *dx = nullptr, *dy = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
    do {
        if ((e = hipMalloc((void **)&dx, n_in * sizeof(float))) != hipSuccess) { rc = hip_fail(e, "hipMalloc(x)"); break; }
        if ((e = hipMalloc(&dq, ws_bytes)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(ws)"); break; }
        if ((e = hipMalloc(&dw, w_bytes)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(w)"); break; }
        if ((e = hipMalloc((void **)&dy, y_elems * sizeof(float))) != hipSuccess) { rc = hip_fail(e, "hipMalloc(y)"); break; }
        if ((e = hipMemcpyAsync(dx, input, n_in * sizeof(float), hipMemcpyHostToDevice, s)) != hipSuccess) { rc = hip_fail(e, "H2D x"); break; }
        if ((e = hipMemcpyAsync(dw, weight_q4_0, w_bytes, hipMemcpyHostToDevice, s)) != hipSuccess) { rc = hip_fail(e, "H2D w"); break; }
        if ((rc = linear_q4_0_forward_device(s, dq, dx, dw, dy, in_features, out_features, num_tokens)) != JJO_OK) break;
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

// ---------------------------------------------------------------- MoE FFN (Q4_0 experts)
namespace {
int check_moe_shape(int num_tokens, int hidden, int inter, int num_experts, int top_k) {
    if (num_tokens <= 0 || hidden <= 0 || inter <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "moe: invalid num_tokens=%d hidden=%d intermediate=%d", num_tokens,
                         hidden, inter);
    if (hidden % kQSuper != 0 || inter % kQSuper != 0)
        return set_error(JJO_ERR_INVALID_ARG, "moe: hidden_size and intermediate_size must be multiples of %d",
                         kQSuper);
    if (num_experts <= 0 || num_experts > 1024 || top_k <= 0 || top_k > 32 || top_k > num_experts)
        return set_error(JJO_ERR_INVALID_ARG, "moe: need 1 <= top_k <= min(32, num_experts), num_experts <= 1024 "
                         "(got top_k=%d num_experts=%d)", top_k, num_experts);
    if ((int64_t)num_tokens * top_k > 0x7fffffffLL / 4)
        return set_error(JJO_ERR_INVALID_ARG, "moe: too many routes");
    if (num_tokens > 65535 || ((int64_t)num_tokens * top_k + 127) / 128 + num_experts > 65535)
        return set_error(JJO_ERR_INVALID_ARG, "moe: num_tokens=%d with top_k=%d exceeds one launch's grid",
                         num_tokens, top_k);
    return JJO_OK;
}

struct MoeWs {
    float *route_w;
    int32_t *ids, *offsets, *src_route, *dst_of_route;
    uint8_t *xq, *xp, *midq;
    float *eout;
    float *gate_up;  // [R][2I] fp32, decode path only
    int64_t bytes;
};

// Token counts up to which the FFN runs its expert matrices as routed GEMVs (every
// weight byte of an active expert read once, its routes taken in chunks) instead of
// 128-route MFMA tiles, which leave most of the GPU idle when each expert holds a
// handful of routes.  Measured against the MFMA path on 8, 64 and 256 experts (top-2,
// top-8, top-8): the GEMVs win up to 16 tokens on all three and lose from 24-32 on.
#ifndef JJO_MOE_GEMV_TOKENS
#define JJO_MOE_GEMV_TOKENS 16
#endif
// Also routed at any token count while an active expert averages at most this many
// routes (many experts, e.g. 256 experts top-8 at 32-64 tokens: 1241 -> 1068 us at 32).
#ifndef JJO_MOE_ROUTED_MEAN
#define JJO_MOE_ROUTED_MEAN 2
#endif
bool moe_decode_path(int T, int H, int I, int E, int top_k) {
    const int R = T * top_k, active = E < R ? E : R;
    const bool sparse = (R + active - 1) / active <= JJO_MOE_ROUTED_MEAN;
    return (T <= JJO_MOE_GEMV_TOKENS || sparse) && H <= 16384 && I <= 16384;
}

// Workspace carve-up, every part 256-byte aligned.
MoeWs moe_ws_layout(uint8_t *base, int T, int H, int I, int E, int top_k) {
    const int64_t R = (int64_t)T * top_k;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        uint8_t *p = base ? base + off : nullptr;
        off += (bytes + 255) / 256 * 256;
        return p;
    };
    MoeWs w{};
    w.route_w = (float *)take(R * 4);
    w.ids = (int32_t *)take(R * 4);
    w.offsets = (int32_t *)take((int64_t)(E + 1) * 4);
    w.src_route = (int32_t *)take(R * 4);
    w.dst_of_route = (int32_t *)take(R * 4);
    w.xq = take((int64_t)T * (H / kQSuper) * kQ8BlockBytes);
    w.xp = take(R * (H / kQSuper) * kQ8BlockBytes);
    w.midq = take(R * (I / kQSuper) * kQ8BlockBytes);
    w.eout = (float *)take(R * H * 4);
    w.gate_up = moe_decode_path(T, H, I, E, top_k) ? (float *)take(R * 2 * I * 4) : nullptr;
    w.bytes = off;
    return w;
}
}  // namespace

int moe_top_k_device(void *stream, const float *logits, float *route_weights, int32_t *expert_ids,
                     int num_tokens, int num_experts, int top_k) {
    clear_error();
    int rc = check_moe_shape(num_tokens, kQSuper, kQSuper, num_experts, top_k);
    if (rc != JJO_OK) return rc;
    if (logits == nullptr || route_weights == nullptr || expert_ids == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "moe_top_k: null pointer argument");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e = launch_moe_top_k(logits, route_weights, expert_ids, num_tokens, num_experts, top_k,
                                    (hipStream_t)stream);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "moe_top_k launch");
}

int moe_dispatch_q8_1_device(void *stream, const int32_t *expert_ids, const void *x_q8_1, int num_tokens,
                             int top_k, int hidden_size, int num_experts, int32_t *expert_offsets,
                             int32_t *src_route, int32_t *dst_of_route, void *x_q8_1_permuted) {
    clear_error();
    int rc = check_moe_shape(num_tokens, hidden_size, kQSuper, num_experts, top_k);
    if (rc != JJO_OK) return rc;
    if (expert_ids == nullptr || expert_offsets == nullptr || src_route == nullptr || dst_of_route == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "moe_dispatch: null pointer argument");
    if ((x_q8_1 == nullptr) != (x_q8_1_permuted == nullptr))
        return set_error(JJO_ERR_INVALID_ARG, "moe_dispatch: give both Q8_1 buffers or neither");
    if (x_q8_1 != nullptr && (!aligned(x_q8_1, 16) || !aligned(x_q8_1_permuted, 16)))
        return set_error(JJO_ERR_INVALID_ARG, "moe_dispatch: Q8_1 buffers must be 16-byte aligned");
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipStream_t s = (hipStream_t)stream;
    const int R = num_tokens * top_k;
    hipError_t e = launch_moe_dispatch(expert_ids, R, num_experts, expert_offsets, src_route, dst_of_route, s);
    if (e != hipSuccess) return hip_fail(e, "moe_dispatch launch");
    if (x_q8_1 != nullptr) {
        e = launch_moe_gather_q8_1(x_q8_1, src_route, x_q8_1_permuted, num_tokens, R, top_k, hidden_size, s);
        if (e != hipSuccess) return hip_fail(e, "moe_gather_q8_1 launch");
    }
    return JJO_OK;
}

int swiglu_quantize_q8_1_device(void *stream, const float *gate_up, void *mid_q8_1, float *mid_f32,
                                int rows, int intermediate_size) {
    clear_error();
    if (rows <= 0 || intermediate_size <= 0 || intermediate_size % kQSuper != 0)
        return set_error(JJO_ERR_INVALID_ARG, "swiglu_quantize: rows > 0 and intermediate_size %% %d == 0 required",
                         kQSuper);
    if (gate_up == nullptr || mid_q8_1 == nullptr || !aligned(gate_up, 16) || !aligned(mid_q8_1, 16) ||
        (mid_f32 != nullptr && !aligned(mid_f32, 16)))
        return set_error(JJO_ERR_INVALID_ARG, "swiglu_quantize: non-null 16-byte aligned buffers required");
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    hipError_t e = launch_swiglu_quantize_q8_1(gate_up, mid_q8_1, mid_f32, intermediate_size, rows,
                                               (hipStream_t)stream);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "swiglu_quantize launch");
}

int moe_q4_0_gate_up_device(void *stream, const void *w_gate, const void *w_up, const void *x_q8_1_permuted,
                            const int32_t *expert_offsets, int num_experts, float *gate_up, int hidden_size,
                            int intermediate_size, int n_routes) {
    clear_error();
    int rc = validate_mm(w_gate, x_q8_1_permuted, gate_up, hidden_size, 2 * intermediate_size, n_routes);
    if (rc != JJO_OK) return rc;
    if (w_up == nullptr || !aligned(w_up, 4) || expert_offsets == nullptr || num_experts <= 0 ||
        num_experts > 4096)
        return set_error(JJO_ERR_INVALID_ARG, "moe_gate_up: bad w_up / expert_offsets / num_experts");
    if (intermediate_size % 128 != 0)
        return set_error(JJO_ERR_INVALID_ARG, "moe_gate_up: intermediate_size must be a multiple of 128");
    if ((rc = check_grouped_grid(n_routes, num_experts)) != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e =
        grouped_gemv(n_routes, hidden_size)
            ? launch_gemv_routed(w_gate, w_up, x_q8_1_permuted, expert_offsets, num_experts, n_routes,
                                 mean_routes(n_routes, num_experts), gate_up, 2 * intermediate_size, hidden_size,
                                 intermediate_size, false, (hipStream_t)stream)
            : launch_gemm_mfma_grouped(w_gate, x_q8_1_permuted, expert_offsets, num_experts, nullptr, gate_up,
                                       hidden_size, 2 * intermediate_size, n_routes, (hipStream_t)stream, w_up,
                                       intermediate_size);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "moe_gate_up launch");
}

int moe_q4_0_gate_up_swiglu_q8_1_device(void *stream, const void *w_gate, const void *w_up,
                                        const void *x_q8_1_permuted, const int32_t *expert_offsets, int num_experts,
                                        void *mid_q8_1, int hidden_size, int intermediate_size, int n_routes) {
    clear_error();
    int rc = validate_mm(w_gate, x_q8_1_permuted, mid_q8_1, hidden_size, 2 * intermediate_size, n_routes);
    if (rc != JJO_OK) return rc;
    if (w_up == nullptr || !aligned(w_up, 4) || expert_offsets == nullptr || num_experts <= 0 ||
        num_experts > 4096)
        return set_error(JJO_ERR_INVALID_ARG, "moe_gate_up_swiglu: bad w_up / expert_offsets / num_experts");
    if (intermediate_size % 128 != 0)
        return set_error(JJO_ERR_INVALID_ARG, "moe_gate_up_swiglu: intermediate_size must be a multiple of 128");
    if ((rc = check_grouped_grid(n_routes, num_experts)) != JJO_OK) return rc;
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipError_t e = launch_gemm_gate_up_swiglu_q8_1(w_gate, w_up, x_q8_1_permuted, expert_offsets, num_experts,
                                                   mid_q8_1, hidden_size, intermediate_size, n_routes,
                                                   (hipStream_t)stream);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "moe_gate_up_swiglu launch");
}

int moe_combine_device(void *stream, const float *expert_out, const int32_t *dst_of_route,
                       const float *route_weights, float *y, int num_tokens, int hidden_size, int top_k) {
    clear_error();
    if (num_tokens <= 0 || num_tokens > 65535 || hidden_size <= 0 || hidden_size % 4 != 0 || top_k <= 0)
        return set_error(JJO_ERR_INVALID_ARG, "moe_combine: 0 < num_tokens <= 65535, top_k > 0 and hidden_size %% 4 == 0");
    if (expert_out == nullptr || dst_of_route == nullptr || route_weights == nullptr || y == nullptr ||
        !aligned(expert_out, 16) || !aligned(y, 16))
        return set_error(JJO_ERR_INVALID_ARG, "moe_combine: non-null buffers, 16-byte aligned expert_out and y");
    int rc = require_gfx950();
    if (rc != JJO_OK) return rc;
    hipError_t e = launch_moe_combine(expert_out, dst_of_route, route_weights, y, num_tokens, hidden_size, top_k,
                                      (hipStream_t)stream);
    return e == hipSuccess ? JJO_OK : hip_fail(e, "moe_combine launch");
}

int64_t moe_q4_0_ffn_workspace_bytes(int num_tokens, int hidden_size, int intermediate_size, int num_experts,
                                     int top_k) {
    if (check_moe_shape(num_tokens, hidden_size, intermediate_size, num_experts, top_k) != JJO_OK) return -1;
    return moe_ws_layout(nullptr, num_tokens, hidden_size, intermediate_size, num_experts, top_k).bytes;
}

}  // extern "C"

namespace {
// The Q4_0 MoE FFN; split: the three expert weight buffers are in the split layout.
int moe_ffn_run(bool split, void *stream, const float *x, const float *logits, const void *w_gate, const void *w_up,
                const void *w_down, float *y, int num_tokens, int hidden_size, int intermediate_size, int num_experts,
                int top_k, void *workspace, int64_t workspace_bytes) {
    clear_error();
    const int T = num_tokens, H = hidden_size, I = intermediate_size, E = num_experts;
    int rc = check_moe_shape(T, H, I, E, top_k);
    if (rc != JJO_OK) return rc;
    if (x == nullptr || logits == nullptr || w_gate == nullptr || w_up == nullptr || w_down == nullptr ||
        y == nullptr || workspace == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "moe_ffn: null pointer argument");
    const int wal = split ? 16 : 4;
    if (!aligned(x, 16) || !aligned(y, 16) || !aligned(workspace, 256) || !aligned(w_gate, wal) ||
        !aligned(w_up, wal) || !aligned(w_down, wal))
        return set_error(JJO_ERR_INVALID_ARG, "moe_ffn: x, y 16-byte, workspace 256-byte, weights %d-byte aligned",
                         wal);
    const MoeWs ws = moe_ws_layout((uint8_t *)workspace, T, H, I, E, top_k);
    if (workspace_bytes < ws.bytes)
        return set_error(JJO_ERR_INVALID_ARG, "moe_ffn: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                         (long long)ws.bytes);
    if ((rc = require_gfx950()) != JJO_OK) return rc;
    hipStream_t s = (hipStream_t)stream;
    const int R = T * top_k;
    hipError_t e;
    if (moe_decode_path(T, H, I, E, top_k)) {
        // Chunk size of the routed GEMVs: the mean routes per active expert (an expert
        // with more takes several chunks with its weights held in registers).
        // 1) quantize + top-k + dispatch + gather, 2) gate|up (both matrices, one
        // launch) -> fp32 [R][2I], 3) SwiGLU + Q8_1, 4) down projection, 5) combine
        if (R <= kMoeDecodeRoutes) {
            if ((e = launch_moe_route_decode(x, logits, T, H, E, top_k, ws.route_w, ws.ids, ws.offsets,
                                             ws.src_route, ws.dst_of_route, ws.xp, s)) != hipSuccess)
                return hip_fail(e, "moe_ffn routing");
        } else {  // more routes (top_k > 24) than the one-launch routing holds: four launches
            if ((e = launch_quantize_q8_1(x, ws.xq, H, T, 1, s)) != hipSuccess) return hip_fail(e, "moe_ffn quantize x");
            if ((e = launch_moe_top_k(logits, ws.route_w, ws.ids, T, E, top_k, s)) != hipSuccess)
                return hip_fail(e, "moe_ffn top_k");
            if ((e = launch_moe_dispatch(ws.ids, R, E, ws.offsets, ws.src_route, ws.dst_of_route, s)) != hipSuccess)
                return hip_fail(e, "moe_ffn dispatch");
            if ((e = launch_moe_gather_q8_1(ws.xq, ws.src_route, ws.xp, T, R, top_k, H, s)) != hipSuccess)
                return hip_fail(e, "moe_ffn gather");
        }
        const int per_expert = mean_routes(R, E);
        if ((e = launch_gemv_routed(w_gate, w_up, ws.xp, ws.offsets, E, R, per_expert, ws.gate_up, 2 * I, H, I,
                                    split, s)) != hipSuccess)
            return hip_fail(e, "moe_ffn gate_up (routed GEMV)");
        if ((e = launch_swiglu_quantize_q8_1(ws.gate_up, ws.midq, nullptr, I, R, s)) != hipSuccess)
            return hip_fail(e, "moe_ffn swiglu");
        if ((e = launch_gemv_routed(w_down, nullptr, ws.midq, ws.offsets, E, R, per_expert, ws.eout, H, I, H, split,
                                    s)) != hipSuccess)
            return hip_fail(e, "moe_ffn down (routed GEMV)");
        if ((e = launch_moe_combine(ws.eout, ws.dst_of_route, ws.route_w, y, T, H, top_k, s)) != hipSuccess)
            return hip_fail(e, "moe_ffn combine");
        return JJO_OK;
    }
    // 1) x -> Q8_1 (once per token), 2) top-k gating, 3) stable dispatch + Q8_1 row gather
    if ((e = launch_quantize_q8_1(x, ws.xq, H, T, 1, s)) != hipSuccess) return hip_fail(e, "moe_ffn quantize x");
    if ((e = launch_moe_top_k(logits, ws.route_w, ws.ids, T, E, top_k, s)) != hipSuccess)
        return hip_fail(e, "moe_ffn top_k");
    if ((e = launch_moe_dispatch(ws.ids, R, E, ws.offsets, ws.src_route, ws.dst_of_route, s)) != hipSuccess)
        return hip_fail(e, "moe_ffn dispatch");
    if ((e = launch_moe_gather_q8_1(ws.xq, ws.src_route, ws.xp, T, R, top_k, H, s)) != hipSuccess)
        return hip_fail(e, "moe_ffn gather");
    // 4) gate|up of every route's expert in one grouped launch whose epilogue applies
    //    SwiGLU and writes the Q8_1 input of the down projection (no fp32 gate|up)
    if ((e = launch_gemm_gate_up_swiglu_q8_1(w_gate, w_up, ws.xp, ws.offsets, E, ws.midq, H, I, R, s, split)) !=
        hipSuccess)
        return hip_fail(e, "moe_ffn gate_up_swiglu");
    // 5) down projection, 6) weighted combine back to token order
    if ((e = launch_gemm_mfma_grouped(w_down, ws.midq, ws.offsets, E, nullptr, ws.eout, I, H, R, s, nullptr, 0,
                                      split)) != hipSuccess)
        return hip_fail(e, "moe_ffn down");
    if ((e = launch_moe_combine(ws.eout, ws.dst_of_route, ws.route_w, y, T, H, top_k, s)) != hipSuccess)
        return hip_fail(e, "moe_ffn combine");
    return JJO_OK;
}
}  // namespace

extern "C" {

int moe_q4_0_ffn_forward_device(void *stream, const float *x, const float *logits, const void *w_gate,
                                const void *w_up, const void *w_down, float *y, int num_tokens, int hidden_size,
                                int intermediate_size, int num_experts, int top_k, void *workspace,
                                int64_t workspace_bytes) {
    return moe_ffn_run(false, stream, x, logits, w_gate, w_up, w_down, y, num_tokens, hidden_size,
                       intermediate_size, num_experts, top_k, workspace, workspace_bytes);
}

int moe_q4_0s_ffn_forward_device(void *stream, const float *x, const float *logits, const void *w_gate_split,
                                 const void *w_up_split, const void *w_down_split, float *y, int num_tokens,
                                 int hidden_size, int intermediate_size, int num_experts, int top_k, void *workspace,
                                 int64_t workspace_bytes) {
    return moe_ffn_run(true, stream, x, logits, w_gate_split, w_up_split, w_down_split, y, num_tokens, hidden_size,
                       intermediate_size, num_experts, top_k, workspace, workspace_bytes);
}

}  // extern "C"
