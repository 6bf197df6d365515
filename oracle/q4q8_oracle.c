/*
 * q4q8_oracle.c — TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the reference's Q8_1 quantizer and Q4_0 x Q8_1 matmul
 * (AshburnLee/JJJetson_Ops).  This file is the checker that the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP path
 * against.  Nothing in the product library links or calls it.
 *
 * Build (no fast-math, no FP contraction, IEEE fp32):
 *   gcc -O2 -fPIC -shared -ffp-contract=off -fno-fast-math q4q8_oracle.c -o liboracle_q4q8.so -lm
 *
 * Pinning status of each function (how the tests check it is stated in
 * tests/test_oracle.py):
 *   oracle_f32_to_f16 / oracle_f16_to_f32 : pinned (numpy float16 casts on
 *       every fp16 bit pattern / a sweep of fp32 values).
 *   oracle_quantize_q8_1      : pinned (known answers: ties, zero groups,
 *       summation-order witnesses; the reference test's own q8_1_ref check at
 *       its tolerances; exact-rational check of d).
 *   oracle_block_sums         : pinned (brute-force integer dot on tiny inputs,
 *       closed forms for constant nibbles).
 *   oracle_matmul_f64/_f32    : pinned (textbook dot at K=32, closed forms,
 *       dequantized fp64 W.x).
 *   oracle_quantize_q4_0      : data generator of this build, not part of the
 *       reference; checked for the round-trip bound |w - deq(w)| <= d/2.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- fp16 helpers (IEEE binary16, round-to-nearest-even) ---------------- */

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) { /* inf or nan */
        if (absx > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((absx >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
    if (absx < 0x38800000u) {                                     /* result subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign;            /* < 2^-25: rounds to 0 */
        /* value = mant * 2^(e-150); result unit is 2^-24, so q = mant >> (126-e) */
        uint32_t e = absx >> 23;
        uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
        uint32_t rshift = 126u - e; /* 14..24 */
        uint32_t q = mant >> rshift;
        uint32_t rem = mant & ((1u << rshift) - 1u);
        uint32_t half = 1u << (rshift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal */
    uint32_t e16 = ((absx >> 23) - 112u);
    uint32_t mant = absx & 0x7fffffu;
    uint32_t q = (e16 << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carry may bump exponent: fine */
    return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---- Q8_1 quantizer ------------------------------------------------------
 * Follows quantize_q8_1_kernel, src/cuda/q8_1.cu:40-103:
 *   lanes t=0..7 of a 32-group hold x[4t..4t+3]                       (:40,52)
 *   amax: per-lane fmaxf chain, then xor-shuffle 4,2,1 with fmaxf       (:55-60)
 *   sum : per-lane ((x0+x1)+x2)+x3, then xor-shuffle 4,2,1 additions     (:62-68)
 *   d_inv = amax > 0 ? 127/amax : 0 ; q = roundf(x*d_inv)              (:71-79)
 *   ds4[g] = half2(1/d_inv, sum) (RNE), so a zero group stores d=+inf   (:102)
 *   block index = z*(ne1*gridDim.y*4) + (k/128)*ne1 + m                 (:84-86)
 * with gridDim.y = ceil(K/512) (src/cuda/q8_1.cu:173).
 * Groups of the last superblock that lie beyond K (K % 128 != 0) are written
 * as zero bytes here (the reference leaves them unwritten).
 * Requires K % 32 == 0.
 */
static void quantize_group(const float *x, int8_t *qs, uint16_t *ds /* [2] */) {
    float lane_max[8], lane_sum[8];
    for (int t = 0; t < 8; ++t) {
        const float *v = x + 4 * t;
        lane_max[t] = fmaxf(fabsf(v[0]), fmaxf(fabsf(v[1]), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        float s = v[0] + v[1];
        s = s + v[2];
        s = s + v[3];
        lane_sum[t] = s;
    }
    for (int off = 4; off > 0; off >>= 1) {
        float nm[8], ns[8];
        for (int t = 0; t < 8; ++t) {
            nm[t] = fmaxf(lane_max[t], lane_max[t ^ off]);
            ns[t] = lane_sum[t] + lane_sum[t ^ off];
        }
        memcpy(lane_max, nm, sizeof nm);
        memcpy(lane_sum, ns, sizeof ns);
    }
    const float amax = lane_max[0];
    const float sum = lane_sum[0];
    const float d_inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
    for (int i = 0; i < 32; ++i) {
        volatile float p = x[i] * d_inv; /* single rounding of the product */
        qs[i] = (int8_t)roundf(p);
    }
    volatile float one_over = 1.0f / d_inv;
    ds[0] = oracle_f32_to_f16(one_over);
    ds[1] = oracle_f32_to_f16(sum);
}

int64_t oracle_q8_1_n_blocks(const int64_t *dims) {
    const int64_t K = dims[0], ne1 = dims[1], nz = dims[2] * dims[3];
    if (nz <= 1) return ne1 * ((K + 127) / 128);
    return nz * ne1 * 4 * ((K + 511) / 512);
}

int oracle_quantize_q8_1(const float *x, uint8_t *out, const int64_t *dims) {
    const int64_t K = dims[0], ne1 = dims[1], ne2 = dims[2], ne3 = dims[3];
    if (K <= 0 || K % 32 != 0 || ne1 <= 0 || ne2 <= 0 || ne3 <= 0) return 1;
    const int64_t nz = ne2 * ne3;
    const int64_t n_super = (K + 127) / 128;
    const int64_t slice_blocks = ne1 * 4 * ((K + 511) / 512);
    memset(out, 0, (size_t)(oracle_q8_1_n_blocks(dims) * 144));
    for (int64_t z = 0; z < nz; ++z) {
        for (int64_t m = 0; m < ne1; ++m) {
            const float *xm = x + (z * ne1 + m) * K;
            for (int64_t sb = 0; sb < n_super; ++sb) {
                uint8_t *blk = out + (z * slice_blocks + sb * ne1 + m) * 144;
                for (int g = 0; g < 4; ++g) {
                    const int64_t k0 = sb * 128 + g * 32;
                    if (k0 >= K) break;
                    uint16_t ds[2];
                    quantize_group(xm + k0, (int8_t *)(blk + 16 + 32 * g), ds);
                    memcpy(blk + 4 * g, &ds[0], 2);
                    memcpy(blk + 4 * g + 2, &ds[1], 2);
                }
            }
        }
    }
    return 0;
}

/* Restates parse_q8_1_output, src/cuda/q8_1.cu:197-216. */
void oracle_parse_q8_1(const uint8_t *in, int8_t *qs, float *scale, float *sum, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = in + b * 144;
        memcpy(qs + b * 128, blk + 16, 128);
        for (int g = 0; g < 4; ++g) {
            uint16_t d, s;
            memcpy(&d, blk + 4 * g, 2);
            memcpy(&s, blk + 4 * g + 2, 2);
            scale[b * 4 + g] = oracle_f16_to_f32(d);
            sum[b * 4 + g] = oracle_f16_to_f32(s);
        }
    }
}

/* ---- Q4_0 x Q8_1 ----------------------------------------------------------
 * Activation block (token m, 32-group b) of the quantizer's layout:
 *   superblock s = b/4 at block index s*M + m, group g = b%4.
 * (The reference kernel itself indexes m*(K/128)+s, src/cuda/mm_q4_0_q8_1.cu:230,246;
 * the two orders agree only for M == 1.  This oracle, like the HIP path, reads the
 * quantizer's order.)
 */
static inline const uint8_t *xblock(const uint8_t *xq, int64_t M, int64_t m, int64_t b) {
    return xq + ((b / 4) * M + m) * 144;
}

/* sumi = sum_{j<32} nib_j * q_j, nibble j = low(qs[j]) for j<16, high(qs[j-16]) else.
 * Restates q4_0_q8_1_vec_dot_impl's integer part, src/cuda/mm_q4_0_q8_1.cu:75-90. */
static inline int32_t block_dot(const uint8_t *wblk, const int8_t *q) {
    int32_t s = 0;
    for (int j = 0; j < 16; ++j) {
        s += (int32_t)(wblk[2 + j] & 0x0f) * (int32_t)q[j];
        s += (int32_t)(wblk[2 + j] >> 4) * (int32_t)q[j + 16];
    }
    return s;
}

int oracle_block_sums(const uint8_t *w, const uint8_t *xq, int32_t *sumi, int64_t K, int64_t N,
                      int64_t M) {
    if (K % 128 != 0) return 1;
    const int64_t nb = K / 32;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t *xb = xblock(xq, M, m, b);
                sumi[(m * N + n) * nb + b] =
                    block_dot(w + (n * nb + b) * 18, (const int8_t *)(xb + 16 + 32 * (b % 4)));
            }
    return 0;
}

/* Per-block term of src/cuda/mm_q4_0_q8_1.cu:91-92:
 *   d_w * (sumi * d_x - 8 * s_x)
 * mode 0: evaluated in fp64, blocks summed in fp64 (the "exact" value).
 * mode 1: fp32 in the reference kernel's order: acc += term sequentially over b
 *         (:256-269), term = d_w * fmaf(sumi, d_x, -8*s_x) (nvcc contracts the
 *         inner expression), then acc = fmaf(d_w, t, acc).
 */
int oracle_matmul(const uint8_t *w, const uint8_t *xq, float *y, int64_t K, int64_t N, int64_t M,
                  int mode) {
    if (K % 128 != 0) return 1;
    const int64_t nb = K / 32;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double acc64 = 0.0;
            float acc32 = 0.0f;
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t *wb = w + (n * nb + b) * 18;
                const uint8_t *xb = xblock(xq, M, m, b);
                const int g = (int)(b % 4);
                uint16_t dwh, dxh, sxh;
                memcpy(&dwh, wb, 2);
                memcpy(&dxh, xb + 4 * g, 2);
                memcpy(&sxh, xb + 4 * g + 2, 2);
                const float dw = oracle_f16_to_f32(dwh);
                const float dx = oracle_f16_to_f32(dxh);
                const float sx = oracle_f16_to_f32(sxh);
                const int32_t s = block_dot(wb, (const int8_t *)(xb + 16 + 32 * g));
                if (mode == 0) {
                    acc64 += (double)dw * ((double)s * (double)dx - 8.0 * (double)sx);
                } else {
                    const float t = fmaf((float)s, dx, -8.0f * sx);
                    acc32 = fmaf(dw, t, acc32);
                }
            }
            y[m * N + n] = (mode == 0) ? (float)acc64 : acc32;
        }
    return 0;
}

/* ---- Q4_0 weight generator (this build's; the reference ships none) ------
 * ggml-style: per 32-block take the element of largest magnitude `mx`,
 * d = mx / -8, id = d != 0 ? 1/d : 0, nib = min(15, (int)(w*id + 8.5)),
 * store fp16(d).  Rows of K/32 blocks, row-major.
 */
int oracle_quantize_q4_0(const float *w, uint8_t *out, int64_t N, int64_t K) {
    if (K % 32 != 0) return 1;
    const int64_t nb = K / 32;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t b = 0; b < nb; ++b) {
            const float *v = w + n * K + b * 32;
            float amax = 0.0f, mx = 0.0f;
            for (int j = 0; j < 32; ++j)
                if (fabsf(v[j]) > amax) {
                    amax = fabsf(v[j]);
                    mx = v[j];
                }
            const float d = mx / -8.0f;
            const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
            uint8_t *blk = out + (n * nb + b) * 18;
            uint16_t dh = oracle_f32_to_f16(d);
            memcpy(blk, &dh, 2);
            for (int j = 0; j < 16; ++j) {
                volatile float a = v[j] * id + 8.5f;
                volatile float c = v[j + 16] * id + 8.5f;
                int lo = (int)a, hi = (int)c;
                if (lo > 15) lo = 15;
                if (hi > 15) hi = 15;
                if (lo < 0) lo = 0;
                if (hi < 0) hi = 0;
                blk[2 + j] = (uint8_t)(lo | (hi << 4));
            }
        }
    return 0;
}
