/* C client of linear_q4_0_forward_host (the engine linear's host-buffer entry):
 * y = W . x for Q4_0 weights quantized with quantize_q4_0_host, compared with the
 * fp64 product of the dequantized weights and the unquantized x (tolerance: the
 * Q8_1 rounding of x).  Exit 0 on success.  Needs a gfx950 GPU. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "jjjetson_ops_amd.h"

#define IN 512
#define OUT 96
#define T 3

static float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15), e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

int main(void) {
    static float w[OUT * IN], x[T * IN], y[T * OUT];
    uint32_t r = 12345u;
    for (int i = 0; i < OUT * IN; ++i) { r = r * 1664525u + 1013904223u; w[i] = ((float)(r >> 8) / 16777216.0f - 0.5f) * 0.04f; }
    for (int i = 0; i < T * IN; ++i) { r = r * 1664525u + 1013904223u; x[i] = (float)(r >> 8) / 16777216.0f - 0.5f; }
    const int64_t qb = q4_0_bytes(OUT, IN);
    uint8_t *q = (uint8_t *)malloc((size_t)qb);
    if (quantize_q4_0_host(w, q, OUT, IN, 0) != JJO_OK) return 3;
    if (linear_q4_0_forward_host(x, q, y, IN, T, OUT) != JJO_OK) {
        fprintf(stderr, "linear: %s\n", jjo_last_error());
        return 4;
    }
    double err = 0.0, ref_norm = 0.0;
    for (int t = 0; t < T; ++t)
        for (int n = 0; n < OUT; ++n) {
            double acc = 0.0;
            for (int b = 0; b < IN / 32; ++b) {
                const uint8_t *blk = q + ((size_t)n * (IN / 32) + b) * 18;
                uint16_t dh;
                memcpy(&dh, blk, 2);
                const double d = half_to_float(dh);
                for (int j = 0; j < 16; ++j) {
                    acc += d * ((blk[2 + j] & 15) - 8) * x[t * IN + b * 32 + j];
                    acc += d * ((blk[2 + j] >> 4) - 8) * x[t * IN + b * 32 + j + 16];
                }
            }
            err += (y[t * OUT + n] - acc) * (y[t * OUT + n] - acc);
            ref_norm += acc * acc;
        }
    const double rel = sqrt(err / ref_norm);
    printf("rel %.3e\n", rel);
    free(q);
    return rel < 2e-2 ? 0 : 5;
}
