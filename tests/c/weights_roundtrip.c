/* C client of the Q4_0 weight entries in include/jjjetson_ops_amd.h, built with
 * plain gcc: quantize a matrix on the host, write it with an F32 tensor to a
 * .safetensors file, read the file back and check every byte.  Exit 0 on success. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "jjjetson_ops_amd.h"

#define ROWS 8
#define COLS 64

int main(int argc, char **argv) {
    if (argc != 2) return 2;
    float w[ROWS * COLS], norm[COLS];
    for (int i = 0; i < ROWS * COLS; ++i) w[i] = (float)((i * 37) % 101 - 50) / 128.0f;
    for (int i = 0; i < COLS; ++i) norm[i] = 1.0f + (float)i / 64.0f;
    const int64_t qbytes = q4_0_bytes(ROWS, COLS);
    if (qbytes != ROWS * (COLS / 32) * 18) return 3;
    uint8_t *q = (uint8_t *)malloc((size_t)qbytes);
    if (quantize_q4_0_host(w, q, ROWS, COLS, 1) != JJO_OK) return 4;

    int64_t qdims[2] = {ROWS, COLS}, ndims[1] = {COLS};
    jjo_host_tensor out[2];
    memset(out, 0, sizeof out);
    out[0].name = (char *)"layer0.w_up";
    out[0].data = q;
    out[0].dims = qdims;
    out[0].ndim = 2;
    out[0].dtype = JJO_WEIGHT_DTYPE_Q4_0;
    out[0].nbytes = qbytes;
    out[1].name = (char *)"layer0.w_input_layernorm";
    out[1].data = norm;
    out[1].dims = ndims;
    out[1].ndim = 1;
    out[1].dtype = JJO_WEIGHT_DTYPE_F32;
    out[1].nbytes = (int64_t)sizeof norm;
    if (safetensors_write_file_q4_0(argv[1], out, 2) != JJO_OK) {
        fprintf(stderr, "write: %s\n", jjo_last_error());
        return 5;
    }

    jjo_host_tensor *in = NULL;
    int n = 0;
    if (safetensors_read_file_q4_0(argv[1], &in, &n) != JJO_OK || n != 2) {
        fprintf(stderr, "read: %s\n", jjo_last_error());
        return 6;
    }
    const jjo_host_tensor *t = jjo_host_tensors_find(in, n, "layer0.w_up");
    if (t == NULL || t->dtype != JJO_WEIGHT_DTYPE_Q4_0 || t->ndim != 2 || t->dims[0] != ROWS ||
        t->dims[1] != COLS || t->nbytes != qbytes || memcmp(t->data, q, (size_t)qbytes) != 0)
        return 7;
    t = jjo_host_tensors_find(in, n, "layer0.w_input_layernorm");
    if (t == NULL || t->dtype != JJO_WEIGHT_DTYPE_F32 || t->ndim != 1 || t->dims[0] != COLS ||
        memcmp(t->data, norm, sizeof norm) != 0)
        return 8;
    if (jjo_host_tensors_find(in, n, "missing") != NULL) return 9;
    jjo_host_tensors_free(in, n);
    free(q);
    /* errors come back as codes with a message, never as an exit */
    if (safetensors_read_file_q4_0("/nonexistent/x.safetensors", &in, &n) != JJO_ERR_INVALID_ARG) return 10;
    if (strstr(jjo_last_error(), "cannot open") == NULL) return 11;
    puts("ok");
    return 0;
}
