/*
 * A C99 consumer of include/pt_hip.h: the call sequence of the reference's
 * cuda_tensor_reduce / cuda_tensor_reduce_arg (src/cuda_array/ca_private.c:
 * 236-342) over a float32 [rows, cols] matrix, written the way the PHP
 * extension's C host code would make it.
 *
 *   pt_reduce_driver <rows> <cols> <input.f32> <output.bin>
 *
 * Reads rows*cols float32 values, computes along axis 1 the sum, the max
 * (launch_reduction's replacement) and the argmax (launch_arg_reduction's),
 * and writes sum[rows] (float32), max[rows] (float32), argmax[rows] (int32)
 * in that order.  Exit status 0 on success; on a failing call it prints the
 * call, its status string and pt_last_error() and exits with 2.
 */
#include <stdio.h>
#include <stdlib.h>

#include "pt_hip.h"

#define CHECK(call)                                                                          \
    do {                                                                                     \
        pt_status st_ = (call);                                                              \
        if (st_ != PT_OK) {                                                                  \
            fprintf(stderr, "%s: %s (%s)\n", #call, pt_status_string(st_), pt_last_error()); \
            return 2;                                                                        \
        }                                                                                    \
    } while (0)

static int run(int rows, int cols, const char *in_path, const char *out_path)
{
    size_t n = (size_t)rows * (size_t)cols;
    float *host = (float *)malloc(n * sizeof(float));
    float *sum = (float *)malloc((size_t)rows * sizeof(float));
    float *mx = (float *)malloc((size_t)rows * sizeof(float));
    int32_t *arg = (int32_t *)malloc((size_t)rows * sizeof(int32_t));
    FILE *f;
    void *d_in = NULL, *d_sum = NULL, *d_max = NULL, *d_arg = NULL;
    int shape[2];
    size_t strides[2];

    if (!host || !sum || !mx || !arg) return 3;
    f = fopen(in_path, "rb");
    if (!f || fread(host, sizeof(float), n, f) != n) return 4;
    fclose(f);

    shape[0] = rows;
    shape[1] = cols;
    strides[0] = (size_t)cols;
    strides[1] = 1;

    CHECK(pt_init());
    /* result dtypes as ca_private.c:318-324 derives them */
    if (pt_reduce_result_dtype(PT_FLOAT32, PT_OP_REDUCE_SUM) != PT_FLOAT32) return 5;
    if (pt_reduce_result_dtype(PT_FLOAT32, PT_OP_REDUCE_MAX) != PT_FLOAT32) return 5;
    /* cuda_tensor_create_* allocations from the pool, then the upload */
    CHECK(pt_alloc(&d_in, n * sizeof(float), NULL));
    CHECK(pt_alloc(&d_sum, (size_t)rows * sizeof(float), NULL));
    CHECK(pt_alloc(&d_max, (size_t)rows * sizeof(float), NULL));
    CHECK(pt_alloc(&d_arg, (size_t)rows * sizeof(int32_t), NULL));
    CHECK(pt_memcpy_h2d(d_in, host, n * sizeof(float), NULL));
    /* launch_reduction / launch_arg_reduction + status checks */
    CHECK(pt_reduce(d_in, d_sum, PT_FLOAT32, PT_OP_REDUCE_SUM, shape, strides, 2, 1, 0, NULL));
    CHECK(pt_reduce(d_in, d_max, PT_FLOAT32, PT_OP_REDUCE_MAX, shape, strides, 2, 1, 0, NULL));
    CHECK(pt_arg_reduce(d_in, (int32_t *)d_arg, PT_FLOAT32, PT_OP_ARG_MAX, shape, strides, 2, 1, 0, NULL));
    /* toHost: synchronous downloads */
    CHECK(pt_memcpy_d2h(sum, d_sum, (size_t)rows * sizeof(float), NULL));
    CHECK(pt_memcpy_d2h(mx, d_max, (size_t)rows * sizeof(float), NULL));
    CHECK(pt_memcpy_d2h(arg, d_arg, (size_t)rows * sizeof(int32_t), NULL));
    CHECK(pt_stream_synchronize(NULL));
    CHECK(pt_free(d_in, NULL));
    CHECK(pt_free(d_sum, NULL));
    CHECK(pt_free(d_max, NULL));
    CHECK(pt_free(d_arg, NULL));

    f = fopen(out_path, "wb");
    if (!f) return 4;
    if (fwrite(sum, sizeof(float), (size_t)rows, f) != (size_t)rows ||
        fwrite(mx, sizeof(float), (size_t)rows, f) != (size_t)rows ||
        fwrite(arg, sizeof(int32_t), (size_t)rows, f) != (size_t)rows)
        return 4;
    fclose(f);
    free(host);
    free(sum);
    free(mx);
    free(arg);
    return 0;
}

int main(int argc, char **argv)
{
    int rows, cols;
    if (argc != 5) {
        fprintf(stderr, "usage: %s rows cols input.f32 output.bin\n", argv[0]);
        return 1;
    }
    rows = atoi(argv[1]);
    cols = atoi(argv[2]);
    if (rows <= 0 || cols <= 0) return 1;
    return run(rows, cols, argv[3], argv[4]);
}
