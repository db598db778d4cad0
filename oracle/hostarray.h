/*
 * CPU ORACLE — test infrastructure only.
 *
 * A scalar, single-threaded C restatement of the reference's HostArray CPU
 * implementation (lcmialichi/php-gpu-tensors src/contiguous_array_ce.c) plus
 * restatements of the CudaArray composite semantics that HostArray lacks
 * (argMax/argMin, var/std, softmax, layerNorm).  Every function cites the
 * reference file:line it follows.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / CPU baseline.  The product
 * path (php-gpu-tensors_amd/) never links or calls it.
 *
 * Pinning (what checks each function beyond retyping its formula) is listed
 * per function below; tests/test_oracle_*.py hold those checks.
 */
#ifndef ORACLE_HOSTARRAY_H
#define ORACLE_HOSTARRAY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: identical numbering to src/data_types.h:8-25 (dtype_t). */
enum {
    OR_F32 = 0, OR_F64 = 1, OR_I8 = 2, OR_I16 = 3, OR_I32 = 4, OR_I64 = 5,
    OR_U8 = 6, OR_U16 = 7, OR_U32 = 8, OR_U64 = 9, OR_BOOL = 10,
    OR_F16 = 11, OR_BF16 = 12
};

/* operation codes: identical numbering to src/operations_strctures.h:4-67. */
enum {
    OR_OP_ADD = 0, OR_OP_SUB = 1, OR_OP_MUL = 2, OR_OP_DIV = 3,
    OR_OP_EXP = 5, OR_OP_EXPM1 = 6, OR_OP_SQRT = 7, OR_OP_LOG = 8,
    OR_OP_LOG1P = 9, OR_OP_EXP2 = 10, OR_OP_LOG2 = 11, OR_OP_LOG10 = 12,
    OR_OP_ASIN = 13, OR_OP_ACOS = 14, OR_OP_ATAN = 15, OR_OP_SINH = 16,
    OR_OP_COSH = 17, OR_OP_TANH = 18, OR_OP_SIN = 19, OR_OP_COS = 20,
    OR_OP_TAN = 21, OR_OP_ABS = 22, OR_OP_NEG = 23, OR_OP_CEIL = 26,
    OR_OP_FLOOR = 27, OR_OP_ROUND = 28,
    OR_OP_REDUCE_SUM = 35, OR_OP_REDUCE_MEAN = 36, OR_OP_REDUCE_MAX = 37,
    OR_OP_REDUCE_MIN = 38,
    OR_OP_ARG_MAX = 42, OR_OP_ARG_MIN = 43
};

/* Status codes returned by every oracle entry point. */
enum { OR_OK = 0, OR_EINVAL = 1 };

/* ---- dtype conversions: src/data_types.c:46-131 -------------------------
 * Pinned by: matmul_low_precision.phpt:28-46 vectors (RNE ties, overflow,
 * subnormals, underflow) and by exhaustive/bulk comparison against numpy's
 * float16 and torch's bfloat16 RNE casts (tests/test_oracle_dtypes.py). */
uint16_t or_f32_to_f16(float value);
float or_f16_to_f32(uint16_t value);
uint16_t or_f32_to_bf16(float value);
float or_bf16_to_f32(uint16_t value);
void or_f32_to_f16_n(const float *in, uint16_t *out, size_t n);
void or_f16_to_f32_n(const uint16_t *in, float *out, size_t n);
void or_f32_to_bf16_n(const float *in, uint16_t *out, size_t n);
void or_bf16_to_f32_n(const uint16_t *in, float *out, size_t n);

/* Result dtype of a HostArray reduction (contiguous_array_ce.c:1194-1195). */
int or_reduce_result_dtype(int dtype, int op);

/* ---- HostArray::sum/mean/min/max: contiguous_array_ce.c:1163-1270 -------
 * x is contiguous row-major with the given shape.  axis < 0 reduces all
 * elements (output shape [1]).  out receives or_reduce_result_dtype() values.
 * Pinned by: ca_sum_reduce / ca_mean_reduce / ca_max_reduce / ca_min_reduce
 * expectations, exact integer-valued closed forms, fsum bounds and
 * numpy.nanmax/nanmin equality (tests/test_oracle_reduce.py). */
int or_reduce(const void *x, int dtype, const int *shape, int ndims, int axis,
              int op, void *out);

/* ---- CudaArray::argMax/argMin semantics (HostArray has none:
 * host_array_unsupported.h:31): reduction_ops.cuh:319-401 + ca_private.c:263.
 * int32 indices, ties -> lowest index, NaN never selected, an axis whose
 * best value equals the identity (all -inf for argmax) yields 0.
 * Pinned by: ca_argmax_reduce.phpt expectations, numpy.argmax on NaN-free
 * data (first occurrence), and hand-built tie/NaN/-inf rows. */
int or_arg_reduce(const void *x, int dtype, const int *shape, int ndims,
                  int axis, int op, int32_t *out);

/* ---- CudaArray::var/std semantics: cuda_array_ce.c:1850-1940,
 * Welford combine reduction_ops.cuh:97-112, M2/(n - correction).
 * Sequential Welford carried in double; output float32 for float32/f16/bf16
 * input, float64 otherwise (ca_private.c:717).
 * Pinned by: cudaarray_variance.phpt expectations and numpy.var(ddof=c). */
int or_moments(const void *x, int dtype, const int *shape, int ndims, int axis,
               int correction, int standard_deviation, void *out);

/* ---- CudaArray::softmax composite: cuda_array_ce.c:1942-2001 ------------
 * max -> subtract -> expf -> sum -> divide, each step rounded to float32
 * (float64 for f64/int input).  Inner reductions follow HostArray order
 * (sequential).  Last-axis only: rows x n contiguous.
 * Pinned by: cudaarray_softmax.phpt:58-62 closed form
 * (0.090031 0.244728 0.665241), float64 numpy softmax bound, sum-to-one. */
int or_softmax_f32(const float *x, size_t rows, size_t n, float *out);
int or_softmax_f64(const double *x, size_t rows, size_t n, double *out);

/* ---- CudaArray::layerNorm composite: cuda_array_ce.c:2215-2339 ----------
 * mean (HostArray order) -> center -> square -> mean -> +eps -> sqrtf ->
 * divide -> *gamma -> +beta, each rounded to float32.  gamma/beta may be
 * NULL.  Normalizes the trailing n elements of each of rows rows.
 * Pinned by: cudaarray_layernorm.phpt:81-83 (-0.99998 0.99998;
 * -1.49996 2.49994; 0.89442; -1.22474) and float64 numpy bound. */
int or_layernorm_f32(const float *x, size_t rows, size_t n, float eps,
                     const float *gamma, const float *beta, float *out);

/* ---- HostArray::matmul: contiguous_array_ce.c:1280-1343 -----------------
 * Batched broadcast matmul over strided operands (strides in elements),
 * per element sequential fmaf over k, result cast to the operand dtype
 * (f32, f16 or bf16; RNE through data_types.c:373-436).  shape_c must be
 * the tensor_matmul_shape() of a and b; c is written contiguous.
 * Pinned by: ca_matmul.phpt, host_array_math.phpt:78-89,
 * matmul_low_precision.phpt:55-70, ca_matmul_accelerated.phpt integer
 * patterns, exactness on integer-valued data and the gamma_K error bound
 * against float64 numpy. */
int or_matmul(const void *a, const int *shape_a, const size_t *strides_a, int nd_a,
              const void *b, const int *shape_b, const size_t *strides_b, int nd_b,
              int dtype, void *c, const int *shape_c, int nd_c);
/* or_matmul with its outputs split over `threads` host threads (1..256): the
 * same per-output sum, so the same bits. */
int or_matmul_mt(const void *a, const int *shape_a, const size_t *strides_a, int nd_a,
                 const void *b, const int *shape_b, const size_t *strides_b, int nd_b,
                 int dtype, void *c, const int *shape_c, int nd_c, int threads);

/* ---- HostArray binary arithmetic: contiguous_array_ce.c:1345-1447 -------
 * Floating dtypes only (f32/f64/f16/bf16), broadcast shapes, contiguous
 * operands.  result dtype = promote_types_for_arithmetic (data_types.c:
 * 492-516); for non-f64 results both operands are rounded to float and the
 * op is evaluated in float, then stored with the result dtype's rounding.
 * Pinned by: fusion_precision.phpt:15-16 (a+b*c without contraction),
 * numpy float32 elementwise equality, broadcast expectations of
 * fusion_broadcast_cast.phpt. */
int or_binary(const void *a, int dtype_a, const int *shape_a, int nd_a,
              const void *b, int dtype_b, const int *shape_b, int nd_b,
              int op, void *out, int dtype_out, const int *shape_out, int nd_out);

/* Tensor-scalar form (scalar already rounded to the result dtype by the
 * caller, contiguous_array_ce.c:1382-1392); reverse swaps operand order. */
int or_binary_scalar(const void *a, int dtype_a, size_t n, double scalar,
                     int op, int reverse, void *out, int dtype_out);

/* ---- HostArray unary libm math: contiguous_array_ce.c:1075-1131 ---------
 * f64 evaluated with the double libm function, other floating dtypes with
 * the float variant, stored with the dtype's rounding.
 * Pinned by: numpy float32/float64 ufunc agreement within 2 ulp and exact
 * special values (tanh(0)=0, tanh(+-inf)=+-1). */
int or_unary(const void *x, int dtype, size_t n, int op, void *out);

/* ---- CudaArray::where (HostArray::where contiguous_array_ce.c:1021-1073) -
 * Broadcast select: cond != 0 ? x : y, elements copied bitwise. */
int or_where(const void *cond, int dtype_c, const int *shape_c, int nd_c,
             const void *x, const int *shape_x, int nd_x,
             const void *y, const int *shape_y, int nd_y, int dtype_xy,
             void *out, const int *shape_out, int nd_out);

/* ---- CudaArray::gather / scatterAdd along one axis -----------------------
 * Restates the reference's gather_kernel / scatter_add_kernel
 * (src/backends/cuda/indexed_ops.cu:108-133, 179-204; the HostArray has no
 * indexed ops) for contiguous operands: for every coordinate c of the index
 * shape, gather writes out[c] = x[c with c[axis] := idx[c]] (elements copied
 * bitwise); scatter-add starts from a copy of x and adds upd[c] at that
 * position, in flat index order (f32 / f64 only).  Returns OR_EINVAL with
 * *bad = the first index outside [0, shape_x[axis]) (cuda_validate_indices,
 * indexed_ops.cu:226-256).
 * Pinned by: numpy take_along_axis (gather) and np.add.at (scatter-add) on
 * random shapes and axes, and the reference's cudaarray_extended.phpt /
 * indexed_low_precision.phpt vectors. */
int or_gather(const void *x, int dtype, const int *shape_x, const int32_t *idx,
              const int *shape_idx, int ndims, int axis, void *out, int32_t *bad);
int or_scatter_add(const void *x, int dtype, const int *shape_x, const int32_t *idx,
                   const int *shape_idx, const void *upd, int ndims, int axis,
                   void *out, int32_t *bad);

#ifdef __cplusplus
}
#endif

#endif
