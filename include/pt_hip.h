/*
 * pt_hip.h — C-ABI of the MI355X (gfx950) device backend for php-gpu-tensors.
 *
 * This is the drop-in boundary: the PHP extension's unchanged C host code
 * (src/cuda_array/ca_private.c, src/cuda_array/cuda_array_ce.c composites,
 * src/fusion_*.c, src/cuda.c, src/tensor*.c) calls these functions where it
 * called the CUDA launchers, the CUDA wrapper and the CUDA memory pool.
 * Every entry point names the reference interface it replaces (file:line in
 * lcmialichi/php-gpu-tensors).
 *
 * Conventions
 *  - Plain C types only: pointers, sizes, ints.  No HIP, torch or PHP types.
 *  - dtype codes are the reference's dtype_t values (src/data_types.h:8-25)
 *    and op codes its operation_type_t values
 *    (src/operations_strctures.h:4-67), so the host passes its enums through.
 *  - Shapes are int[ndims], strides are size_t[ndims] in ELEMENTS (as in
 *    tensor_t, src/tensor.h:49-79); broadcast dimensions carry stride 0.
 *    All shape/stride arrays are host memory, read during the call only.
 *  - Data pointers are device pointers; launchers write caller-allocated
 *    outputs and never allocate outputs (scratch is internal, stream-ordered).
 *  - Every function returns a pt_status.  PT_ERR_INVALID maps to the
 *    reference's InvalidArgumentException, every other non-zero status to
 *    RuntimeException (src/cuda_exceptions.h:13-23).  pt_last_error()
 *    holds a thread-local message describing the most recent failure.
 *  - stream == NULL means the library's default stream (the reference
 *    launches eager work on the legacy default stream).
 */
#ifndef PT_HIP_H
#define PT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int pt_status;
enum {
    PT_OK = 0,
    PT_ERR_INVALID = 1,      /* bad argument: InvalidArgumentException */
    PT_ERR_RUNTIME = 2,      /* HIP runtime / launch failure */
    PT_ERR_UNSUPPORTED = 3,  /* dtype/op combination not provided */
    PT_ERR_NOMEM = 4,        /* device allocation failed */
    PT_ERR_COMPILE = 5,      /* hipRTC compilation failed */
    PT_ERR_NO_DEVICE = 6     /* no gfx950 device visible */
};

typedef void *pt_stream_t;   /* a hipStream_t */
typedef void *pt_event_t;    /* a hipEvent_t */
typedef void *pt_module_t;   /* a hipModule_t */
typedef void *pt_function_t; /* a hipFunction_t */
typedef void *pt_graph_t;    /* a captured hipGraph_t + its hipGraphExec_t */

/* dtype codes (src/data_types.h:8-25) */
enum {
    PT_FLOAT32 = 0, PT_FLOAT64 = 1, PT_INT8 = 2, PT_INT16 = 3, PT_INT32 = 4,
    PT_INT64 = 5, PT_UINT8 = 6, PT_UINT16 = 7, PT_UINT32 = 8, PT_UINT64 = 9,
    PT_BOOL = 10, PT_FLOAT16 = 11, PT_BFLOAT16 = 12
};

/* op codes used at this boundary (src/operations_strctures.h:4-67) */
enum {
    PT_OP_ADD = 0, PT_OP_SUB = 1, PT_OP_MUL = 2, PT_OP_DIV = 3, PT_OP_POW = 4,
    PT_OP_EXP = 5, PT_OP_EXPM1 = 6, PT_OP_SQRT = 7, PT_OP_LOG = 8,
    PT_OP_LOG1P = 9, PT_OP_EXP2 = 10, PT_OP_LOG2 = 11, PT_OP_LOG10 = 12,
    PT_OP_ASIN = 13, PT_OP_ACOS = 14, PT_OP_ATAN = 15, PT_OP_SINH = 16,
    PT_OP_COSH = 17, PT_OP_TANH = 18, PT_OP_SIN = 19, PT_OP_COS = 20,
    PT_OP_TAN = 21, PT_OP_ABS = 22, PT_OP_NEG = 23, PT_OP_CEIL = 26,
    PT_OP_FLOOR = 27, PT_OP_ROUND = 28,
    PT_OP_GT = 29, PT_OP_LT = 30, PT_OP_EQ = 31, PT_OP_NE = 32, PT_OP_GE = 33,
    PT_OP_LE = 34,
    PT_OP_REDUCE_SUM = 35, PT_OP_REDUCE_MEAN = 36, PT_OP_REDUCE_MAX = 37,
    PT_OP_REDUCE_MIN = 38, PT_OP_REDUCE_PROD = 39,
    PT_OP_ARG_MAX = 42, PT_OP_ARG_MIN = 43,
    PT_OP_MAXIMUM = 54, PT_OP_MINIMUM = 55,
    PT_OP_REDUCE_ALL = 57, PT_OP_REDUCE_ANY = 58
};

/* A scalar operand (replaces scalar_value_t, src/data_types.h:38-59):
 * the active member is selected by dtype. */
typedef struct {
    union {
        double f64;
        float f32;
        int64_t i64;
        uint64_t u64;
        uint16_t u16;  /* float16 / bfloat16 bit pattern */
    } v;
    int dtype;
} pt_scalar_t;

/* --------------------------------------------------------------- device --
 * Replaces src/cuda_wrapper.h:11-26 (cuda_wrapper_get_device_count,
 * _get_device_properties, _set_device, _synchronize, _get_error_string). */
typedef struct {
    char name[256];
    char arch[64];           /* e.g. "gfx950:sramecc+:xnack-" */
    int compute_units;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;
    size_t total_memory;
    size_t lds_per_block;
    int warp_size;           /* 64 on CDNA */
    int max_threads_per_block;
    int l2_cache_bytes;
} pt_device_info;

pt_status pt_init(void);
pt_status pt_device_count(int *count);
pt_status pt_device_set(int device);
pt_status pt_device_get(int *device);
pt_status pt_device_info_get(int device, pt_device_info *info);
pt_status pt_device_synchronize(void);
const char *pt_status_string(pt_status status);
const char *pt_last_error(void);
pt_status pt_version(int *major, int *minor);

/* --------------------------------------------------------------- streams --
 * The reference's Fusion executor creates private non-blocking streams and
 * readiness events (src/fusion_execute.c:385-412); these replace those
 * cuStream / cuEvent calls. */
pt_status pt_stream_create(pt_stream_t *stream);
pt_status pt_stream_destroy(pt_stream_t stream);
pt_status pt_stream_synchronize(pt_stream_t stream);
pt_status pt_stream_query(pt_stream_t stream, int *finished);
pt_status pt_stream_wait_event(pt_stream_t stream, pt_event_t event);
pt_stream_t pt_default_stream(void);
/* Stream used on the calling thread by calls that pass a NULL stream (the
 * runtime stream when `stream` is NULL).  Lets a host runtime route whole
 * operations to the branches of a multi-stream graph capture; replaces the
 * plan stream of fusion_enqueue (fusion_execute.c:385-412). */
pt_status pt_stream_set_current(pt_stream_t stream);
pt_status pt_event_create(pt_event_t *event);
pt_status pt_event_destroy(pt_event_t event);
pt_status pt_event_record(pt_event_t event, pt_stream_t stream);
pt_status pt_event_synchronize(pt_event_t event);
pt_status pt_event_query(pt_event_t event, int *finished);
pt_status pt_event_elapsed_ms(pt_event_t start, pt_event_t stop, float *ms);

/* ---------------------------------------------------------------- memory --
 * Replaces the best-fit pool of src/backends/cuda/memory_pool.h:34-44
 * (tensor_mem_init, cuda_mem_alloc, cuda_mem_free) with a stream-ordered
 * HIP memory pool; frees are ordered on the given stream instead of
 * assuming default-stream ordering.  pool_bytes is the retained-memory
 * threshold (INI phptensors.cuda.memory_pool_size, src/cuda.c:64-81). */
pt_status pt_mem_init(size_t pool_bytes);
pt_status pt_alloc(void **ptr, size_t bytes, pt_stream_t stream);
pt_status pt_free(void *ptr, pt_stream_t stream);
pt_status pt_mem_info(size_t *free_bytes, size_t *total_bytes, size_t *pool_reserved);
/* Transfers (replace cudaMemcpy in src/cuda_array/tensor_transfer.c:45-65,
 * src/cuda_array/tensor_factory.c:301-326).  Synchronous w.r.t. the host.
 * A pageable host buffer of 4 MiB or more is moved through the library's
 * two pinned 16 MiB chunks, the host copy of one overlapping the DMA of the
 * other; pinned buffers (pt_host_alloc_pinned) are copied directly. */
pt_status pt_memcpy_h2d(void *dst, const void *src, size_t bytes, pt_stream_t stream);
pt_status pt_memcpy_d2h(void *dst, const void *src, size_t bytes, pt_stream_t stream);
pt_status pt_memcpy_d2d(void *dst, const void *src, size_t bytes, pt_stream_t stream);
pt_status pt_memset(void *dst, int value, size_t bytes, pt_stream_t stream);
pt_status pt_host_alloc_pinned(void **ptr, size_t bytes);
pt_status pt_host_free_pinned(void *ptr);

/* ------------------------------------------------------------ reductions --
 * pt_reduce replaces launch_reduction (src/backends/cuda/reduction_ops.h:
 * 15-22) + cuda_reduction_status (:12): sum/mean/max/min/prod along `axis`
 * (axis < 0: all elements, output shape [1]); all/any (OP_REDUCE_ALL / ANY,
 * cuda_array_ce.c:1791-1823) write bool: every / some element unequal to zero.
 * Output dtype as
 * ca_private.c:318-324: mean -> float32 for f32/f16/bf16 input, float64 for
 * f64/int/bool; f16/bf16 sum/max/min/prod -> float32 (the reference casts
 * them to float32 first, ca_private.c:297-304); other ops keep the input
 * dtype (integer sums wrap modulo the dtype width).  max/min skip NaN.
 * An empty reduced axis with max/min is PT_ERR_INVALID.
 * base_offset is in elements. */
pt_status pt_reduce(const void *input, void *output, int dtype, int op,
                    const int *shape, const size_t *strides, int ndims, int axis,
                    size_t base_offset, pt_stream_t stream);

/* Output dtype pt_reduce writes for (dtype, op); -1 if unsupported. */
int pt_reduce_result_dtype(int dtype, int op);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same arguments, kernels and results as pt_reduce,
 * but the scratch those kernels use (global-reduction partials,
 * column-split partials, the packed copy of a strided input) comes from a
 * static 1 MiB buffer the library holds on each device, not from the pool;
 * nothing is allocated.  A reduction that needs more scratch fails with
 * PT_ERR_INVALID.  Every call on a device shares that device's buffer, and
 * calls that overlap on one device (other threads or streams) are ordered
 * on the GPU rather than racing: each call's stream waits for the event the
 * previous call recorded after its kernels (created once per device at the
 * first call; a call allocates nothing).  Under stream capture that
 * hand-off is skipped, so a graph holding the call must not run while
 * another call on the device does. */
pt_status pt_reduce_noalloc(const void *input, void *output, int dtype, int op,
                            const int *shape, const size_t *strides, int ndims, int axis,
                            size_t base_offset, pt_stream_t stream);

/* Replaces launch_arg_reduction (reduction_ops.h:31-38): int32 indices of
 * the max/min along axis (axis < 0: flattened), ties -> lowest index, NaN
 * never selected, an axis whose best value equals the identity -> 0
 * (reduction_ops.cuh:319-401). */
pt_status pt_arg_reduce(const void *input, int32_t *output, int dtype, int op,
                        const int *shape, const size_t *strides, int ndims, int axis,
                        size_t base_offset, pt_stream_t stream);

/* Replaces launch_moments_reduction (reduction_ops.h:23-29): variance
 * M2/(n - correction) (or its sqrt when standard_deviation != 0) along axis
 * (axis < 0: all elements).  result_dtype must be PT_FLOAT32 for
 * f32/f16/bf16 input and PT_FLOAT64 otherwise (ca_private.c:717). */
pt_status pt_moments(const void *input, void *output, int input_dtype, int result_dtype,
                     const int *shape, const size_t *strides, int ndims, int axis,
                     int correction, int standard_deviation, pt_stream_t stream);

/* -------------------------------------------------- fused row kernels ----
 * New fused entry points replacing the CudaArray composites (5 launches and
 * 3 temporaries for softmax, cuda_array_ce.c:1942-2001; 9-11 launches for
 * layerNorm, :2215-2339) with one HBM read and one write.
 *
 * pt_softmax: y = exp(x - max) / sum(exp(x - max)) along `axis` of a
 * strided input; output contiguous with the input's shape.  output_dtype
 * is PT_FLOAT32 for f32/f16/bf16 input and PT_FLOAT64 otherwise
 * (cuda_array_ce.c:1944-1948).  An empty axis is PT_ERR_INVALID when the
 * tensor has elements outside it. */
pt_status pt_softmax(const void *input, void *output, int input_dtype, int output_dtype,
                     const int *shape, const size_t *strides, int ndims, int axis,
                     pt_stream_t stream);

/* pt_layernorm: normalizes each of `rows` contiguous rows of n elements:
 * y = (x - mean) / sqrt(mean((x - mean)^2) + eps) * gamma + beta with the
 * biased variance and eps inside the sqrt (cuda_array_ce.c:2295-2323).
 * input_dtype f32/f16/bf16/f64; compute_dtype PT_FLOAT32 or PT_FLOAT64 is
 * also the output dtype; gamma/beta (may be NULL) are contiguous [n] arrays
 * of compute_dtype.  The host makes the normalized axes trailing and
 * contiguous before the call. */
pt_status pt_layernorm(const void *input, void *output, int input_dtype, int compute_dtype,
                       size_t rows, size_t n, double eps,
                       const void *gamma, const void *beta, pt_stream_t stream);

/* ------------------------------------------------------------------ GEMM --
 * Replaces cuda_matmul_launcher (src/backends/cuda/matmul_kernels.h:40-44),
 * cuda_batched_matmul_nd_launcher (:47-51) and
 * cuda_low_precision_matmul_nd_launcher (:53-57) with one entry point:
 * C[batch] = A[batch] @ B[batch] for dtype f32, f16 or bf16 (matching
 * operands; fp32 accumulation; f16/bf16 outputs rounded to nearest even).
 * Shapes follow tensor_matmul_shape (src/tensor_shape.h:46-59): leading
 * batch dims broadcast, strides (elements) may describe transposed or
 * broadcast views of A and B; C must be contiguous row-major. */
pt_status pt_matmul(const void *a, const void *b, void *c, int dtype,
                    const int *shape_a, const size_t *strides_a, int nd_a,
                    const int *shape_b, const size_t *strides_b, int nd_b,
                    const int *shape_c, int nd_c, pt_stream_t stream);

/* Precision policy (replaces cuda_blas_set_precision / _precision_name,
 * matmul_kernels.h:31-33).  0 = fp32-strict (the default); 1 = tf32 is
 * refused with PT_ERR_UNSUPPORTED, as the reference refuses it on a device
 * without TF32 (tests/matmul_precision.phpt:51-56): gfx950 has no xf32 MFMA.
 * Other values: PT_ERR_INVALID.  The mode never changes on an error. */
pt_status pt_matmul_set_precision(int precision);
const char *pt_matmul_precision_name(void);

/* Tile override for the MFMA kernels, the tuning knob that replaces
 * cuda_blas_tune_matmul (matmul_kernels.h:34-38): 0 = 256x128, 1 = 128x128,
 * 2 = 64x64, 3 = 256x256 workgroup tiles, 5 = 256x256 with a doubled K step
 * (4, 6 and 7 are not built and are refused), 8 = 256x256 direct-to-LDS
 * kernel for f16/bf16 (whole tiles, K a multiple of 64, k-contiguous A;
 * other cases run tile 3), 9 = 256x128 with 8 waves, 10 / 11 = 128x128 with
 * 8 waves (single / doubled K step), 12 / 13 = 128x64 with 4 waves and two
 * workgroups per CU (single / doubled K step); 11-13 are fp32 only and
 * 16-bit requests run 128x128.  14-37 = the 16-bit LDS-ring kernels (37, the
 * whole-line ring, is the default for large bf16/fp16 products), 38 = the
 * fp32 LDS-ring kernel (128x128 tiles), the default for fp32 products of
 * 128x128 tiles and up whose operands come in 16-byte packs and whose K is
 * a multiple of 32 (others run tile 10; 16-bit requests run 128x128).
 * -1 = automatic choice (default). */
pt_status pt_matmul_set_tile(int tile);
/* Measured tile choice for one problem, the counterpart of
 * cuda_blas_tune_matmul (matmul_kernels.h:34-38; a cuBLASLt candidate sweep
 * there, matmul_kernels.cu:336-456).  Every tile configuration built for the
 * dtype runs once untimed and five times between HIP events on `stream`,
 * writing `c`; the fastest median is kept for this (dtype, M, N, K, batch,
 * operand layout) and used by later pt_matmul calls with no tile override
 * (backend info then reports a "-tuned" matmul).  tiles / median_ms receive
 * up to max_candidates entries, *count how many were written, *selected the
 * index of the fastest; `c` ends holding the product.  A problem with
 * M*N*K below 1e7 is not eligible (PT_ERR_INVALID), as the reference tunes
 * only its cuBLASLt range. */
pt_status pt_matmul_tune(const void *a, const void *b, void *c, int dtype,
                         const int *shape_a, const size_t *strides_a, int nd_a,
                         const int *shape_b, const size_t *strides_b, int nd_b,
                         const int *shape_c, int nd_c, int *tiles, float *median_ms,
                         int max_candidates, int *count, int *selected, pt_stream_t stream);

/* Instruction-schedule variant of the MFMA kernels (tuning knob):
 * 0 = compiler default, 1 and 2 = iglp strategies (2 is the default),
 * 3 = MFMA / LDS-read interleave, 4 and 5 = two 256x128 workgroups per CU
 * (tile 0) without / with the iglp strategy. */
pt_status pt_matmul_set_schedule(int sched);

/* Backend counters (replace cuda_backend_info, backend_info.h:7-16). */
typedef struct {
    char last_matmul[32];
    uint64_t mfma_gemm_calls;
    uint64_t generic_gemm_calls;
    uint64_t row_reduce_calls;
    uint64_t column_reduce_calls;
    uint64_t strided_reduce_calls;
    uint64_t global_reduce_calls;
    uint64_t fused_row_calls;
    uint64_t elementwise_calls;
    uint64_t rtc_compiles;
    uint64_t graph_launches;
    uint64_t staged_copies;  /* transfers staged through the pinned ring */
} pt_backend_info;
pt_status pt_backend_info_get(pt_backend_info *info);
pt_status pt_backend_info_reset(void);

/* ----------------------------------------------------------- elementwise --
 * pt_broadcast replaces launch_broadcast (src/backends/cuda/broadcast_ops.h:
 * 10-16): out[i] = a[i] (op) b[i] over the output shape; strides_a/b are
 * aligned to the output rank with stride 0 on broadcast dims.  Both
 * operands are converted to the output dtype (float for f16/bf16 outputs)
 * and the op is evaluated there, as broadcast_kernel_with_cast /
 * _low_precision (broadcast_ops.cuh:62-150); comparisons write 1/0 in the
 * output (promoted) dtype.  Ops: + - * / ** maximum minimum > < == != >= <=.
 * No contraction: a*b+c is two rounded operations. */
pt_status pt_broadcast(const void *a, int dtype_a, const size_t *strides_a, size_t offset_a,
                       const void *b, int dtype_b, const size_t *strides_b, size_t offset_b,
                       void *out, int dtype_out, int op,
                       const int *shape, int ndims, pt_stream_t stream);

/* Replaces launch_scalar / launch_scalar_inv (scalar_ops.h:11-37):
 * out = in (op) scalar, or scalar (op) in when reverse != 0, evaluated in
 * the output dtype like pt_broadcast. */
pt_status pt_scalar(const void *input, int dtype_in, const size_t *strides, size_t offset,
                    const pt_scalar_t *scalar, int reverse, void *out, int dtype_out,
                    int op, const int *shape, int ndims, pt_stream_t stream);

/* Replaces launch_unary_op (unary_ops.h:12-21): out = f(in), computed in
 * float32 for f32/f16/bf16 and float64 for f64; output dtype = input dtype. */
pt_status pt_unary(const void *input, int dtype, const size_t *strides, size_t offset,
                   void *out, int op, const int *shape, int ndims, pt_stream_t stream);

/* Replaces launch_tensor_cast (factory_kernels.h:28-31) and
 * launch_pack_strided (factory_kernels.cu:35): strided input -> contiguous
 * output with dtype conversion (same dtype = pack). */
pt_status pt_cast(const void *input, int dtype_in, const size_t *strides, size_t offset,
                  void *out, int dtype_out, const int *shape, int ndims, pt_stream_t stream);

/* Replaces launch_where_kernel (where_kernels.cu:67-107): out = cond != 0 ?
 * x : y with broadcasting (strides aligned to the output rank). */
pt_status pt_where(const void *cond, int dtype_cond, const size_t *strides_cond,
                   const void *x, const size_t *strides_x,
                   const void *y, const size_t *strides_y, int dtype_xy,
                   void *out, const int *shape, int ndims, pt_stream_t stream);

/* Replaces the fill kernels of factory_kernels.cu (zeros/ones/full). */
pt_status pt_fill(void *out, int dtype, size_t n, const pt_scalar_t *value, pt_stream_t stream);

/* --------------------------------------------------------------- indexed --
 * Replaces cuda_validate_indices, cuda_launch_gather, cuda_launch_scatter_add
 * (src/backends/cuda/indexed_ops.h:25-42), called from cuda_tensor_gather /
 * cuda_tensor_scatter_add (src/cuda_array/ca_private.c:916-1007) and from
 * Fusion's indexed native steps (src/fusion_execute.c:198-226).
 *
 * Indices are int32 with the input's rank; outside the indexed axis the
 * index shape equals the input shape.  A validation record is a device
 * int32[3] {operation, index, axis_size}: operation 0 = valid, 1 = a gather
 * index, 2 = a scatter-add index outside [0, axis_size) (the first one a
 * kernel meets; cuda_index_validation_result, indexed_ops.h:11-23).
 *
 * pt_index_validate clears `record` and checks every index against
 * [0, axis_size), writing operation 1 on the first invalid one; the caller
 * downloads the record (12 bytes) to learn the outcome, as ca_private.c:924
 * does before it launches. */
pt_status pt_index_validate(const int32_t *indices, const int *index_shape, const size_t *index_strides,
                            size_t index_offset, int ndims, int axis, int axis_size, int32_t *record,
                            pt_stream_t stream);
/* out[c] = input[c with c[axis] := indices[c]] for every coordinate c of the
 * index shape; out is contiguous row-major of the index shape and the
 * input's dtype (any dtype: elements are copied bit for bit).  With
 * validation != NULL an invalid index writes 0 to its output and is recorded
 * there (the caller clears the record first, e.g. with pt_memset); with NULL
 * the caller has validated the indices. */
pt_status pt_gather(const void *input, int dtype, const int *input_shape, const size_t *input_strides,
                    size_t input_offset, const int32_t *indices, const int *index_shape,
                    const size_t *index_strides, size_t index_offset, int ndims, int axis, void *output,
                    int32_t *validation, pt_stream_t stream);
/* output[c with c[axis] := indices[c]] += updates[c] (atomic float32 /
 * float64 adds; the order of adds to one element is not fixed).  The
 * caller first copies the input into `output` (strides output_strides,
 * extent axis_size along the axis), as cuda_launch_scatter_copy does. */
pt_status pt_scatter_add(const int32_t *indices, const int *index_shape, const size_t *index_strides,
                         size_t index_offset, const void *updates, const size_t *update_strides,
                         size_t update_offset, int dtype, int ndims, int axis, int axis_size, void *output,
                         const size_t *output_strides, int32_t *validation, pt_stream_t stream);

/* ------------------------------------------------------ runtime compile --
 * Replaces cuda_compile_generated_source (src/compiler_ce.h:15) + NVRTC
 * (compiler_ce.c:513-560) + cuModuleLoadData/cuModuleGetFunction
 * (fusion_cache.c:141, fusion_plan.c:613-623): compiles HIP C++ with
 * hipRTC for the current gfx950 device (-O3, -ffp-contract=off) and loads
 * the code object.  log (optional) receives the compiler log on failure. */
pt_status pt_rtc_compile(const char *source, const char *program_name,
                         pt_module_t *module, char *log, size_t log_bytes);
pt_status pt_module_function(pt_module_t module, const char *name, pt_function_t *function);
pt_status pt_module_unload(pt_module_t module);
/* Replaces cuLaunchKernel (fusion_execute.c): params is the kernel
 * argument array as for hipModuleLaunchKernel. */
pt_status pt_launch(pt_function_t function, unsigned grid_x, unsigned block_x,
                    void **params, pt_stream_t stream);

/* Scratch workspace of the calling thread.  Replaces the per-stream
 * reduction workspaces that natives captured into a graph use
 * (src/backends/cuda/reduction_ops.cu:11-60, released with the capture
 * stream at fusion_plan.c:198-204).  Between begin and end, the scratch of
 * multi-kernel operations (split-K partials, column and global reduction
 * partials) is carved from [base, base + bytes) instead of the stream-
 * ordered pool, so a captured graph holds no allocation; an operation whose
 * scratch does not fit fails with PT_ERR_NOMEM.  A region is not handed
 * out again before end, so operations that run concurrently (branches of a
 * captured graph) never share scratch.  base NULL and bytes 0: measuring
 * mode (pool allocations, total recorded).  end reports the scratch bytes
 * taken between begin and end (256-byte granules). */
pt_status pt_workspace_begin(void *base, size_t bytes);
pt_status pt_workspace_end(size_t *peak_bytes);

/* --------------------------------------------------------------- graphs --
 * Replaces the cuGraphCreate / cuGraphAddKernelNode / Instantiate /
 * ExecKernelNodeSetParams / cuGraphLaunch sequence of fusion_execute.c:
 * 518-597 with stream capture: begin, issue any pt_* launches on the
 * stream, end.  pt_graph_update re-captures into an existing executable
 * graph (hipGraphExecUpdate) when buffer pointers change. */
pt_status pt_graph_begin_capture(pt_stream_t stream);
pt_status pt_graph_end_capture(pt_stream_t stream, pt_graph_t *graph);
pt_status pt_graph_end_capture_update(pt_stream_t stream, pt_graph_t graph);
pt_status pt_graph_launch(pt_graph_t graph, pt_stream_t stream);
pt_status pt_graph_destroy(pt_graph_t graph);
pt_status pt_graph_node_count(pt_graph_t graph, size_t *nodes);

#ifdef __cplusplus
}
#endif

#endif
