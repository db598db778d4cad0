/*
 * phpt_host.h — C API of the host runtime (libphptensors_host.so).
 *
 * This is the host-side mirror of the reference's CudaArray / Fusion
 * operator surface (src/cuda_array/cuda_array_ce.c, src/fusion.c), the
 * layer a PHP extension's Zend glue would call.  It sits above the device
 * C-ABI of include/pt_hip.h and never touches HIP itself.  Tensors are
 * opaque reference-counted handles; every call that can fail returns NULL
 * (or a negative value) and records an error retrievable with
 * phpt_error_kind() (1 = InvalidArgumentException, 2 = RuntimeException)
 * and phpt_error_message().
 */
#ifndef PHPT_HOST_H
#define PHPT_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct phpt_tensor phpt_tensor;
typedef struct phpt_graph phpt_graph;

#define PHPT_GLOBAL_AXIS (-1000)

int phpt_error_kind(void);
const char *phpt_error_message(void);
void phpt_clear_error(void);

/* ---- lifecycle / transfers (tensor_factory.c, tensor_transfer.c) ---- */
phpt_tensor *phpt_from_host(const void *data, int dtype, const int *shape, int ndims);
phpt_tensor *phpt_full(const int *shape, int ndims, int dtype, double value, int64_t ivalue, int kind);
int phpt_to_host(phpt_tensor *t, void *out, size_t bytes);
phpt_tensor *phpt_retain(phpt_tensor *t);
void phpt_release(phpt_tensor *t);
int phpt_dtype(phpt_tensor *t);
int phpt_ndims(phpt_tensor *t);
void phpt_shape(phpt_tensor *t, int *shape);
void phpt_strides(phpt_tensor *t, size_t *strides);
size_t phpt_size(phpt_tensor *t);
int phpt_is_lazy(phpt_tensor *t);
/* 1 for a tensor made by a view operation (slice, transpose, reshape,
 * broadcast, select): __serialize refuses those (cuda_array_ce.c:276-280) */
int phpt_is_view(phpt_tensor *t);
/* Device address of the tensor's first element (storage plus offset), for
 * a host that hands the buffer to another library; NULL for a value still
 * recorded in a Fusion scope.  No counterpart in the reference, whose
 * tensor_t exposes its pointer to C code directly (src/tensor.h:49-79). */
const void *phpt_device_pointer(phpt_tensor *t);
int phpt_dtype_from_name(const char *name);
const char *phpt_dtype_name(int dtype);

/* ---- views ---- */
phpt_tensor *phpt_reshape(phpt_tensor *t, const int *shape, int ndims);
phpt_tensor *phpt_transpose(phpt_tensor *t, const int *perm, int nperm);
phpt_tensor *phpt_broadcast_to(phpt_tensor *t, const int *shape, int ndims);
phpt_tensor *phpt_slice(phpt_tensor *t, int axis, int start, int stop, int step);
phpt_tensor *phpt_select(phpt_tensor *t, int axis, int index);

/* ---- operations (ca_private.c / cuda_array_ce.c) ---- */
/* scalar kind: 0 = float (value), 1 = int (ivalue), 2 = bool (ivalue) */
phpt_tensor *phpt_binary(phpt_tensor *a, phpt_tensor *b, int op);
phpt_tensor *phpt_scalar_op(phpt_tensor *a, double value, int64_t ivalue, int kind, int op, int reverse);
phpt_tensor *phpt_unary(phpt_tensor *a, int op);
phpt_tensor *phpt_reduce(phpt_tensor *a, int axis, int op);
phpt_tensor *phpt_reduce_arg(phpt_tensor *a, int axis, int op);
phpt_tensor *phpt_variance(phpt_tensor *a, int axis, long correction, int std_dev);
phpt_tensor *phpt_softmax(phpt_tensor *a, int axis);
phpt_tensor *phpt_layernorm(phpt_tensor *a, const int *axes, int naxes, double eps,
                            phpt_tensor *scale, phpt_tensor *bias);
phpt_tensor *phpt_matmul(phpt_tensor *a, phpt_tensor *b);
/* cuda_tune_matmul: times every tile configuration for a @ b, keeps the
 * fastest for that problem and returns the product; tiles / median_ms get up
 * to max_candidates entries.  NULL on error (too small: invalid argument). */
phpt_tensor *phpt_tune_matmul(phpt_tensor *a, phpt_tensor *b, int *tiles, float *median_ms,
                              int max_candidates, int *count, int *selected);
phpt_tensor *phpt_where(phpt_tensor *c, phpt_tensor *x, phpt_tensor *y);
/* CudaArray::gather / scatterAdd (cuda_array_ce.c:2423-2465): int32 indices,
 * axis may be negative */
phpt_tensor *phpt_gather(phpt_tensor *a, phpt_tensor *indices, long long axis);
phpt_tensor *phpt_scatter_add(phpt_tensor *a, phpt_tensor *indices, phpt_tensor *updates, long long axis);
phpt_tensor *phpt_astype(phpt_tensor *a, int dtype);
phpt_tensor *phpt_copy(phpt_tensor *a);

/* ---- Fusion (fusion.c, fusion_capture.c, fusion_plan.c, fusion_execute.c) ---- */
int phpt_fusion_begin(int compiling);
int phpt_fusion_active(void);
void phpt_fusion_abort(void);
phpt_tensor *phpt_fusion_input(phpt_tensor *example, int index);
/* Ends the scope and builds the plan whose roots are `outputs`.  For a
 * compile() scope the result is reusable; run() scopes call
 * phpt_fusion_run_once instead. */
phpt_graph *phpt_fusion_end(phpt_tensor **outputs, int count, int use_graph);
/* Ends a run() scope: executes once and replaces every lazy output (and
 * every recorded value still referenced elsewhere) with its result. */
int phpt_fusion_run_once(phpt_tensor **outputs, int count);
int phpt_graph_run(phpt_graph *g, phpt_tensor **inputs, int ninputs, phpt_tensor **outputs, int noutputs);
/* Replays the plan `count` times back to back on the runtime stream,
 * synchronizes once and returns the last execution's outputs (like
 * phpt_graph_run: their number, or -1).  Each execution drops the one
 * before it, so all reuse the plan's buffers, and whole groups of eight run
 * through one graph launch.  No counterpart in the reference, whose run()
 * synchronizes per replay (fusion.c:599-641); it exists to time replay
 * throughput. */
int phpt_graph_replay(phpt_graph *g, phpt_tensor **inputs, int ninputs, int count, phpt_tensor **outputs,
                      int noutputs);
/* FusionGraph::runAsync / FusionExecution (fusion.c:561-692): each
 * submission returns its own execution (NULL on error); several may be
 * pending for a plan without a captured graph.  wait returns the number of
 * outputs and fills `outputs`; release waits if needed and frees. */
typedef struct phpt_execution phpt_execution;
phpt_execution *phpt_graph_run_async(phpt_graph *g, phpt_tensor **inputs, int ninputs);
int phpt_execution_wait(phpt_execution *e, phpt_tensor **outputs, int noutputs);
int phpt_execution_is_finished(phpt_execution *e);
void phpt_execution_release(phpt_execution *e);
int phpt_graph_num_outputs(phpt_graph *g);
const char *phpt_graph_source(phpt_graph *g);
/* Statistics as "key=value;" pairs (FusionGraph::getStats, fusion.c:723-772). */
const char *phpt_graph_stats(phpt_graph *g);
/* Steps as "key=value,...;" entries (FusionGraph::getPlan, fusion.c:775-795). */
const char *phpt_graph_plan(phpt_graph *g);
/* fails (RuntimeException) while executions are pending */
int phpt_graph_set_profiling(phpt_graph *g, int enabled);
void phpt_graph_release(phpt_graph *g);
/* Module cache counters (Fusion::getCacheStats, fusion_cache.c:50-62). */
const char *phpt_fusion_cache_stats(void);
void phpt_fusion_clear_cache(void);

#ifdef __cplusplus
}
#endif

#endif
