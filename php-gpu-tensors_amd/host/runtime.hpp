// Host runtime of the MI355X backend: the C++ counterpart of the reference's
// tensor runtime and op dispatch (src/tensor.c, src/operations.c,
// src/cuda_array/ca_private.c, the cuda_array_ce.c composites and the Fusion
// compiler src/fusion_*.c).  It owns tensor metadata, applies the
// reference's dtype/shape rules, and reaches the GPU only through the C-ABI
// of include/pt_hip.h.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <memory>
#include <string>
#include <vector>

#include "../../include/pt_hip.h"

namespace phpt {

constexpr int kMaxDims = 10;        // MAX_DIMS, src/tensor.h:16
constexpr int kGlobalAxis = -1000;  // REDUCE_GLOBAL_FLAG analogue

// ------------------------------------------------------------------ errors
enum ErrorKind { ERR_NONE = 0, ERR_INVALID = 1, ERR_RUNTIME = 2 };
void set_invalid(const char *fmt, ...);
void set_runtime(const char *fmt, ...);
void clear_error();
int error_kind();
const char *error_message();
bool check_status(pt_status st, const char *what);  // false + error set on failure
pt_status last_failed_status();  // status of the latest check_status that failed
void reset_failed_status();

// ------------------------------------------------------------------ dtypes
// dtype_t numbering of src/data_types.h:8-25 (PT_* codes).
size_t dtype_size(int dt);
bool is_floating(int dt);
bool is_integer(int dt);
bool is_signed(int dt);
bool is_valid_dtype(int dt);
const char *dtype_name(int dt);
int dtype_from_name(const char *name);

// Scalar value with its dtype, as scalar_value_t (src/data_types.h:38-59).
struct Scalar {
    int dtype = PT_FLOAT64;
    double f = 0.0;       // float32/float64/float16/bfloat16 value (as double)
    int64_t i = 0;        // signed integers
    uint64_t u = 0;       // unsigned integers / bool
    bool is_neg = false;
    long double as_ld() const;
};
Scalar scalar_from_double(double v);
Scalar scalar_from_int(int64_t v);
Scalar scalar_from_bool(bool v);
// cast_single_value (data_types.c:373-436); returns false when the value is
// not representable (integer range), leaving `out` unchanged.
bool cast_scalar(const Scalar &in, int target, Scalar &out);
pt_scalar_t to_pt_scalar(const Scalar &s);

int promote_types(int a, int b);                                // :301-349
int promote_scalar_for_arithmetic(int t, int s, int op, bool is_neg);  // :438-490
int promote_types_for_arithmetic(int a, int b, int op);        // :492-516
bool can_safely_cast_to(int from, int to);                      // :570-629

// ------------------------------------------------------------------ tensors
struct Storage {
    void *ptr = nullptr;
    size_t bytes = 0;
    Storage() = default;
    Storage(const Storage &) = delete;
    Storage &operator=(const Storage &) = delete;
    ~Storage();
};

struct FusionNode;

struct Tensor {
    std::shared_ptr<Storage> storage;
    int dtype = PT_FLOAT32;
    int ndims = 0;
    int shape[kMaxDims] = {0};
    size_t strides[kMaxDims] = {0};  // elements
    size_t offset = 0;               // elements
    bool read_only = false;          // broadcast views
    bool is_view = false;            // made by a view operation (shares storage)
    bool fusion_failed = false;      // recorded in a Fusion scope that was aborted
    std::shared_ptr<FusionNode> node;  // set while recorded in a Fusion scope
    uint64_t id = 0;

    size_t numel() const;
    bool contiguous() const;
    bool lazy() const { return node != nullptr && !storage; }
    void *data() const;
    std::vector<int> shape_vec() const { return std::vector<int>(shape, shape + ndims); }
};
using TensorP = std::shared_ptr<Tensor>;

uint64_t next_tensor_id();
void contiguous_strides(const int *shape, int ndims, size_t *strides);
bool shape_metrics(const int *shape, int ndims, size_t *elements);  // tensor_shape_metrics
bool broadcast_shape(const int *a, int na, const int *b, int nb, int *out, int *nout);
bool matmul_shape(const int *a, int na, const int *b, int nb, int *out, int *nout);

TensorP make_empty(const int *shape, int ndims, int dtype);  // allocated, uninitialised
TensorP make_meta(const int *shape, int ndims, int dtype);   // metadata only (lazy)
TensorP from_host(const void *data, const int *shape, int ndims, int dtype);
bool to_host(const TensorP &t, void *out, size_t bytes);     // logical row-major bytes
TensorP full(const int *shape, int ndims, int dtype, const Scalar &value);
TensorP materialize(const TensorP &t);                       // contiguous copy if needed

// Native steps of a plan captured into a HIP graph must not allocate: while
// allocation_forbidden() is set, make_empty fails.  A plan hands a native
// step its (stable) output buffer with preset_output; the native operation
// takes it through output_tensor when shape and dtype match.
bool &allocation_forbidden();
uint64_t allocation_refusals();  // allocations refused while forbidden (this thread)
void preset_output(const TensorP &t);
TensorP output_tensor(const int *shape, int ndims, int dtype);

// views (share storage)
TensorP view(const TensorP &t, const int *shape, const size_t *strides, int ndims, size_t offset);
TensorP reshape(const TensorP &t, const int *shape, int ndims);
TensorP transpose(const TensorP &t, const int *perm, int nperm);
TensorP broadcast_to(const TensorP &t, const int *shape, int ndims);
TensorP slice_axis(const TensorP &t, int axis, int start, int stop, int step);
TensorP select_index(const TensorP &t, int axis, int index);

// ------------------------------------------------------------------ eager ops
// Names and validation follow src/cuda_array/ca_private.c.
TensorP cuda_tensor_op(const TensorP &a, const TensorP &b, int op);
TensorP cuda_scalar_op(const TensorP &a, const Scalar &s, int op);
TensorP cuda_inv_scalar_op(const TensorP &a, const Scalar &s, int op);
TensorP cuda_unary_op(const TensorP &a, int op);
TensorP cuda_tensor_reduce(const TensorP &a, int axis, int op);      // axis may be kGlobalAxis
TensorP cuda_tensor_reduce_arg(const TensorP &a, int axis, int op);  // axis may be kGlobalAxis
TensorP cuda_array_variance(const TensorP &a, int axis, long correction, bool std_dev);
TensorP cuda_array_softmax(const TensorP &a, int axis);
TensorP cuda_array_layernorm(const TensorP &a, const int *axes, int naxes, double eps,
                             const TensorP &scale, const TensorP &bias);
TensorP cuda_tensor_matmul(const TensorP &a, const TensorP &b);
TensorP cuda_tune_matmul(const TensorP &a, const TensorP &b, int *tiles, float *median_ms, int max_candidates,
                         int *count, int *selected);
TensorP cuda_tensor_where(const TensorP &c, const TensorP &x, const TensorP &y);
// gather / scatterAdd along `axis` (ca_private.c:916-1007); int32 indices
TensorP cuda_tensor_gather(const TensorP &input, const TensorP &indices, int axis);
TensorP cuda_tensor_scatter_add(const TensorP &input, const TensorP &indices, const TensorP &updates, int axis);
// validation record of the executing Fusion plan (nullptr outside one)
int32_t *&index_record();
TensorP tensor_cast(const TensorP &a, int dtype);
TensorP astype(const TensorP &a, int dtype);  // safe casts only (CudaArray::astype)
TensorP copy(const TensorP &a);

// ------------------------------------------------------------------ fusion
// Recording mirrors src/fusion_capture.c: inside a Fusion scope every op on
// CudaArray values appends a node and returns a lazy tensor (shape and
// dtype known, no storage).
enum NodeKind {
    N_INPUT = 0,   // placeholder bound at run time (Fusion::compile inputs)
    N_BINARY,      // tensor (op) tensor
    N_SCALAR,      // tensor (op) scalar, or scalar (op) tensor when reverse
    N_UNARY,
    N_CAST,
    N_WHERE,
    N_VIEW,        // affine index map over the source's logical layout
    N_NATIVE       // boundary op executed by a native kernel
};

enum NativeKind {
    NAT_MATMUL = 0, NAT_REDUCE, NAT_ARG_REDUCE, NAT_MOMENTS, NAT_SOFTMAX, NAT_LAYERNORM, NAT_GATHER, NAT_SCATTER_ADD
};

struct NativeSpec {
    int kind = NAT_MATMUL;
    int op = 0;
    int axis = 0;
    long correction = 0;
    bool std_dev = false;
    double eps = 0.0;
    int naxes = 0;
    int axes[kMaxDims] = {0};
    bool has_scale = false, has_bias = false;
};

struct FusionNode {
    NodeKind kind = N_INPUT;
    int op = 0;
    std::vector<TensorP> inputs;
    Scalar scalar;
    bool reverse = false;
    // N_VIEW: out index -> source linear index = offset + sum coord_d * stride_d
    size_t view_strides[kMaxDims] = {0};
    size_t view_offset = 0;
    NativeSpec native;
    int input_index = -1;  // N_INPUT: position in the compile() input list
};

bool fusion_active();
TensorP fusion_record(NodeKind kind, int op, std::vector<TensorP> inputs, const int *shape,
                      int ndims, int dtype);
TensorP fusion_record_scalar(const TensorP &a, const Scalar &s, int op, bool reverse, int dtype);
TensorP fusion_record_view(const TensorP &a, const int *shape, const size_t *strides, int ndims,
                           size_t offset);
TensorP fusion_record_native(const NativeSpec &spec, std::vector<TensorP> inputs, const int *shape,
                             int ndims, int dtype);
// Execute the recorded graph that produces a lazy tensor (in-scope
// materialization, e.g. toArray() inside Fusion::run) and attach storage.
bool fusion_materialize(const TensorP &t);

// Eager implementations of native boundary ops (inputs materialized).
TensorP native_execute(const NativeSpec &spec, const std::vector<TensorP> &inputs);
}  // namespace phpt

// Opaque C handle of phpt_host.h: one reference to a tensor.
struct phpt_tensor {
    phpt::TensorP t;
};
