// C API of the host runtime (phpt_host.h): handle management, transfers,
// views and operations.  Views of values recorded inside a Fusion scope
// become view nodes; everything else goes straight to runtime.hpp.
#include "phpt_host.h"
#include "runtime.hpp"

#include <limits.h>

#include <string.h>

using namespace phpt;

static phpt_tensor *wrap(const TensorP &t)
{
    if (!t) return nullptr;
    auto *h = new phpt_tensor;
    h->t = t;
    return h;
}

static Scalar make_scalar(double value, int64_t ivalue, int kind)
{
    if (kind == 1) return scalar_from_int(ivalue);
    if (kind == 2) return scalar_from_bool(ivalue != 0);
    return scalar_from_double(value);
}

// View of a recorded (lazy) value: strides are relative to the value's
// contiguous logical layout.
static phpt_tensor *lazy_view(const TensorP &t, const int *shape, const size_t *strides, int nd, size_t off)
{
    return wrap(fusion_record_view(t, shape, strides, nd, off));
}

extern "C" {

int phpt_error_kind(void) { return error_kind(); }
const char *phpt_error_message(void) { return error_message(); }
void phpt_clear_error(void) { clear_error(); }

phpt_tensor *phpt_from_host(const void *data, int dtype, const int *shape, int ndims)
{
    clear_error();
    if (!is_valid_dtype(dtype)) {
        set_invalid("Unknown dtype");
        return nullptr;
    }
    return wrap(from_host(data, shape, ndims, dtype));
}

phpt_tensor *phpt_full(const int *shape, int ndims, int dtype, double value, int64_t ivalue, int kind)
{
    clear_error();
    Scalar s = make_scalar(value, ivalue, kind), cs;
    if (!cast_scalar(s, dtype, cs)) {
        set_invalid("Fill value cannot be represented as %s", dtype_name(dtype));
        return nullptr;
    }
    return wrap(full(shape, ndims, dtype, cs));
}

int phpt_to_host(phpt_tensor *t, void *out, size_t bytes)
{
    clear_error();
    if (t->t->lazy() && !fusion_materialize(t->t)) return -1;
    return to_host(t->t, out, bytes) ? 0 : -1;
}

phpt_tensor *phpt_retain(phpt_tensor *t) { return wrap(t->t); }
void phpt_release(phpt_tensor *t) { delete t; }
int phpt_dtype(phpt_tensor *t) { return t->t->dtype; }
int phpt_ndims(phpt_tensor *t) { return t->t->ndims; }
void phpt_shape(phpt_tensor *t, int *shape)
{
    for (int d = 0; d < t->t->ndims; d++) shape[d] = t->t->shape[d];
}
void phpt_strides(phpt_tensor *t, size_t *strides)
{
    for (int d = 0; d < t->t->ndims; d++) strides[d] = t->t->strides[d];
}
size_t phpt_size(phpt_tensor *t) { return t->t->numel(); }
int phpt_is_lazy(phpt_tensor *t) { return t->t->lazy() ? 1 : 0; }
int phpt_is_view(phpt_tensor *t) { return t->t->is_view ? 1 : 0; }
const void *phpt_device_pointer(phpt_tensor *t) { return t->t->lazy() ? nullptr : t->t->data(); }
int phpt_dtype_from_name(const char *name) { return dtype_from_name(name); }
const char *phpt_dtype_name(int dtype) { return dtype_name(dtype); }

// ------------------------------------------------------------------ views
phpt_tensor *phpt_reshape(phpt_tensor *h, const int *shape, int ndims)
{
    clear_error();
    const TensorP &t = h->t;
    if (t->lazy()) {
        // resolve -1 and check the element count like the eager path
        int sh[kMaxDims];
        size_t known = 1;
        int infer = -1;
        for (int d = 0; d < ndims; d++) {
            sh[d] = shape[d];
            if (shape[d] == -1) infer = d;
            else known *= (size_t)shape[d];
        }
        if (infer >= 0 && known) sh[infer] = (int)(t->numel() / known);
        size_t n = 1;
        for (int d = 0; d < ndims; d++) n *= (size_t)sh[d];
        if (n != t->numel()) {
            set_invalid("Reshape requires that the number of elements remains the same");
            return nullptr;
        }
        size_t st[kMaxDims];
        contiguous_strides(sh, ndims, st);
        return lazy_view(t, sh, st, ndims, 0);
    }
    return wrap(reshape(t, shape, ndims));
}

phpt_tensor *phpt_transpose(phpt_tensor *h, const int *perm, int nperm)
{
    clear_error();
    const TensorP &t = h->t;
    if (t->lazy()) {
        size_t cs[kMaxDims];
        contiguous_strides(t->shape, t->ndims, cs);
        TensorP meta = make_meta(t->shape, t->ndims, t->dtype);
        for (int d = 0; d < t->ndims; d++) meta->strides[d] = cs[d];
        meta->storage = std::make_shared<Storage>();  // metadata-only stand-in for the view math
        TensorP v = transpose(meta, perm, nperm);
        meta->storage.reset();
        if (!v) return nullptr;
        return lazy_view(t, v->shape, v->strides, v->ndims, v->offset);
    }
    return wrap(transpose(t, perm, nperm));
}

phpt_tensor *phpt_broadcast_to(phpt_tensor *h, const int *shape, int ndims)
{
    clear_error();
    const TensorP &t = h->t;
    if (t->lazy()) {
        TensorP meta = make_meta(t->shape, t->ndims, t->dtype);
        meta->storage = std::make_shared<Storage>();
        TensorP v = broadcast_to(meta, shape, ndims);
        meta->storage.reset();
        if (!v) return nullptr;
        return lazy_view(t, v->shape, v->strides, v->ndims, v->offset);
    }
    return wrap(broadcast_to(t, shape, ndims));
}

phpt_tensor *phpt_slice(phpt_tensor *h, int axis, int start, int stop, int step)
{
    clear_error();
    const TensorP &t = h->t;
    if (t->lazy()) {
        TensorP meta = make_meta(t->shape, t->ndims, t->dtype);
        meta->storage = std::make_shared<Storage>();
        TensorP v = slice_axis(meta, axis, start, stop, step);
        meta->storage.reset();
        if (!v) return nullptr;
        return lazy_view(t, v->shape, v->strides, v->ndims, v->offset);
    }
    return wrap(slice_axis(t, axis, start, stop, step));
}

phpt_tensor *phpt_select(phpt_tensor *h, int axis, int index)
{
    clear_error();
    const TensorP &t = h->t;
    if (t->lazy()) {
        TensorP meta = make_meta(t->shape, t->ndims, t->dtype);
        meta->storage = std::make_shared<Storage>();
        TensorP v = select_index(meta, axis, index);
        meta->storage.reset();
        if (!v) return nullptr;
        return lazy_view(t, v->shape, v->strides, v->ndims, v->offset);
    }
    return wrap(select_index(t, axis, index));
}

// ------------------------------------------------------------- operations
phpt_tensor *phpt_binary(phpt_tensor *a, phpt_tensor *b, int op)
{
    clear_error();
    return wrap(cuda_tensor_op(a->t, b->t, op));
}

phpt_tensor *phpt_scalar_op(phpt_tensor *a, double value, int64_t ivalue, int kind, int op, int reverse)
{
    clear_error();
    Scalar s = make_scalar(value, ivalue, kind);
    return wrap(reverse ? cuda_inv_scalar_op(a->t, s, op) : cuda_scalar_op(a->t, s, op));
}

phpt_tensor *phpt_unary(phpt_tensor *a, int op)
{
    clear_error();
    return wrap(cuda_unary_op(a->t, op));
}

static int normalize_axis(const TensorP &t, int axis, bool *ok)
{
    *ok = true;
    if (axis == PHPT_GLOBAL_AXIS) return kGlobalAxis;
    int a = axis < 0 ? axis + t->ndims : axis;
    if (a < 0 || a >= t->ndims) {
        set_invalid("Axis %d out of bounds for tensor with %d dimensions", axis, t->ndims);
        *ok = false;
    }
    return a;
}

phpt_tensor *phpt_reduce(phpt_tensor *a, int axis, int op)
{
    clear_error();
    bool ok;
    int ax = normalize_axis(a->t, axis, &ok);
    if (!ok) return nullptr;
    return wrap(cuda_tensor_reduce(a->t, ax, op));
}

phpt_tensor *phpt_reduce_arg(phpt_tensor *a, int axis, int op)
{
    clear_error();
    bool ok;
    int ax = normalize_axis(a->t, axis, &ok);
    if (!ok) return nullptr;
    return wrap(cuda_tensor_reduce_arg(a->t, ax, op));
}

phpt_tensor *phpt_variance(phpt_tensor *a, int axis, long correction, int std_dev)
{
    clear_error();
    bool ok;
    int ax = normalize_axis(a->t, axis, &ok);
    if (!ok) return nullptr;
    return wrap(cuda_array_variance(a->t, ax, correction, std_dev != 0));
}

phpt_tensor *phpt_softmax(phpt_tensor *a, int axis)
{
    clear_error();
    int ax = axis < 0 ? axis + a->t->ndims : axis;
    if (ax < 0 || ax >= a->t->ndims) {
        set_invalid("Softmax axis is out of range for tensor rank %d", a->t->ndims);
        return nullptr;
    }
    return wrap(cuda_array_softmax(a->t, ax));
}

phpt_tensor *phpt_layernorm(phpt_tensor *a, const int *axes, int naxes, double eps, phpt_tensor *scale,
                            phpt_tensor *bias)
{
    clear_error();
    return wrap(cuda_array_layernorm(a->t, axes, naxes, eps, scale ? scale->t : nullptr,
                                     bias ? bias->t : nullptr));
}

phpt_tensor *phpt_matmul(phpt_tensor *a, phpt_tensor *b)
{
    clear_error();
    return wrap(cuda_tensor_matmul(a->t, b->t));
}

phpt_tensor *phpt_tune_matmul(phpt_tensor *a, phpt_tensor *b, int *tiles, float *median_ms,
                              int max_candidates, int *count, int *selected)
{
    clear_error();
    return wrap(cuda_tune_matmul(a->t, b->t, tiles, median_ms, max_candidates, count, selected));
}

phpt_tensor *phpt_where(phpt_tensor *c, phpt_tensor *x, phpt_tensor *y)
{
    clear_error();
    return wrap(cuda_tensor_where(c->t, x->t, y->t));
}

// cuda_array_index_axis (cuda_array_ce.c:2405-2421): negative axes count
// from the end
static bool index_axis(const TensorP &t, long long requested, int *axis)
{
    if (requested < INT_MIN || requested > INT_MAX) {
        set_invalid("Indexed operation axis is outside the supported integer range");
        return false;
    }
    int normalized = (int)requested;
    if (normalized < 0) normalized += t->ndims;
    if (normalized < 0 || normalized >= t->ndims) {
        set_invalid("Indexed operation axis is out of range for tensor rank %d", t->ndims);
        return false;
    }
    *axis = normalized;
    return true;
}

phpt_tensor *phpt_gather(phpt_tensor *a, phpt_tensor *indices, long long axis)
{
    clear_error();
    int ax;
    if (!index_axis(a->t, axis, &ax)) return nullptr;
    return wrap(cuda_tensor_gather(a->t, indices->t, ax));
}

phpt_tensor *phpt_scatter_add(phpt_tensor *a, phpt_tensor *indices, phpt_tensor *updates, long long axis)
{
    clear_error();
    int ax;
    if (!index_axis(a->t, axis, &ax)) return nullptr;
    return wrap(cuda_tensor_scatter_add(a->t, indices->t, updates->t, ax));
}

phpt_tensor *phpt_astype(phpt_tensor *a, int dtype)
{
    clear_error();
    return wrap(astype(a->t, dtype));
}

phpt_tensor *phpt_copy(phpt_tensor *a)
{
    clear_error();
    return wrap(copy(a->t));
}

}  // extern "C"
