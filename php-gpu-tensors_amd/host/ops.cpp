// Eager op dispatch of the host runtime: validation, dtype promotion,
// result allocation and the C-ABI launch for every CudaArray operation on
// the hot path.  Follows src/cuda_array/ca_private.c (cuda_tensor_op,
// cuda_scalar_op, cuda_inv_scalar_op, cuda_unary_op, cuda_tensor_reduce,
// cuda_tensor_reduce_arg, cuda_tensor_moments_reduce, cuda_tensor_matmul)
// and the cuda_array_ce.c composites (variance :1850-1902, softmax
// :1942-2001, layerNorm :2215-2339), which here call the fused row kernels.
// Inside a Fusion scope every entry point records a node instead.
#include "runtime.hpp"

#include <math.h>
#include <string.h>

#include <algorithm>

namespace phpt {

// Strides of `t` aligned to an output of rank `nd` (leading dims and
// extent-1 dims get stride 0), as prepare_broadcast_operation
// (src/operations.c:9-30, 69-81).
static void aligned_strides(const Tensor &t, int nd, size_t *out)
{
    int off = nd - t.ndims;
    for (int d = 0; d < nd; d++) {
        int s = d - off;
        out[d] = (s < 0 || t.shape[s] == 1) ? 0 : t.strides[s];
    }
}

static bool guard(const TensorP &t)
{
    if (!t) {
        if (!error_kind()) set_invalid("Missing tensor operand");
        return false;
    }
    if (t->lazy() && !fusion_active() && !fusion_materialize(t)) return false;
    return true;
}

static void *base_ptr(const TensorP &t) { return t->storage ? t->storage->ptr : nullptr; }

// ------------------------------------------------------------- binary ops
TensorP cuda_tensor_op(const TensorP &a, const TensorP &b, int op)
{
    if (!a || !b) {
        set_invalid("Missing tensor operand");
        return nullptr;
    }
    int shape[kMaxDims], nd;
    if (!broadcast_shape(a->shape, a->ndims, b->shape, b->ndims, shape, &nd)) {
        set_invalid("Broadcast failed: operand shapes are incompatible");
        return nullptr;
    }
    int dt = promote_types_for_arithmetic(a->dtype, b->dtype, op);
    if (dt < 0) {
        set_invalid("No exact common dtype for %s and %s; cast operands explicitly",
                    dtype_name(a->dtype), dtype_name(b->dtype));
        return nullptr;
    }
    if (!can_safely_cast_to(a->dtype, dt)) {
        set_invalid("Cannot safely promote operand A (%s) to %s", dtype_name(a->dtype), dtype_name(dt));
        return nullptr;
    }
    if (!can_safely_cast_to(b->dtype, dt)) {
        set_invalid("Cannot safely promote operand B (%s) to %s", dtype_name(b->dtype), dtype_name(dt));
        return nullptr;
    }
    if (fusion_active()) return fusion_record(N_BINARY, op, {a, b}, shape, nd, dt);
    if (!guard(a) || !guard(b)) return nullptr;
    TensorP out = make_empty(shape, nd, dt);
    if (!out || !out->numel()) return out;
    size_t sa[kMaxDims], sb[kMaxDims];
    aligned_strides(*a, nd, sa);
    aligned_strides(*b, nd, sb);
    if (!check_status(pt_broadcast(base_ptr(a), a->dtype, sa, a->offset, base_ptr(b), b->dtype, sb,
                                   b->offset, out->storage->ptr, dt, op, shape, nd, nullptr),
                      "Broadcast kernel launch failed"))
        return nullptr;
    return out;
}

static TensorP scalar_impl(const TensorP &a, const Scalar &s, int op, bool reverse)
{
    if (!a) {
        set_invalid("Missing tensor operand");
        return nullptr;
    }
    int dt = promote_scalar_for_arithmetic(a->dtype, s.dtype, op, s.is_neg);
    Scalar cs;
    if (dt < 0 || !cast_scalar(s, dt, cs)) {
        set_invalid("Scalar cannot be represented by the promoted dtype; cast operands explicitly");
        return nullptr;
    }
    if (fusion_active()) return fusion_record_scalar(a, cs, op, reverse, dt);
    if (!guard(a)) return nullptr;
    TensorP out = make_empty(a->shape, a->ndims, dt);
    if (!out || !out->numel()) return out;
    pt_scalar_t ps = to_pt_scalar(cs);
    if (!check_status(pt_scalar(base_ptr(a), a->dtype, a->strides, a->offset, &ps, reverse ? 1 : 0,
                                out->storage->ptr, dt, op, a->shape, a->ndims, nullptr),
                      "Scalar kernel launch failed"))
        return nullptr;
    return out;
}

TensorP cuda_scalar_op(const TensorP &a, const Scalar &s, int op) { return scalar_impl(a, s, op, false); }
TensorP cuda_inv_scalar_op(const TensorP &a, const Scalar &s, int op) { return scalar_impl(a, s, op, true); }

TensorP cuda_unary_op(const TensorP &a, int op)
{
    if (!a) {
        set_invalid("Missing tensor operand");
        return nullptr;
    }
    if (fusion_active()) return fusion_record(N_UNARY, op, {a}, a->shape, a->ndims, a->dtype);
    if (!guard(a)) return nullptr;
    TensorP out = make_empty(a->shape, a->ndims, a->dtype);
    if (!out || !out->numel()) return out;
    if (!check_status(pt_unary(base_ptr(a), a->dtype, a->strides, a->offset, out->storage->ptr, op,
                               a->shape, a->ndims, nullptr),
                      "Unary kernel launch failed"))
        return nullptr;
    return out;
}

TensorP tensor_cast(const TensorP &a, int dtype)
{
    if (!a) return nullptr;
    if (a->dtype == dtype) return a;
    if (fusion_active()) return fusion_record(N_CAST, 0, {a}, a->shape, a->ndims, dtype);
    if (!guard(a)) return nullptr;
    TensorP out = make_empty(a->shape, a->ndims, dtype);
    if (!out || !out->numel()) return out;
    if (!check_status(pt_cast(base_ptr(a), a->dtype, a->strides, a->offset, out->storage->ptr, dtype,
                              a->shape, a->ndims, nullptr),
                      "Cast kernel launch failed"))
        return nullptr;
    return out;
}

TensorP astype(const TensorP &a, int dtype)
{
    if (!is_valid_dtype(dtype) || !can_safely_cast_to(a->dtype, dtype)) {
        set_invalid("Cannot safely cast from %s to %s", dtype_name(a->dtype),
                    is_valid_dtype(dtype) ? dtype_name(dtype) : "unknown");
        return nullptr;
    }
    return tensor_cast(a, dtype);
}

TensorP copy(const TensorP &a)
{
    if (!guard(a)) return nullptr;
    if (a->lazy()) return a;  // recorded values are already fresh buffers
    TensorP out = make_empty(a->shape, a->ndims, a->dtype);
    if (!out || !out->numel()) return out;
    if (!check_status(pt_cast(base_ptr(a), a->dtype, a->strides, a->offset, out->storage->ptr,
                              a->dtype, a->shape, a->ndims, nullptr), "copy"))
        return nullptr;
    return out;
}

TensorP cuda_tensor_where(const TensorP &c, const TensorP &x, const TensorP &y)
{
    if (!c || !x || !y) {
        set_invalid("Missing tensor operand");
        return nullptr;
    }
    if (x->dtype != y->dtype) {
        set_invalid("where requires x and y to have the same dtype");
        return nullptr;
    }
    int inter[kMaxDims], shape[kMaxDims], ni, nd;
    if (!broadcast_shape(x->shape, x->ndims, y->shape, y->ndims, inter, &ni) ||
        !broadcast_shape(c->shape, c->ndims, inter, ni, shape, &nd)) {
        set_invalid("where operands have incompatible shapes");
        return nullptr;
    }
    if (fusion_active()) return fusion_record(N_WHERE, 0, {c, x, y}, shape, nd, x->dtype);
    if (!guard(c) || !guard(x) || !guard(y)) return nullptr;
    TensorP out = make_empty(shape, nd, x->dtype);
    if (!out || !out->numel()) return out;
    size_t sc[kMaxDims], sx[kMaxDims], sy[kMaxDims];
    aligned_strides(*c, nd, sc);
    aligned_strides(*x, nd, sx);
    aligned_strides(*y, nd, sy);
    // pt_where takes operand base pointers already offset
    const char *pc = (const char *)base_ptr(c) + c->offset * dtype_size(c->dtype);
    const char *px = (const char *)base_ptr(x) + x->offset * dtype_size(x->dtype);
    const char *py = (const char *)base_ptr(y) + y->offset * dtype_size(y->dtype);
    if (!check_status(pt_where(pc, c->dtype, sc, px, sx, py, sy, x->dtype, out->storage->ptr, shape,
                               nd, nullptr),
                      "where kernel launch failed"))
        return nullptr;
    return out;
}

// ------------------------------------------------------------- indexed ops
// Device validation record of the Fusion plan being executed: while set,
// indexed natives record invalid indices there (one download per plan
// execution) instead of validating before they launch.
int32_t *&index_record()
{
    static thread_local int32_t *record = nullptr;
    return record;
}

// cuda_tensor_validate_indexed_shapes (ca_private.c:885-914)
static bool validate_indexed_shapes(const TensorP &input, const TensorP &indices, const TensorP &updates, int axis,
                                    const char *operation)
{
    if (!input || !indices || axis < 0 || axis >= input->ndims || indices->ndims != input->ndims ||
        indices->dtype != PT_INT32) {
        set_invalid("%s requires int32 indices with the same rank and a valid axis", operation);
        return false;
    }
    for (int d = 0; d < input->ndims; d++) {
        if (d != axis && input->shape[d] != indices->shape[d]) {
            set_invalid("%s input and index shapes must match outside the indexed axis", operation);
            return false;
        }
        if (updates && updates->shape[d] != indices->shape[d]) {
            set_invalid("%s updates must have the same shape as indices", operation);
            return false;
        }
    }
    if (updates && updates->dtype != input->dtype) {
        set_invalid("%s input and updates must have the same dtype", operation);
        return false;
    }
    return true;
}

// Eager validation (cuda_validate_indices before the launch): one device
// pass, then a 12-byte download of the record.
static bool validate_indices(const TensorP &indices, int axis, int axis_size, const char *operation)
{
    if (!indices->numel()) return true;
    void *rec = nullptr;
    if (!check_status(pt_alloc(&rec, 3 * sizeof(int32_t), nullptr), "Failed to validate indices")) return false;
    int32_t host[3] = {0, 0, 0};
    bool ok = check_status(pt_index_validate((const int32_t *)base_ptr(indices), indices->shape, indices->strides,
                                             indices->offset, indices->ndims, axis, axis_size, (int32_t *)rec,
                                             nullptr),
                           "Failed to validate indices") &&
              check_status(pt_memcpy_d2h(host, rec, sizeof(host), nullptr), "Failed to validate indices");
    pt_free(rec, nullptr);
    if (ok && host[0] != 0) {
        set_invalid("%s indices must be within [0, %d)", operation, axis_size);
        return false;
    }
    return ok;
}

TensorP cuda_tensor_gather(const TensorP &input, const TensorP &indices, int axis)
{
    if (!validate_indexed_shapes(input, indices, nullptr, axis, "gather")) return nullptr;
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_GATHER;
        sp.axis = axis;
        return fusion_record_native(sp, {input, indices}, indices->shape, indices->ndims, input->dtype);
    }
    if (!guard(input) || !guard(indices)) return nullptr;
    int32_t *record = index_record();
    if (!record && !validate_indices(indices, axis, input->shape[axis], "gather")) return nullptr;
    TensorP out = output_tensor(indices->shape, indices->ndims, input->dtype);
    if (!out || !out->numel()) return out;
    if (!check_status(pt_gather(base_ptr(input), input->dtype, input->shape, input->strides, input->offset,
                                (const int32_t *)base_ptr(indices), indices->shape, indices->strides,
                                indices->offset, input->ndims, axis, out->storage->ptr, record, nullptr),
                      "gather kernel failed"))
        return nullptr;
    return out;
}

TensorP cuda_tensor_scatter_add(const TensorP &input, const TensorP &indices, const TensorP &updates, int axis)
{
    if (!validate_indexed_shapes(input, indices, updates, axis, "scatterAdd")) return nullptr;
    // float16 / bfloat16 run in float32 (ca_private.c:957-968): the result is float32
    const bool low = input->dtype == PT_FLOAT16 || input->dtype == PT_BFLOAT16;
    const int dt = low ? PT_FLOAT32 : input->dtype;
    if (dt != PT_FLOAT32 && dt != PT_FLOAT64) {
        set_invalid("scatterAdd currently supports float32 and float64 tensors");
        return nullptr;
    }
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_SCATTER_ADD;
        sp.axis = axis;
        return fusion_record_native(sp, {input, indices, updates}, input->shape, input->ndims, dt);
    }
    if (!guard(input) || !guard(indices) || !guard(updates)) return nullptr;
    TensorP in = input, up = updates;
    if (low) {
        in = tensor_cast(input, PT_FLOAT32);
        up = in ? tensor_cast(updates, PT_FLOAT32) : nullptr;
        if (!up) return nullptr;
    }
    int32_t *record = index_record();
    if (!record && !validate_indices(indices, axis, input->shape[axis], "scatterAdd")) return nullptr;
    TensorP out = output_tensor(in->shape, in->ndims, dt);
    if (!out || !out->numel()) return out;
    // the input's values first (cuda_launch_scatter_copy), then the adds
    if (!check_status(pt_cast(base_ptr(in), dt, in->strides, in->offset, out->storage->ptr, dt, in->shape, in->ndims,
                              nullptr),
                      "scatterAdd kernel failed") ||
        !check_status(pt_scatter_add((const int32_t *)base_ptr(indices), indices->shape, indices->strides,
                                     indices->offset, base_ptr(up), up->strides, up->offset, dt, in->ndims, axis,
                                     in->shape[axis], out->storage->ptr, out->strides, record, nullptr),
                      "scatterAdd kernel failed"))
        return nullptr;
    return out;
}

// ------------------------------------------------------------- reductions
// calculate_reduction_shape (src/operations.c:37-67)
static int reduction_shape(const Tensor &t, int axis, int *shape)
{
    if (axis == kGlobalAxis) {
        shape[0] = 1;
        return 1;
    }
    int j = 0;
    for (int d = 0; d < t.ndims; d++)
        if (d != axis) shape[j++] = t.shape[d];
    if (!j) {
        shape[0] = 1;
        j = 1;
    }
    return j;
}

static bool check_axis(const Tensor &t, int axis)
{
    if (axis == kGlobalAxis) return true;
    if (axis < 0 || axis >= t.ndims) {
        set_invalid("Invalid axis %d for reduction operation. Must be between 0 and %d.", axis,
                    t.ndims - 1);
        return false;
    }
    return true;
}

TensorP cuda_tensor_reduce(const TensorP &a, int axis, int op)
{
    if (!a || !check_axis(*a, axis)) return nullptr;
    int rdt = pt_reduce_result_dtype(a->dtype, op);
    if (rdt < 0) {
        set_invalid("Unsupported reduction");
        return nullptr;
    }
    int shape[kMaxDims];
    int nd = reduction_shape(*a, axis, shape);
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_REDUCE;
        sp.op = op;
        sp.axis = axis;
        return fusion_record_native(sp, {a}, shape, nd, rdt);
    }
    if (!guard(a)) return nullptr;
    TensorP out = output_tensor(shape, nd, rdt);
    if (!out) return nullptr;
    if (!check_status(pt_reduce(base_ptr(a), out->storage->ptr, a->dtype, op, a->shape, a->strides,
                                a->ndims, axis == kGlobalAxis ? -1 : axis, a->offset, nullptr),
                      "Reduction kernel launch failed"))
        return nullptr;
    return out;
}

TensorP cuda_tensor_reduce_arg(const TensorP &a, int axis, int op)
{
    if (!a || !check_axis(*a, axis)) return nullptr;
    if (axis == kGlobalAxis && a->numel() > (size_t)INT32_MAX) {
        set_invalid("Global arg reduction requires at most INT_MAX elements");
        return nullptr;
    }
    int shape[kMaxDims];
    int nd = reduction_shape(*a, axis, shape);
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_ARG_REDUCE;
        sp.op = op;
        sp.axis = axis;
        return fusion_record_native(sp, {a}, shape, nd, PT_INT32);
    }
    if (!guard(a)) return nullptr;
    TensorP out = output_tensor(shape, nd, PT_INT32);
    if (!out) return nullptr;
    if (!check_status(pt_arg_reduce(base_ptr(a), (int32_t *)out->storage->ptr, a->dtype, op, a->shape,
                                    a->strides, a->ndims, axis == kGlobalAxis ? -1 : axis, a->offset,
                                    nullptr),
                      "Arg reduction kernel launch failed"))
        return nullptr;
    return out;
}

TensorP cuda_array_variance(const TensorP &a, int axis, long correction, bool std_dev)
{
    if (!a || !check_axis(*a, axis)) return nullptr;
    size_t count = axis == kGlobalAxis ? a->numel() : (size_t)a->shape[axis];
    if (correction < 0 || (size_t)correction >= count) {
        set_invalid("Variance correction must be non-negative and smaller than the reduced dimension");
        return nullptr;
    }
    int rdt = (a->dtype == PT_FLOAT32 || a->dtype == PT_FLOAT16 || a->dtype == PT_BFLOAT16)
              ? PT_FLOAT32 : PT_FLOAT64;
    int shape[kMaxDims];
    int nd = reduction_shape(*a, axis, shape);
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_MOMENTS;
        sp.axis = axis;
        sp.correction = correction;
        sp.std_dev = std_dev;
        return fusion_record_native(sp, {a}, shape, nd, rdt);
    }
    if (!guard(a)) return nullptr;
    TensorP src = a;
    if (a->offset) {
        src = materialize(a);
        if (!src) return nullptr;
    }
    TensorP out = output_tensor(shape, nd, rdt);
    if (!out) return nullptr;
    if (!check_status(pt_moments(base_ptr(src), out->storage->ptr, src->dtype, rdt, src->shape,
                                 src->strides, src->ndims, axis == kGlobalAxis ? -1 : axis,
                                 (int)correction, std_dev ? 1 : 0, nullptr),
                      "Variance reduction kernel failed"))
        return nullptr;
    return out;
}

TensorP cuda_array_softmax(const TensorP &a, int axis)
{
    if (!a) return nullptr;
    if (axis < 0 || axis >= a->ndims) {
        set_invalid("Softmax axis is out of range for tensor rank %d", a ? a->ndims : 0);
        return nullptr;
    }
    int odt = (a->dtype == PT_FLOAT64 || is_integer(a->dtype) || a->dtype == PT_BOOL) ? PT_FLOAT64
                                                                                     : PT_FLOAT32;
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_SOFTMAX;
        sp.axis = axis;
        return fusion_record_native(sp, {a}, a->shape, a->ndims, odt);
    }
    if (!guard(a)) return nullptr;
    TensorP src = a;
    if (!is_floating(a->dtype)) {
        src = tensor_cast(a, PT_FLOAT64);
        if (!src) return nullptr;
    }
    if (src->offset) {
        src = materialize(src);
        if (!src) return nullptr;
    }
    TensorP out = output_tensor(a->shape, a->ndims, odt);
    if (!out) return nullptr;
    if (!check_status(pt_softmax(base_ptr(src), out->storage->ptr, src->dtype, odt, src->shape,
                                 src->strides, src->ndims, axis, nullptr),
                      "Softmax kernel failed"))
        return nullptr;
    return out;
}

// cuda_array_layernorm (cuda_array_ce.c:2215-2339) with validation
// (:2037-2087 axes, :2131-2155 parameters, :2219-2247 eps / dtype).
TensorP cuda_array_layernorm(const TensorP &a, const int *axes_in, int naxes, double eps,
                             const TensorP &scale, const TensorP &bias)
{
    if (!a) return nullptr;
    if (naxes <= 0 || naxes > a->ndims) {
        set_invalid("LayerNorm requires a non-empty list of distinct axes");
        return nullptr;
    }
    int axes[kMaxDims];
    int seen[kMaxDims] = {0};
    for (int i = 0; i < naxes; i++) {
        int ax = axes_in[i] < 0 ? axes_in[i] + a->ndims : axes_in[i];
        if (ax < 0 || ax >= a->ndims) {
            set_invalid("LayerNorm axis is out of range for tensor rank %d", a->ndims);
            return nullptr;
        }
        if (seen[ax]) {
            set_invalid("LayerNorm axes must not contain duplicates");
            return nullptr;
        }
        seen[ax] = 1;
        axes[i] = ax;
    }
    if (!isfinite(eps) || eps <= 0.0) {
        set_invalid("LayerNorm epsilon must be finite and greater than zero");
        return nullptr;
    }
    for (int i = 0; i < naxes; i++)
        if (!a->shape[axes[i]]) {
            set_invalid("LayerNorm cannot normalize an empty dimension");
            return nullptr;
        }
    const TensorP *params[2] = {&scale, &bias};
    const char *pname[2] = {"scale", "bias"};
    for (int p = 0; p < 2; p++) {
        const TensorP &t = *params[p];
        if (!t) continue;
        if (!is_floating(t->dtype)) {
            set_invalid("LayerNorm %s must have a floating-point dtype", pname[p]);
            return nullptr;
        }
        if (t->ndims != naxes) {
            set_invalid("LayerNorm %s rank must match the number of normalized axes", pname[p]);
            return nullptr;
        }
        for (int i = 0; i < naxes; i++)
            if (t->shape[i] != a->shape[axes[i]]) {
                set_invalid("LayerNorm %s shape does not match the normalized dimensions", pname[p]);
                return nullptr;
            }
    }
    int cdt = (a->dtype == PT_FLOAT64 || !is_floating(a->dtype)) ? PT_FLOAT64 : PT_FLOAT32;
    if ((scale && scale->dtype == PT_FLOAT64) || (bias && bias->dtype == PT_FLOAT64)) cdt = PT_FLOAT64;
    if (cdt == PT_FLOAT32 && (!isfinite((float)eps) || (float)eps <= 0.0f)) {
        set_invalid("LayerNorm epsilon is not representable as float32");
        return nullptr;
    }
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_LAYERNORM;
        sp.eps = eps;
        sp.naxes = naxes;
        for (int i = 0; i < naxes; i++) sp.axes[i] = axes[i];
        sp.has_scale = scale != nullptr;
        sp.has_bias = bias != nullptr;
        std::vector<TensorP> ins = {a};
        if (scale) ins.push_back(scale);
        if (bias) ins.push_back(bias);
        return fusion_record_native(sp, ins, a->shape, a->ndims, cdt);
    }
    if (!guard(a) || (scale && !guard(scale)) || (bias && !guard(bias))) return nullptr;

    // normalized axes in ascending order go last; the rest keep their order
    int sorted[kMaxDims];
    for (int i = 0; i < naxes; i++) sorted[i] = axes[i];
    std::sort(sorted, sorted + naxes);
    int perm[kMaxDims], k = 0;
    for (int d = 0; d < a->ndims; d++)
        if (!seen[d]) perm[k++] = d;
    for (int i = 0; i < naxes; i++) perm[k++] = sorted[i];
    bool identity = true;
    for (int d = 0; d < a->ndims; d++) identity = identity && perm[d] == d;

    TensorP x = a;
    if (!is_floating(x->dtype)) {
        x = tensor_cast(x, PT_FLOAT64);
        if (!x) return nullptr;
    } else if (x->dtype != PT_FLOAT64 && cdt == PT_FLOAT64 && x->dtype != PT_FLOAT32) {
        x = tensor_cast(x, PT_FLOAT64);
        if (!x) return nullptr;
    }
    TensorP xp = identity ? x : transpose(x, perm, a->ndims);
    if (!xp) return nullptr;
    xp = materialize(xp);
    if (!xp) return nullptr;
    size_t n = 1;
    for (int i = 0; i < naxes; i++) n *= (size_t)a->shape[sorted[i]];
    size_t rows = n ? a->numel() / n : 0;

    // parameters: dims follow `axes`; reorder them to ascending-axis order
    auto prep = [&](const TensorP &p) -> TensorP {
        if (!p) return nullptr;
        int pperm[kMaxDims];
        for (int i = 0; i < naxes; i++)
            for (int j = 0; j < naxes; j++)
                if (axes[j] == sorted[i]) pperm[i] = j;
        TensorP q = tensor_cast(p, cdt);
        if (!q) return nullptr;
        q = transpose(q, pperm, naxes);
        if (!q) return nullptr;
        return materialize(q);
    };
    TensorP g = prep(scale), b = prep(bias);
    if ((scale && !g) || (bias && !b)) return nullptr;

    int pshape[kMaxDims];
    for (int d = 0; d < a->ndims; d++) pshape[d] = a->shape[perm[d]];
    TensorP outp = identity ? output_tensor(pshape, a->ndims, cdt) : make_empty(pshape, a->ndims, cdt);
    if (!outp) return nullptr;
    if (rows && !check_status(pt_layernorm(xp->data(), outp->storage->ptr, xp->dtype, cdt, rows, n, eps,
                                           g ? g->data() : nullptr, b ? b->data() : nullptr, nullptr),
                              "LayerNorm kernel failed"))
        return nullptr;
    if (identity) return outp;
    int inv[kMaxDims];
    for (int d = 0; d < a->ndims; d++) inv[perm[d]] = d;
    TensorP back = transpose(outp, inv, a->ndims);
    if (!back) return nullptr;
    return materialize(back);
}

// ------------------------------------------------------------------ matmul
TensorP cuda_tensor_matmul(const TensorP &a, const TensorP &b)
{
    if (!a || !b) {
        set_invalid("Missing tensor operand");
        return nullptr;
    }
    if (a->dtype != b->dtype ||
        (a->dtype != PT_FLOAT32 && a->dtype != PT_FLOAT16 && a->dtype != PT_BFLOAT16)) {
        set_invalid("matmul requires matching float32, float16 or bfloat16 operands");
        return nullptr;
    }
    int shape[kMaxDims], nd;
    if (!matmul_shape(a->shape, a->ndims, b->shape, b->ndims, shape, &nd)) {
        set_invalid("matmul requires rank >= 2, matching inner dimensions and broadcast-compatible batches");
        return nullptr;
    }
    if (fusion_active()) {
        NativeSpec sp;
        sp.kind = NAT_MATMUL;
        return fusion_record_native(sp, {a, b}, shape, nd, a->dtype);
    }
    if (!guard(a) || !guard(b)) return nullptr;
    TensorP out = output_tensor(shape, nd, a->dtype);
    if (!out) return nullptr;
    const char *pa = (const char *)base_ptr(a) + a->offset * dtype_size(a->dtype);
    const char *pb = (const char *)base_ptr(b) + b->offset * dtype_size(b->dtype);
    if (!check_status(pt_matmul(pa, pb, out->storage->ptr, a->dtype, a->shape, a->strides, a->ndims,
                                b->shape, b->strides, b->ndims, shape, nd, nullptr),
                      "Matmul backend submission failed"))
        return nullptr;
    return out;
}

// cuda_tune_matmul (matmul_kernels.h:34-38): a measured tile choice kept
// for this problem by the device library; eager only
TensorP cuda_tune_matmul(const TensorP &a, const TensorP &b, int *tiles, float *median_ms, int max_candidates,
                         int *count, int *selected)
{
    if (!a || !b) {
        set_invalid("Missing tensor operand");
        return nullptr;
    }
    if (fusion_active()) {
        set_runtime("matmul tuning cannot run inside a Fusion scope");
        return nullptr;
    }
    if (a->dtype != b->dtype ||
        (a->dtype != PT_FLOAT32 && a->dtype != PT_FLOAT16 && a->dtype != PT_BFLOAT16)) {
        set_invalid("matmul requires matching float32, float16 or bfloat16 operands");
        return nullptr;
    }
    int shape[kMaxDims], nd;
    if (!matmul_shape(a->shape, a->ndims, b->shape, b->ndims, shape, &nd)) {
        set_invalid("matmul requires rank >= 2, matching inner dimensions and broadcast-compatible batches");
        return nullptr;
    }
    if (!guard(a) || !guard(b)) return nullptr;
    TensorP out = output_tensor(shape, nd, a->dtype);
    if (!out) return nullptr;
    const char *pa = (const char *)base_ptr(a) + a->offset * dtype_size(a->dtype);
    const char *pb = (const char *)base_ptr(b) + b->offset * dtype_size(b->dtype);
    if (!check_status(pt_matmul_tune(pa, pb, out->storage->ptr, a->dtype, a->shape, a->strides, a->ndims,
                                     b->shape, b->strides, b->ndims, shape, nd, tiles, median_ms, max_candidates,
                                     count, selected, nullptr),
                      "Matmul tuning failed"))
        return nullptr;
    return out;
}

// ------------------------------------------------------- native dispatcher
TensorP native_execute(const NativeSpec &sp, const std::vector<TensorP> &in)
{
    switch (sp.kind) {
    case NAT_MATMUL: return cuda_tensor_matmul(in[0], in[1]);
    case NAT_REDUCE: return cuda_tensor_reduce(in[0], sp.axis, sp.op);
    case NAT_ARG_REDUCE: return cuda_tensor_reduce_arg(in[0], sp.axis, sp.op);
    case NAT_MOMENTS: return cuda_array_variance(in[0], sp.axis, sp.correction, sp.std_dev);
    case NAT_SOFTMAX: return cuda_array_softmax(in[0], sp.axis);
    case NAT_GATHER: return cuda_tensor_gather(in[0], in[1], sp.axis);
    case NAT_SCATTER_ADD: return cuda_tensor_scatter_add(in[0], in[1], in[2], sp.axis);
    case NAT_LAYERNORM: {
        size_t k = 1;
        TensorP scale = sp.has_scale ? in[k++] : nullptr;
        TensorP bias = sp.has_bias ? in[k++] : nullptr;
        return cuda_array_layernorm(in[0], sp.axes, sp.naxes, sp.eps, scale, bias);
    }
    default:
        set_runtime("Unknown native step");
        return nullptr;
    }
}

}  // namespace phpt
