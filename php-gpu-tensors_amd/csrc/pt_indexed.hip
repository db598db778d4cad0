// Indexed operations along one axis for gfx950: index validation, gather
// and scatter-add (the reference's src/backends/cuda/indexed_ops.cu
// launchers cuda_validate_indices, cuda_launch_gather,
// cuda_launch_scatter_copy and cuda_launch_scatter_add).
//
//   gather:      out[c] = input[c with c[axis] := indices[c]]   (c over the index shape)
//   scatter-add: out = copy of input; out[c with c[axis] := indices[c]] += updates[c]
//
// Indices are int32.  An index outside [0, axis_size) is an error: the
// eager path validates every index first (pt_index_validate: one pass, then
// a 12-byte download), a Fusion plan instead passes a device validation
// record that the kernels fill with the first offending index, so that one
// download per plan execution reports it (fusion_execute.c:204-224, 755-775).
// Index arithmetic is 32-bit when every offset fits, else 64-bit.
#include "pt_common.h"

#include <string.h>

namespace pt {

// validation record {operation, index, axis_size}; operation 0 = valid
enum { IDX_VALID = 0, IDX_GATHER_INVALID = 1, IDX_SCATTER_ADD_INVALID = 2 };

template <typename I>
struct IdxParams {
    int ndims, axis, axis_size;
    int shape[PT_MAX_DIMS];   // index shape (= gather output shape)
    I in_str[PT_MAX_DIMS];    // input / output strides
    I ix_str[PT_MAX_DIMS];    // index strides
    I up_str[PT_MAX_DIMS];    // update strides (scatter-add)
};

__device__ __forceinline__ void record_invalid(int32_t *v, int op, int index, int axis_size)
{
    if (v && atomicCAS(v, IDX_VALID, op) == IDX_VALID) {
        v[1] = index;
        v[2] = axis_size;
    }
}

template <typename I>
__global__ __launch_bounds__(256) void k_index_validate(const int32_t *__restrict__ idx, IdxParams<I> p, I total,
                                                         int32_t *v, int op)
{
    for (I f = (I)blockIdx.x * 256 + threadIdx.x; f < total; f += (I)gridDim.x * 256) {
        I rem = f, xo = 0;
        for (int d = p.ndims - 1; d >= 0; d--) {
            const I c = rem % (I)p.shape[d];
            rem /= (I)p.shape[d];
            xo += c * p.ix_str[d];
        }
        const int sel = idx[xo];
        if (sel < 0 || sel >= p.axis_size) record_invalid(v, op, sel, p.axis_size);
    }
}

template <typename T, typename I>
__global__ __launch_bounds__(256) void k_gather(const T *__restrict__ in, const int32_t *__restrict__ idx,
                                                 T *__restrict__ out, IdxParams<I> p, I total, int32_t *v)
{
    for (I f = (I)blockIdx.x * 256 + threadIdx.x; f < total; f += (I)gridDim.x * 256) {
        I rem = f, xo = 0, io = 0;
        for (int d = p.ndims - 1; d >= 0; d--) {
            const I c = rem % (I)p.shape[d];
            rem /= (I)p.shape[d];
            xo += c * p.ix_str[d];
            if (d != p.axis) io += c * p.in_str[d];
        }
        const int sel = idx[xo];
        if (sel < 0 || sel >= p.axis_size) {
            record_invalid(v, IDX_GATHER_INVALID, sel, p.axis_size);
            out[f] = T{};
        } else {
            out[f] = in[io + (I)sel * p.in_str[p.axis]];
        }
    }
}

template <typename T, typename I>
__global__ __launch_bounds__(256) void k_scatter_add(const int32_t *__restrict__ idx, const T *__restrict__ upd,
                                                      T *out, IdxParams<I> p, I total, int32_t *v)
{
    for (I f = (I)blockIdx.x * 256 + threadIdx.x; f < total; f += (I)gridDim.x * 256) {
        I rem = f, xo = 0, uo = 0, oo = 0;
        for (int d = p.ndims - 1; d >= 0; d--) {
            const I c = rem % (I)p.shape[d];
            rem /= (I)p.shape[d];
            xo += c * p.ix_str[d];
            uo += c * p.up_str[d];
            if (d != p.axis) oo += c * p.in_str[d];
        }
        const int sel = idx[xo];
        if (sel < 0 || sel >= p.axis_size) record_invalid(v, IDX_SCATTER_ADD_INVALID, sel, p.axis_size);
        else atomicAdd(out + oo + (I)sel * p.in_str[p.axis], upd[uo]);
    }
}

// clears a validation record (a kernel, not a memset node, so that the
// call can sit in a captured graph)
__global__ void k_record_reset(int32_t *v)
{
    if (threadIdx.x < 3) v[threadIdx.x] = 0;
}

static unsigned idx_grid(long long total)
{
    long long b = (total + 255) / 256;
    return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

// Largest element offset any of the strided operands can reach.
static long long max_offset(const int *shape, int ndims, const size_t *strides)
{
    long long m = 0;
    for (int d = 0; d < ndims; d++)
        if (shape[d] > 0) m += (long long)(shape[d] - 1) * (long long)(strides ? strides[d] : 0);
    return m;
}

template <typename I>
static void fill_params(IdxParams<I> &p, const int *shape, int ndims, int axis, int axis_size,
                        const size_t *in_str, const size_t *ix_str, const size_t *up_str)
{
    memset(&p, 0, sizeof(p));
    p.ndims = ndims;
    p.axis = axis;
    p.axis_size = axis_size;
    for (int d = 0; d < ndims; d++) {
        p.shape[d] = shape[d];
        p.in_str[d] = in_str ? (I)in_str[d] : 0;
        p.ix_str[d] = ix_str ? (I)ix_str[d] : 0;
        p.up_str[d] = up_str ? (I)up_str[d] : 0;
    }
}

static pt_status check_rank_axis(int ndims, int axis, const char *what)
{
    if (ndims < 1 || ndims > PT_MAX_DIMS) return fail(PT_ERR_INVALID, "%s: rank %d", what, ndims);
    if (axis < 0 || axis >= ndims) return fail(PT_ERR_INVALID, "%s: axis %d", what, axis);
    return PT_OK;
}

static long long total_of(const int *shape, int ndims)
{
    long long t = 1;
    for (int d = 0; d < ndims; d++) {
        if (shape[d] < 0) return -1;
        t *= shape[d];
    }
    return t;
}

template <typename T>
static void launch_gather_t(const void *in, const int32_t *idx, void *out, const int *shape, int ndims, int axis,
                            int axis_size, const size_t *in_str, const size_t *ix_str, long long total,
                            bool i32, int32_t *v, hipStream_t s)
{
    if (i32) {
        IdxParams<uint32_t> p;
        fill_params(p, shape, ndims, axis, axis_size, in_str, ix_str, nullptr);
        k_gather<T, uint32_t><<<idx_grid(total), 256, 0, s>>>((const T *)in, idx, (T *)out, p, (uint32_t)total, v);
    } else {
        IdxParams<unsigned long long> p;
        fill_params(p, shape, ndims, axis, axis_size, in_str, ix_str, nullptr);
        k_gather<T, unsigned long long><<<idx_grid(total), 256, 0, s>>>((const T *)in, idx, (T *)out, p,
                                                                        (unsigned long long)total, v);
    }
}

}  // namespace pt

using namespace pt;

extern "C" {

pt_status pt_index_validate(const int32_t *indices, const int *index_shape, const size_t *index_strides,
                            size_t index_offset, int ndims, int axis, int axis_size, int32_t *record,
                            pt_stream_t stream)
{
    PT_TRY(ensure_init());
    PT_TRY(check_rank_axis(ndims, axis, "index validation"));
    if (!record) return fail(PT_ERR_INVALID, "index validation: no record");
    const long long total = total_of(index_shape, ndims);
    if (total < 0) return fail(PT_ERR_INVALID, "index validation: negative extent");
    hipStream_t s = stream_of(stream);
    int32_t *v = record;
    k_record_reset<<<1, 64, 0, s>>>(v);
    PT_LAUNCH_CHECK("index validation reset");
    if (total > 0) {
        const int32_t *ix = indices + index_offset;
        const bool i32 = total < (1LL << 31) && max_offset(index_shape, ndims, index_strides) < (1LL << 31);
        if (i32) {
            IdxParams<uint32_t> p;
            fill_params(p, index_shape, ndims, axis, axis_size, nullptr, index_strides, nullptr);
            k_index_validate<uint32_t><<<idx_grid(total), 256, 0, s>>>(ix, p, (uint32_t)total, v, IDX_GATHER_INVALID);
        } else {
            IdxParams<unsigned long long> p;
            fill_params(p, index_shape, ndims, axis, axis_size, nullptr, index_strides, nullptr);
            k_index_validate<unsigned long long><<<idx_grid(total), 256, 0, s>>>(ix, p, (unsigned long long)total, v,
                                                                                IDX_GATHER_INVALID);
        }
        PT_LAUNCH_CHECK("index validation");
    }
    return PT_OK;
}

pt_status pt_gather(const void *input, int dtype, const int *input_shape, const size_t *input_strides,
                    size_t input_offset, const int32_t *indices, const int *index_shape,
                    const size_t *index_strides, size_t index_offset, int ndims, int axis, void *output,
                    int32_t *validation, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    PT_TRY(check_rank_axis(ndims, axis, "gather"));
    if (!dtype_valid(dtype)) return fail(PT_ERR_INVALID, "gather: unknown dtype");
    for (int d = 0; d < ndims; d++)
        if (d != axis && input_shape[d] != index_shape[d])
            return fail(PT_ERR_INVALID, "gather input and index shapes must match outside the indexed axis");
    const long long total = total_of(index_shape, ndims);
    if (total < 0) return fail(PT_ERR_INVALID, "gather: negative extent");
    if (total == 0) return PT_OK;
    hipStream_t s = stream_of(stream);
    const size_t es = dtype_size(dtype);
    const char *in = (const char *)input + input_offset * es;
    const int32_t *ix = indices + index_offset;
    long long reach = max_offset(input_shape, ndims, input_strides);
    const long long ireach = max_offset(index_shape, ndims, index_strides);
    if (ireach > reach) reach = ireach;
    const bool i32 = total < (1LL << 31) && reach < (1LL << 31);
    const int axis_size = input_shape[axis];
    switch (es) {
    case 1: launch_gather_t<uint8_t>(in, ix, output, index_shape, ndims, axis, axis_size, input_strides, index_strides,
                                     total, i32, validation, s); break;
    case 2: launch_gather_t<uint16_t>(in, ix, output, index_shape, ndims, axis, axis_size, input_strides,
                                      index_strides, total, i32, validation, s); break;
    case 4: launch_gather_t<uint32_t>(in, ix, output, index_shape, ndims, axis, axis_size, input_strides,
                                      index_strides, total, i32, validation, s); break;
    default: launch_gather_t<unsigned long long>(in, ix, output, index_shape, ndims, axis, axis_size, input_strides,
                                                 index_strides, total, i32, validation, s); break;
    }
    PT_LAUNCH_CHECK("gather");
    counters().elementwise_calls++;
    return PT_OK;
}

pt_status pt_scatter_add(const int32_t *indices, const int *index_shape, const size_t *index_strides,
                         size_t index_offset, const void *updates, const size_t *update_strides,
                         size_t update_offset, int dtype, int ndims, int axis, int axis_size, void *output,
                         const size_t *output_strides, int32_t *validation, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    PT_TRY(check_rank_axis(ndims, axis, "scatterAdd"));
    if (dtype != PT_FLOAT32 && dtype != PT_FLOAT64)
        return fail(PT_ERR_INVALID, "scatterAdd currently supports float32 and float64 tensors");
    const long long total = total_of(index_shape, ndims);
    if (total < 0) return fail(PT_ERR_INVALID, "scatterAdd: negative extent");
    if (total == 0) return PT_OK;
    hipStream_t s = stream_of(stream);
    const size_t es = dtype_size(dtype);
    const int32_t *ix = indices + index_offset;
    const char *up = (const char *)updates + update_offset * es;
    long long reach = max_offset(index_shape, ndims, index_strides);
    const long long ur = max_offset(index_shape, ndims, update_strides);
    if (ur > reach) reach = ur;
    long long orr = 0;
    for (int d = 0; d < ndims; d++)
        orr += (long long)((d == axis ? axis_size : index_shape[d]) - 1) * (long long)output_strides[d];
    if (orr > reach) reach = orr;
    const bool i32 = total < (1LL << 31) && reach < (1LL << 31);
#define PT_SCATTER(T, I)                                                                                       \
    do {                                                                                                       \
        IdxParams<I> p;                                                                                        \
        fill_params(p, index_shape, ndims, axis, axis_size, output_strides, index_strides, update_strides);    \
        k_scatter_add<T, I><<<idx_grid(total), 256, 0, s>>>(ix, (const T *)up, (T *)output, p, (I)total,       \
                                                            validation);                                       \
    } while (0)
    if (dtype == PT_FLOAT32) {
        if (i32) PT_SCATTER(float, uint32_t);
        else PT_SCATTER(float, unsigned long long);
    } else {
        if (i32) PT_SCATTER(double, uint32_t);
        else PT_SCATTER(double, unsigned long long);
    }
#undef PT_SCATTER
    PT_LAUNCH_CHECK("scatterAdd");
    counters().elementwise_calls++;
    return PT_OK;
}

}  // extern "C"
