/*
 * CPU ORACLE — test infrastructure only (see hostarray.h).
 *
 * Restates the reference HostArray CPU path (src/contiguous_array_ce.c) and
 * the CudaArray composites it lacks.  Scalar, single-threaded, no SIMD
 * pragmas: the same loop order as the reference so that sequential float
 * accumulation rounds the same way.
 */
#include "hostarray.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define OR_MAX_DIMS 10

/* ------------------------------------------------------------------ dtypes */

/* data_types.c:46-80 — float32 -> binary16, round to nearest even, NaN payload
 * kept in the top mantissa bits (forced non-zero), overflow to infinity,
 * gradual underflow with RNE on the shifted mantissa. */
uint16_t or_f32_to_f16(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    uint32_t sign = (bits >> 16) & 0x8000u;
    uint32_t exp8 = (bits >> 23) & 0xffu;
    uint32_t frac = bits & 0x7fffffu;
    if (exp8 == 0xffu) {
        uint32_t payload = frac >> 13;
        if (frac != 0 && payload == 0)
            payload = 1;
        return (uint16_t)(sign | 0x7c00u | payload);
    }
    int e = (int)exp8 - 112; /* rebias 127 -> 15 */
    if (e >= 31)
        return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        uint32_t full = frac | 0x800000u;
        int shift = 14 - e;
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u)))
            q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (frac >> 13);
    uint32_t rem = frac & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
        q++;
    return (uint16_t)(sign | q);
}

/* data_types.c:82-111 — binary16 -> float32 (exact). */
float or_f16_to_f32(uint16_t value)
{
    uint32_t sign = ((uint32_t)value & 0x8000u) << 16;
    uint32_t e = (value >> 10) & 0x1fu;
    uint32_t m = value & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int unbiased = -14;
            while (!(m & 0x400u)) {
                m <<= 1;
                unbiased--;
            }
            bits = sign | ((uint32_t)(unbiased + 127) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

/* data_types.c:113-123 — float32 -> bfloat16 RNE, NaN quieted (bit 6). */
uint16_t or_f32_to_bf16(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x7fffffu))
        return (uint16_t)((bits >> 16) | 0x40u);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

/* data_types.c:125-131 */
float or_bf16_to_f32(uint16_t value)
{
    uint32_t bits = (uint32_t)value << 16;
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

void or_f32_to_f16_n(const float *in, uint16_t *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(in[i]);
}
void or_f16_to_f32_n(const uint16_t *in, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(in[i]);
}
void or_f32_to_bf16_n(const float *in, uint16_t *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_bf16(in[i]);
}
void or_bf16_to_f32_n(const uint16_t *in, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_bf16_to_f32(in[i]);
}

static size_t dtype_bytes(int dtype)
{
    switch (dtype) {
    case OR_F32: case OR_I32: case OR_U32: return 4;
    case OR_F64: case OR_I64: case OR_U64: return 8;
    case OR_I16: case OR_U16: case OR_F16: case OR_BF16: return 2;
    case OR_I8: case OR_U8: case OR_BOOL: return 1;
    default: return 0;
    }
}

static int is_floating(int dtype)
{
    return dtype == OR_F32 || dtype == OR_F64 || dtype == OR_F16 || dtype == OR_BF16;
}

/* contiguous_array_number_at (contiguous_array_ce.c:787-801) widened to
 * long double so int64/uint64 compare exactly like cast_single_value. */
static long double load_ld(const void *base, int dtype, size_t i)
{
    const char *p = (const char *)base + i * dtype_bytes(dtype);
    switch (dtype) {
    case OR_F32: return *(const float *)p;
    case OR_F64: return *(const double *)p;
    case OR_F16: return or_f16_to_f32(*(const uint16_t *)p);
    case OR_BF16: return or_bf16_to_f32(*(const uint16_t *)p);
    case OR_I8: return *(const int8_t *)p;
    case OR_I16: return *(const int16_t *)p;
    case OR_I32: return *(const int32_t *)p;
    case OR_I64: return *(const int64_t *)p;
    case OR_U8: return *(const uint8_t *)p;
    case OR_U16: return *(const uint16_t *)p;
    case OR_U32: return *(const uint32_t *)p;
    case OR_U64: return *(const uint64_t *)p;
    case OR_BOOL: return *(const uint8_t *)p != 0;
    default: return 0;
    }
}

static uint64_t load_bits(const void *base, int dtype, size_t i)
{
    const char *p = (const char *)base + i * dtype_bytes(dtype);
    switch (dtype) {
    case OR_I8: return (uint64_t)(int64_t)*(const int8_t *)p;
    case OR_I16: return (uint64_t)(int64_t)*(const int16_t *)p;
    case OR_I32: return (uint64_t)(int64_t)*(const int32_t *)p;
    case OR_I64: return (uint64_t)*(const int64_t *)p;
    case OR_U8: return *(const uint8_t *)p;
    case OR_U16: return *(const uint16_t *)p;
    case OR_U32: return *(const uint32_t *)p;
    case OR_U64: return *(const uint64_t *)p;
    case OR_BOOL: return *(const uint8_t *)p != 0;
    default: return 0;
    }
}

/* cast_single_value (data_types.c:373-436) for the destination dtypes the
 * oracle produces: floats round through float (RNE) or double. */
static void store_ld(void *base, int dtype, size_t i, long double v)
{
    char *p = (char *)base + i * dtype_bytes(dtype);
    switch (dtype) {
    case OR_F32: *(float *)p = (float)v; break;
    case OR_F64: *(double *)p = (double)v; break;
    case OR_F16: *(uint16_t *)p = or_f32_to_f16((float)v); break;
    case OR_BF16: *(uint16_t *)p = or_f32_to_bf16((float)v); break;
    case OR_I8: *(int8_t *)p = (int8_t)v; break;
    case OR_I16: *(int16_t *)p = (int16_t)v; break;
    case OR_I32: *(int32_t *)p = (int32_t)v; break;
    case OR_I64: *(int64_t *)p = (int64_t)v; break;
    case OR_U8: *(uint8_t *)p = (uint8_t)v; break;
    case OR_U16: *(uint16_t *)p = (uint16_t)v; break;
    case OR_U32: *(uint32_t *)p = (uint32_t)v; break;
    case OR_U64: *(uint64_t *)p = (uint64_t)v; break;
    case OR_BOOL: *(uint8_t *)p = v != 0; break;
    default: break;
    }
}

/* contiguous_array_store_integer_bits (contiguous_array_ce.c:1149-1161):
 * modular integer sums keep the low bits of the accumulator. */
static void store_bits(void *base, int dtype, size_t i, uint64_t bits)
{
    char *p = (char *)base + i * dtype_bytes(dtype);
    if (dtype == OR_BOOL) {
        *(uint8_t *)p = bits != 0;
        return;
    }
    switch (dtype_bytes(dtype)) {
    case 1: *(uint8_t *)p = (uint8_t)bits; break;
    case 2: *(uint16_t *)p = (uint16_t)bits; break;
    case 4: *(uint32_t *)p = (uint32_t)bits; break;
    case 8: *(uint64_t *)p = bits; break;
    }
}

static int valid_dtype(int dtype)
{
    return dtype_bytes(dtype) != 0;
}

static size_t shape_elements(const int *shape, int ndims)
{
    size_t n = 1;
    for (int d = 0; d < ndims; d++) n *= (size_t)shape[d];
    return n;
}

static void contiguous_strides(const int *shape, int ndims, size_t *strides)
{
    size_t s = 1;
    for (int d = ndims - 1; d >= 0; d--) {
        strides[d] = s;
        s *= (size_t)shape[d];
    }
}

/* contiguous_array_broadcast_offset (contiguous_array_ce.c:913-927). */
static size_t broadcast_offset(const int *shape_in, const size_t *strides_in, int nd_in,
                               size_t index, const int *shape, int ndims)
{
    size_t offset = 0;
    int rank_offset = ndims - nd_in;
    for (int axis = ndims - 1; axis >= 0; axis--) {
        size_t coordinate = index % (size_t)shape[axis];
        index /= (size_t)shape[axis];
        int in_axis = axis - rank_offset;
        if (in_axis >= 0 && shape_in[in_axis] != 1)
            offset += coordinate * strides_in[in_axis];
    }
    return offset;
}

/* ------------------------------------------------------------- reductions */

int or_reduce_result_dtype(int dtype, int op)
{
    int out = dtype;
    if (dtype == OR_F16 || dtype == OR_BF16)
        out = OR_F32;
    if (op == OR_OP_REDUCE_MEAN && !is_floating(out))
        out = OR_F64;
    return out;
}

/* contiguous_array_reduce (contiguous_array_ce.c:1163-1270). */
int or_reduce(const void *x, int dtype, const int *shape, int ndims, int axis,
              int op, void *out)
{
    if (!valid_dtype(dtype) || ndims < 0 || ndims > OR_MAX_DIMS || axis >= ndims)
        return OR_EINVAL;
    if (op != OR_OP_REDUCE_SUM && op != OR_OP_REDUCE_MEAN &&
        op != OR_OP_REDUCE_MAX && op != OR_OP_REDUCE_MIN)
        return OR_EINVAL;
    size_t strides[OR_MAX_DIMS];
    contiguous_strides(shape, ndims, strides);
    size_t total = shape_elements(shape, ndims);
    size_t count = axis < 0 ? total : (size_t)shape[axis];
    size_t elements = axis < 0 ? 1 : (count ? total / count : 1);
    if (axis >= 0 && count == 0) {
        elements = 1;
        for (int d = 0; d < ndims; d++)
            if (d != axis) elements *= (size_t)shape[d];
    }
    int rdtype = or_reduce_result_dtype(dtype, op);
    if (elements && !count && (op == OR_OP_REDUCE_MIN || op == OR_OP_REDUCE_MAX))
        return OR_EINVAL; /* :1199-1203 no identity for an empty axis */
    for (size_t o = 0; o < elements; o++) {
        size_t base = 0, rem = o;
        if (axis >= 0)
            for (int d = ndims - 1; d >= 0; d--)
                if (d != axis) {
                    base += (rem % (size_t)shape[d]) * strides[d];
                    rem /= (size_t)shape[d];
                }
        double sum = 0;
        uint64_t bits = 0;
        int have_best = 0;
        long double best = op == OR_OP_REDUCE_MAX ? -INFINITY : INFINITY;
        for (size_t i = 0; i < count; i++) {
            size_t off = axis < 0 ? i : base + i * strides[axis];
            if (op == OR_OP_REDUCE_SUM && !is_floating(rdtype)) {
                uint64_t in = load_bits(x, dtype, off);
                bits = rdtype == OR_BOOL ? (bits || in) : bits + in;
            } else if (op == OR_OP_REDUCE_SUM || op == OR_OP_REDUCE_MEAN) {
                double number = (double)load_ld(x, dtype, off);
                sum = rdtype == OR_F32 ? (float)((float)sum + (float)number) : sum + number;
            } else {
                long double v = load_ld(x, dtype, off);
                if (is_floating(dtype) && isnan(v))
                    continue; /* :1241-1242 NaN skipped */
                if (!have_best || (op == OR_OP_REDUCE_MAX ? v > best : v < best)) {
                    best = v;
                    have_best = 1;
                }
            }
        }
        if (op == OR_OP_REDUCE_SUM && !is_floating(rdtype)) {
            store_bits(out, rdtype, o, bits);
            continue;
        }
        if (op == OR_OP_REDUCE_SUM) {
            store_ld(out, rdtype, o, sum);
        } else if (op == OR_OP_REDUCE_MEAN) {
            double m = !count ? NAN
                : rdtype == OR_F32 ? (float)((float)sum / (float)count) : sum / (double)count;
            store_ld(out, rdtype, o, m);
        } else {
            store_ld(out, rdtype, o, best);
        }
    }
    return OR_OK;
}

/* CudaArray arg reductions (reduction_ops.cuh:319-401; IndexedReductionOp
 * :52-58): a sequential scan with a strict comparison keeps the lowest index
 * of the extreme value; the identity (lowest/highest value, index 0) is only
 * replaced by a strictly better element, so NaN is never chosen and an axis
 * holding only the identity value returns 0. */
int or_arg_reduce(const void *x, int dtype, const int *shape, int ndims,
                  int axis, int op, int32_t *out)
{
    if (!valid_dtype(dtype) || ndims < 0 || ndims > OR_MAX_DIMS || axis >= ndims)
        return OR_EINVAL;
    if (op != OR_OP_ARG_MAX && op != OR_OP_ARG_MIN)
        return OR_EINVAL;
    size_t strides[OR_MAX_DIMS];
    contiguous_strides(shape, ndims, strides);
    size_t total = shape_elements(shape, ndims);
    size_t count = axis < 0 ? total : (size_t)shape[axis];
    size_t elements = 1;
    if (axis >= 0)
        for (int d = 0; d < ndims; d++)
            if (d != axis) elements *= (size_t)shape[d];
    if (elements && !count)
        return OR_EINVAL; /* ca_private.c:254-258 */
    int maximize = op == OR_OP_ARG_MAX;
    for (size_t o = 0; o < elements; o++) {
        size_t base = 0, rem = o;
        if (axis >= 0)
            for (int d = ndims - 1; d >= 0; d--)
                if (d != axis) {
                    base += (rem % (size_t)shape[d]) * strides[d];
                    rem /= (size_t)shape[d];
                }
        long double best;
        if (is_floating(dtype)) {
            best = maximize ? -INFINITY : INFINITY;
        } else {
            /* std::numeric_limits<T>::lowest()/max() identities */
            switch (dtype) {
            case OR_I8: best = maximize ? -128.0L : 127.0L; break;
            case OR_I16: best = maximize ? -32768.0L : 32767.0L; break;
            case OR_I32: best = maximize ? -2147483648.0L : 2147483647.0L; break;
            case OR_I64: best = maximize ? -9223372036854775808.0L : 9223372036854775807.0L; break;
            case OR_U8: best = maximize ? 0 : 255.0L; break;
            case OR_U16: best = maximize ? 0 : 65535.0L; break;
            case OR_U32: best = maximize ? 0 : 4294967295.0L; break;
            case OR_U64: best = maximize ? 0 : 18446744073709551615.0L; break;
            default: best = maximize ? 0 : 1; break;
            }
        }
        int32_t index = 0;
        for (size_t i = 0; i < count; i++) {
            size_t off = axis < 0 ? i : base + i * strides[axis];
            long double v = load_ld(x, dtype, off);
            if (maximize ? v > best : v < best) {
                best = v;
                index = (int32_t)i;
            }
        }
        out[o] = index;
    }
    return OR_OK;
}

/* CudaArray var/std (cuda_array_ce.c:1850-1940; Welford reduction_ops.cuh:
 * 86-112).  welford_single seeds m2 with value - value so that a non-finite
 * element turns the result into NaN, as on the device. */
int or_moments(const void *x, int dtype, const int *shape, int ndims, int axis,
               int correction, int standard_deviation, void *out)
{
    if (!valid_dtype(dtype) || ndims < 0 || ndims > OR_MAX_DIMS || axis >= ndims)
        return OR_EINVAL;
    size_t strides[OR_MAX_DIMS];
    contiguous_strides(shape, ndims, strides);
    size_t total = shape_elements(shape, ndims);
    size_t count = axis < 0 ? total : (size_t)shape[axis];
    if (correction < 0 || (size_t)correction >= count)
        return OR_EINVAL; /* cuda_array_ce.c:1855-1860 */
    size_t elements = 1;
    if (axis >= 0)
        for (int d = 0; d < ndims; d++)
            if (d != axis) elements *= (size_t)shape[d];
    int rdtype = (dtype == OR_F32 || dtype == OR_F16 || dtype == OR_BF16) ? OR_F32 : OR_F64;
    for (size_t o = 0; o < elements; o++) {
        size_t base = 0, rem = o;
        if (axis >= 0)
            for (int d = ndims - 1; d >= 0; d--)
                if (d != axis) {
                    base += (rem % (size_t)shape[d]) * strides[d];
                    rem /= (size_t)shape[d];
                }
        double n = 0, mean = 0, m2 = 0;
        for (size_t i = 0; i < count; i++) {
            size_t off = axis < 0 ? i : base + i * strides[axis];
            double v = (double)load_ld(x, dtype, off);
            double v_m2 = isfinite(v) ? 0.0 : v - v;
            if (n == 0) {
                n = 1;
                mean = v;
                m2 = v_m2;
                continue;
            }
            double delta = v - mean;
            double c = n + 1;
            mean = mean + delta * 1.0 / c;
            m2 = m2 + v_m2 + delta * delta * n * 1.0 / c;
            n = c;
        }
        double var = m2 / (double)(count - (size_t)correction);
        store_ld(out, rdtype, o, standard_deviation ? sqrt(var) : var);
    }
    return OR_OK;
}

/* ------------------------------------------------------ softmax/layerNorm */

/* cuda_array_softmax (cuda_array_ce.c:1942-2001): reduce MAX, SUB, EXP,
 * reduce SUM, DIV.  The max skips NaN like fmaxf; sums are sequential. */
int or_softmax_f32(const float *x, size_t rows, size_t n, float *out)
{
    if (n == 0 && rows)
        return OR_EINVAL; /* max has no identity on an empty axis */
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * n;
        float *yr = out + r * n;
        float m = -INFINITY;
        for (size_t i = 0; i < n; i++)
            m = fmaxf(m, xr[i]);
        float s = 0.0f;
        for (size_t i = 0; i < n; i++) {
            float shifted = xr[i] - m;
            float e = expf(shifted);
            yr[i] = e;
            s = s + e;
        }
        for (size_t i = 0; i < n; i++)
            yr[i] = yr[i] / s;
    }
    return OR_OK;
}

int or_softmax_f64(const double *x, size_t rows, size_t n, double *out)
{
    if (n == 0 && rows)
        return OR_EINVAL;
    for (size_t r = 0; r < rows; r++) {
        const double *xr = x + r * n;
        double *yr = out + r * n;
        double m = -INFINITY;
        for (size_t i = 0; i < n; i++)
            m = fmax(m, xr[i]);
        double s = 0.0;
        for (size_t i = 0; i < n; i++) {
            double e = exp(xr[i] - m);
            yr[i] = e;
            s = s + e;
        }
        for (size_t i = 0; i < n; i++)
            yr[i] = yr[i] / s;
    }
    return OR_OK;
}

/* cuda_array_layernorm (cuda_array_ce.c:2215-2339) for one trailing axis
 * group: mean -> centered -> squared -> mean -> + eps -> sqrt -> divide,
 * then optional scale and bias, each step rounded to float32. */
int or_layernorm_f32(const float *x, size_t rows, size_t n, float eps,
                     const float *gamma, const float *beta, float *out)
{
    if (n == 0 || !(eps > 0.0f) || !isfinite(eps))
        return OR_EINVAL;
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * n;
        float *yr = out + r * n;
        float s = 0.0f;
        for (size_t i = 0; i < n; i++)
            s = s + xr[i];
        float mean = s / (float)n;
        float sq = 0.0f;
        for (size_t i = 0; i < n; i++) {
            float c = xr[i] - mean;
            yr[i] = c;
            sq = sq + c * c;
        }
        float var = sq / (float)n;
        float dev = sqrtf(var + eps);
        for (size_t i = 0; i < n; i++) {
            float v = yr[i] / dev;
            if (gamma) v = v * gamma[i];
            if (beta) v = v + beta[i];
            yr[i] = v;
        }
    }
    return OR_OK;
}

/* ------------------------------------------------------------------ matmul */

/* contiguous_array_batch_offset (contiguous_array_ce.c:1280-1293). */
static size_t batch_offset(const int *shape_in, const size_t *strides_in, int nd_in,
                           size_t batch, const int *shape, int ndims)
{
    size_t offset = 0;
    for (int d = ndims - 3; d >= 0; d--) {
        size_t coordinate = batch % (size_t)shape[d];
        batch /= (size_t)shape[d];
        int in_axis = d - (ndims - nd_in);
        if (in_axis >= 0 && shape_in[in_axis] != 1)
            offset += coordinate * strides_in[in_axis];
    }
    return offset;
}

/* HostArray::matmul (contiguous_array_ce.c:1295-1343). */
/* Outputs [begin, end) of the product, each one sum of fmaf in k order
 * (contiguous_array_ce.c:1295-1343). */
static void matmul_range(const void *a, const int *shape_a, const size_t *strides_a, int nd_a,
                         const void *b, const int *shape_b, const size_t *strides_b, int nd_b,
                         int dtype, void *c, const int *shape_c, int nd_c, size_t begin, size_t end)
{
    size_t rows = (size_t)shape_c[nd_c - 2], cols = (size_t)shape_c[nd_c - 1];
    int inner = shape_a[nd_a - 1];
    for (size_t i = begin; i < end; i++) {
        size_t batch = i / cols / rows;
        size_t oa = batch_offset(shape_a, strides_a, nd_a, batch, shape_c, nd_c) +
            (i / cols % rows) * strides_a[nd_a - 2];
        size_t ob = batch_offset(shape_b, strides_b, nd_b, batch, shape_c, nd_c) +
            (i % cols) * strides_b[nd_b - 1];
        float sum = 0;
        for (int k = 0; k < inner; k++) {
            float xa = (float)load_ld(a, dtype, oa + (size_t)k * strides_a[nd_a - 1]);
            float xb = (float)load_ld(b, dtype, ob + (size_t)k * strides_b[nd_b - 2]);
            sum = fmaf(xa, xb, sum);
        }
        store_ld(c, dtype, i, sum);
    }
}

int or_matmul(const void *a, const int *shape_a, const size_t *strides_a, int nd_a,
              const void *b, const int *shape_b, const size_t *strides_b, int nd_b,
              int dtype, void *c, const int *shape_c, int nd_c)
{
    if (dtype != OR_F32 && dtype != OR_F16 && dtype != OR_BF16)
        return OR_EINVAL;
    if (nd_a < 2 || nd_b < 2 || nd_c < 2 || shape_a[nd_a - 1] != shape_b[nd_b - 2])
        return OR_EINVAL;
    matmul_range(a, shape_a, strides_a, nd_a, b, shape_b, strides_b, nd_b, dtype, c, shape_c, nd_c, 0,
                 shape_elements(shape_c, nd_c));
    return OR_OK;
}

struct matmul_job {
    const void *a, *b;
    const int *shape_a, *shape_b, *shape_c;
    const size_t *strides_a, *strides_b;
    int nd_a, nd_b, nd_c, dtype;
    void *c;
    size_t begin, end;
};

static void *matmul_worker(void *arg)
{
    const struct matmul_job *j = arg;
    matmul_range(j->a, j->shape_a, j->strides_a, j->nd_a, j->b, j->shape_b, j->strides_b, j->nd_b, j->dtype, j->c,
                 j->shape_c, j->nd_c, j->begin, j->end);
    return NULL;
}

int or_matmul_mt(const void *a, const int *shape_a, const size_t *strides_a, int nd_a,
                 const void *b, const int *shape_b, const size_t *strides_b, int nd_b,
                 int dtype, void *c, const int *shape_c, int nd_c, int threads)
{
    if (dtype != OR_F32 && dtype != OR_F16 && dtype != OR_BF16)
        return OR_EINVAL;
    if (nd_a < 2 || nd_b < 2 || nd_c < 2 || shape_a[nd_a - 1] != shape_b[nd_b - 2])
        return OR_EINVAL;
    if (threads < 1 || threads > 256)
        return OR_EINVAL;
    size_t total = shape_elements(shape_c, nd_c);
    pthread_t tid[256];
    int running[256] = {0};
    struct matmul_job jobs[256];
    for (int t = 0; t < threads; t++) {
        struct matmul_job *j = &jobs[t];
        j->a = a;
        j->b = b;
        j->shape_a = shape_a;
        j->shape_b = shape_b;
        j->shape_c = shape_c;
        j->strides_a = strides_a;
        j->strides_b = strides_b;
        j->nd_a = nd_a;
        j->nd_b = nd_b;
        j->nd_c = nd_c;
        j->dtype = dtype;
        j->c = c;
        j->begin = total * (size_t)t / (size_t)threads;
        j->end = total * (size_t)(t + 1) / (size_t)threads;
    }
    /* ranges 1.. on their own threads (or here, when a thread cannot start),
     * range 0 on the caller's thread */
    for (int t = 1; t < threads; t++) {
        if (pthread_create(&tid[t], NULL, matmul_worker, &jobs[t]) == 0)
            running[t] = 1;
        else
            matmul_worker(&jobs[t]);
    }
    matmul_worker(&jobs[0]);
    for (int t = 1; t < threads; t++)
        if (running[t]) pthread_join(tid[t], NULL);
    return OR_OK;
}

/* -------------------------------------------------------------- elementwise */

static int promote_float(int a, int b, int op)
{
    /* promote_types (data_types.c:301-349) restricted to floating dtypes,
     * then promote_types_for_arithmetic (:492-516). */
    int p;
    if (a == b) p = a;
    else if ((a == OR_F16 || a == OR_BF16) && (b == OR_F16 || b == OR_BF16)) p = OR_F32;
    else if (a == OR_F16 || a == OR_BF16) p = b;
    else if (b == OR_F16 || b == OR_BF16) p = a;
    else p = (a == OR_F64 || b == OR_F64) ? OR_F64 : OR_F32;
    if (op == OR_OP_DIV)
        p = p == OR_F64 ? OR_F64 : OR_F32;
    return p;
}

static double apply_d(int op, double l, double r)
{
    switch (op) {
    case OR_OP_ADD: return l + r;
    case OR_OP_SUB: return l - r;
    case OR_OP_MUL: return l * r;
    default: return l / r;
    }
}

static float apply_f(int op, float l, float r)
{
    switch (op) {
    case OR_OP_ADD: return l + r;
    case OR_OP_SUB: return l - r;
    case OR_OP_MUL: return l * r;
    default: return l / r;
    }
}

/* contiguous_array_binary_apply (contiguous_array_ce.c:1345-1447). */
int or_binary(const void *a, int dtype_a, const int *shape_a, int nd_a,
              const void *b, int dtype_b, const int *shape_b, int nd_b,
              int op, void *out, int dtype_out, const int *shape_out, int nd_out)
{
    if (!is_floating(dtype_a) || !is_floating(dtype_b))
        return OR_EINVAL;
    if (op < OR_OP_ADD || op > OR_OP_DIV)
        return OR_EINVAL;
    if (promote_float(dtype_a, dtype_b, op) != dtype_out)
        return OR_EINVAL;
    size_t sa[OR_MAX_DIMS], sb[OR_MAX_DIMS];
    contiguous_strides(shape_a, nd_a, sa);
    contiguous_strides(shape_b, nd_b, sb);
    size_t total = shape_elements(shape_out, nd_out);
    for (size_t i = 0; i < total; i++) {
        size_t oa = broadcast_offset(shape_a, sa, nd_a, i, shape_out, nd_out);
        size_t ob = broadcast_offset(shape_b, sb, nd_b, i, shape_out, nd_out);
        double l = (double)load_ld(a, dtype_a, oa);
        double r = (double)load_ld(b, dtype_b, ob);
        if (dtype_out != OR_F64)
            store_ld(out, dtype_out, i, apply_f(op, (float)l, (float)r));
        else
            store_ld(out, dtype_out, i, apply_d(op, l, r));
    }
    return OR_OK;
}

int or_binary_scalar(const void *a, int dtype_a, size_t n, double scalar,
                     int op, int reverse, void *out, int dtype_out)
{
    if (!is_floating(dtype_a) || op < OR_OP_ADD || op > OR_OP_DIV)
        return OR_EINVAL;
    for (size_t i = 0; i < n; i++) {
        double t = (double)load_ld(a, dtype_a, i);
        double l = reverse ? scalar : t;
        double r = reverse ? t : scalar;
        if (dtype_out == OR_F32) {
            l = (float)l;
            r = (float)r;
        }
        if (dtype_out != OR_F64)
            store_ld(out, dtype_out, i, apply_f(op, (float)l, (float)r));
        else
            store_ld(out, dtype_out, i, apply_d(op, l, r));
    }
    return OR_OK;
}

static float unary_f(int op, float v)
{
    switch (op) {
    case OR_OP_SQRT: return sqrtf(v);
    case OR_OP_EXP: return expf(v);
    case OR_OP_EXPM1: return expm1f(v);
    case OR_OP_EXP2: return exp2f(v);
    case OR_OP_LOG: return logf(v);
    case OR_OP_LOG1P: return log1pf(v);
    case OR_OP_LOG2: return log2f(v);
    case OR_OP_LOG10: return log10f(v);
    case OR_OP_SIN: return sinf(v);
    case OR_OP_COS: return cosf(v);
    case OR_OP_TAN: return tanf(v);
    case OR_OP_ASIN: return asinf(v);
    case OR_OP_ACOS: return acosf(v);
    case OR_OP_ATAN: return atanf(v);
    case OR_OP_SINH: return sinhf(v);
    case OR_OP_COSH: return coshf(v);
    case OR_OP_TANH: return tanhf(v);
    case OR_OP_ABS: return v < 0 ? -v : v;
    case OR_OP_NEG: return -v;
    case OR_OP_FLOOR: return floorf(v);
    case OR_OP_CEIL: return ceilf(v);
    case OR_OP_ROUND: return roundf(v);
    default: return NAN;
    }
}

static double unary_d(int op, double v)
{
    switch (op) {
    case OR_OP_SQRT: return sqrt(v);
    case OR_OP_EXP: return exp(v);
    case OR_OP_EXPM1: return expm1(v);
    case OR_OP_EXP2: return exp2(v);
    case OR_OP_LOG: return log(v);
    case OR_OP_LOG1P: return log1p(v);
    case OR_OP_LOG2: return log2(v);
    case OR_OP_LOG10: return log10(v);
    case OR_OP_SIN: return sin(v);
    case OR_OP_COS: return cos(v);
    case OR_OP_TAN: return tan(v);
    case OR_OP_ASIN: return asin(v);
    case OR_OP_ACOS: return acos(v);
    case OR_OP_ATAN: return atan(v);
    case OR_OP_SINH: return sinh(v);
    case OR_OP_COSH: return cosh(v);
    case OR_OP_TANH: return tanh(v);
    case OR_OP_ABS: return v < 0 ? -v : v;
    case OR_OP_NEG: return -v;
    case OR_OP_FLOOR: return floor(v);
    case OR_OP_CEIL: return ceil(v);
    case OR_OP_ROUND: return round(v);
    default: return NAN;
    }
}

/* contiguous_array_unary (contiguous_array_ce.c:1080-1131). */
int or_unary(const void *x, int dtype, size_t n, int op, void *out)
{
    if (!is_floating(dtype))
        return OR_EINVAL;
    for (size_t i = 0; i < n; i++) {
        double v = (double)load_ld(x, dtype, i);
        double r = dtype == OR_F64 ? unary_d(op, v) : (double)unary_f(op, (float)v);
        store_ld(out, dtype, i, r);
    }
    return OR_OK;
}

/* HostArray::where (contiguous_array_ce.c:1021-1073). */
int or_where(const void *cond, int dtype_c, const int *shape_c, int nd_c,
             const void *x, const int *shape_x, int nd_x,
             const void *y, const int *shape_y, int nd_y, int dtype_xy,
             void *out, const int *shape_out, int nd_out)
{
    if (!valid_dtype(dtype_c) || !valid_dtype(dtype_xy))
        return OR_EINVAL;
    size_t sc[OR_MAX_DIMS], sx[OR_MAX_DIMS], sy[OR_MAX_DIMS];
    contiguous_strides(shape_c, nd_c, sc);
    contiguous_strides(shape_x, nd_x, sx);
    contiguous_strides(shape_y, nd_y, sy);
    size_t es = dtype_bytes(dtype_xy);
    size_t total = shape_elements(shape_out, nd_out);
    for (size_t i = 0; i < total; i++) {
        size_t oc = broadcast_offset(shape_c, sc, nd_c, i, shape_out, nd_out);
        int pick = load_ld(cond, dtype_c, oc) != 0;
        const char *src = pick
            ? (const char *)x + broadcast_offset(shape_x, sx, nd_x, i, shape_out, nd_out) * es
            : (const char *)y + broadcast_offset(shape_y, sy, nd_y, i, shape_out, nd_out) * es;
        memcpy((char *)out + i * es, src, es);
    }
    return OR_OK;
}

/* Offsets of index-shape coordinate `flat` in x (with the axis coordinate
 * left out) and the coordinate itself (indexed_ops.cu:113-124). */
static size_t indexed_offset(const int *shape_idx, const size_t *sx, int ndims, int axis, size_t flat)
{
    size_t off = 0;
    for (int d = ndims - 1; d >= 0; d--) {
        size_t c = flat % (size_t)shape_idx[d];
        flat /= (size_t)shape_idx[d];
        if (d != axis)
            off += c * sx[d];
    }
    return off;
}

static int indexed_check(const int *shape_x, const int32_t *idx, const int *shape_idx, int ndims, int axis,
                         int32_t *bad)
{
    if (ndims < 1 || ndims > OR_MAX_DIMS || axis < 0 || axis >= ndims)
        return OR_EINVAL;
    for (int d = 0; d < ndims; d++)
        if (d != axis && shape_x[d] != shape_idx[d])
            return OR_EINVAL;
    size_t n = shape_elements(shape_idx, ndims);
    for (size_t i = 0; i < n; i++)
        if (idx[i] < 0 || idx[i] >= shape_x[axis]) {
            if (bad)
                *bad = idx[i];
            return OR_EINVAL;
        }
    return OR_OK;
}

/* gather_kernel (indexed_ops.cu:108-133) over contiguous operands. */
int or_gather(const void *x, int dtype, const int *shape_x, const int32_t *idx,
              const int *shape_idx, int ndims, int axis, void *out, int32_t *bad)
{
    if (!valid_dtype(dtype))
        return OR_EINVAL;
    int st = indexed_check(shape_x, idx, shape_idx, ndims, axis, bad);
    if (st != OR_OK)
        return st;
    size_t sx[OR_MAX_DIMS];
    contiguous_strides(shape_x, ndims, sx);
    size_t es = dtype_bytes(dtype), n = shape_elements(shape_idx, ndims);
    for (size_t i = 0; i < n; i++) {
        size_t off = indexed_offset(shape_idx, sx, ndims, axis, i) + (size_t)idx[i] * sx[axis];
        memcpy((char *)out + i * es, (const char *)x + off * es, es);
    }
    return OR_OK;
}

/* scatter_copy + scatter_add_kernel (indexed_ops.cu:135-151, 179-204):
 * the adds are applied in flat index order. */
int or_scatter_add(const void *x, int dtype, const int *shape_x, const int32_t *idx,
                   const int *shape_idx, const void *upd, int ndims, int axis,
                   void *out, int32_t *bad)
{
    if (dtype != OR_F32 && dtype != OR_F64)
        return OR_EINVAL;
    int st = indexed_check(shape_x, idx, shape_idx, ndims, axis, bad);
    if (st != OR_OK)
        return st;
    size_t sx[OR_MAX_DIMS];
    contiguous_strides(shape_x, ndims, sx);
    size_t es = dtype_bytes(dtype);
    memcpy(out, x, shape_elements(shape_x, ndims) * es);
    size_t n = shape_elements(shape_idx, ndims);
    for (size_t i = 0; i < n; i++) {
        size_t off = indexed_offset(shape_idx, sx, ndims, axis, i) + (size_t)idx[i] * sx[axis];
        if (dtype == OR_F32)
            ((float *)out)[off] += ((const float *)upd)[i];
        else
            ((double *)out)[off] += ((const double *)upd)[i];
    }
    return OR_OK;
}
