// Eager elementwise kernels for gfx950: broadcast binary ops, tensor-scalar
// ops, unary math, dtype casts / strided packs, where-select and fills.
//
// The host collapses the output shape first (adjacent dimensions merge
// when every operand's strides allow it; size-1 dimensions drop), so most
// broadcasts reach the kernels as 1-2 dimensions.  All-contiguous operands
// of one dtype take a vectorized path (16-byte loads and stores); every
// other layout and dtype mix runs the generic path, which decodes the
// collapsed index and converts through the compute type.
//
// Op semantics follow the reference functors (cuda_op_functors.cuh:12-449):
// operands are converted to the output dtype (float for f16/bf16 outputs),
// integer division by zero yields 0, ** takes the integer-exponent path
// when the exponent is integral, maximum/minimum are (a > b) ? a : b and
// (a < b) ? a : b, comparisons produce 1/0 in the output dtype, unary math
// on integers computes in float and converts back.  Math uses the accurate
// device libm (no fast-math); no contraction (-ffp-contract=off).
#include "pt_common.h"

#include <math.h>
#include <string.h>

namespace pt {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte accesses: operands read once and results written once
// bypass cache retention (nontemporal), which keeps HBM streams at full rate.
__device__ __forceinline__ f32x4 ld_stream(const float *p) { return __builtin_nontemporal_load((const f32x4 *)p); }
__device__ __forceinline__ void st_stream(float *p, f32x4 v) { __builtin_nontemporal_store(v, (f32x4 *)p); }

struct EwShape {
    int ndims;
    long long shape[PT_MAX_DIMS];
    long long sa[PT_MAX_DIMS];
    long long sb[PT_MAX_DIMS];
    long long sc[PT_MAX_DIMS];
    long long total;
};

// 32-bit form of an EwShape, used when the element count and every
// operand's largest offset stay below 2^31: index decoding then costs 32-bit
// divisions instead of emulated 64-bit ones.
struct EwShape32 {
    int ndims;
    unsigned shape[PT_MAX_DIMS];
    unsigned sa[PT_MAX_DIMS];
    unsigned sb[PT_MAX_DIMS];
    unsigned sc[PT_MAX_DIMS];
    unsigned total;
};

static bool to32(const EwShape &s, EwShape32 &o)
{
    const long long lim = 0x7fffffffLL;
    if (s.total > lim) return false;
    long long ma = 0, mb = 0, mc = 0;
    for (int d = 0; d < s.ndims; d++) {
        ma += (s.shape[d] - 1) * s.sa[d];
        mb += (s.shape[d] - 1) * s.sb[d];
        mc += (s.shape[d] - 1) * s.sc[d];
    }
    if (ma > lim || mb > lim || mc > lim) return false;
    o.ndims = s.ndims;
    o.total = (unsigned)s.total;
    for (int d = 0; d < s.ndims; d++) {
        o.shape[d] = (unsigned)s.shape[d];
        o.sa[d] = (unsigned)s.sa[d];
        o.sb[d] = (unsigned)s.sb[d];
        o.sc[d] = (unsigned)s.sc[d];
    }
    return true;
}

// Merge dims so that each operand's addressing stays affine; drop extent-1.
static void collapse(const int *shape, int ndims, const size_t *sa, const size_t *sb,
                     const size_t *sc, EwShape &o)
{
    o.ndims = 0;
    o.total = 1;
    for (int d = 0; d < ndims; d++) {
        long long e = shape[d];
        o.total *= e;
        if (e == 1) continue;
        long long a = sa ? (long long)sa[d] : 0, b = sb ? (long long)sb[d] : 0,
                  c = sc ? (long long)sc[d] : 0;
        if (o.ndims > 0) {
            int k = o.ndims - 1;
            if (o.sa[k] == a * e && o.sb[k] == b * e && o.sc[k] == c * e) {
                o.shape[k] *= e;
                o.sa[k] = a;
                o.sb[k] = b;
                o.sc[k] = c;
                continue;
            }
        }
        o.shape[o.ndims] = e;
        o.sa[o.ndims] = a;
        o.sb[o.ndims] = b;
        o.sc[o.ndims] = c;
        o.ndims++;
    }
}

// ------------------------------------------------------------ conversions
template <typename CT>
__device__ __forceinline__ CT ld(const void *p, int dt, long long i)
{
    switch (dt) {
    case PT_FLOAT32: return (CT)((const float *)p)[i];
    case PT_FLOAT64: return (CT)((const double *)p)[i];
    case PT_FLOAT16: return (CT)f16_to_float(((const uint16_t *)p)[i]);
    case PT_BFLOAT16: return (CT)bf16_to_float(((const uint16_t *)p)[i]);
    case PT_INT8: return (CT)((const int8_t *)p)[i];
    case PT_INT16: return (CT)((const int16_t *)p)[i];
    case PT_INT32: return (CT)((const int32_t *)p)[i];
    case PT_INT64: return (CT)((const int64_t *)p)[i];
    case PT_UINT8: return (CT)((const uint8_t *)p)[i];
    case PT_UINT16: return (CT)((const uint16_t *)p)[i];
    case PT_UINT32: return (CT)((const uint32_t *)p)[i];
    case PT_UINT64: return (CT)((const uint64_t *)p)[i];
    case PT_BOOL: return (CT)(((const uint8_t *)p)[i] != 0);
    default: return (CT)0;
    }
}

template <typename CT>
__device__ __forceinline__ void st(void *p, int dt, long long i, CT v)
{
    switch (dt) {
    case PT_FLOAT32: ((float *)p)[i] = (float)v; break;
    case PT_FLOAT64: ((double *)p)[i] = (double)v; break;
    case PT_FLOAT16: ((uint16_t *)p)[i] = float_to_f16((float)v); break;
    case PT_BFLOAT16: ((uint16_t *)p)[i] = float_to_bf16((float)v); break;
    case PT_INT8: ((int8_t *)p)[i] = (int8_t)v; break;
    case PT_INT16: ((int16_t *)p)[i] = (int16_t)v; break;
    case PT_INT32: ((int32_t *)p)[i] = (int32_t)v; break;
    case PT_INT64: ((int64_t *)p)[i] = (int64_t)v; break;
    case PT_UINT8: ((uint8_t *)p)[i] = (uint8_t)v; break;
    case PT_UINT16: ((uint16_t *)p)[i] = (uint16_t)v; break;
    case PT_UINT32: ((uint32_t *)p)[i] = (uint32_t)v; break;
    case PT_UINT64: ((uint64_t *)p)[i] = (uint64_t)v; break;
    case PT_BOOL: ((uint8_t *)p)[i] = v != (CT)0; break;
    default: break;
    }
}

// Compute type of an output dtype: float for f32/f16/bf16, double for f64,
// int64 for signed integers, uint64 for unsigned integers and bool.
enum { CT_F32 = 0, CT_F64, CT_I64, CT_U64 };
static int compute_class(int dt)
{
    switch (dt) {
    case PT_FLOAT32: case PT_FLOAT16: case PT_BFLOAT16: return CT_F32;
    case PT_FLOAT64: return CT_F64;
    case PT_INT8: case PT_INT16: case PT_INT32: case PT_INT64: return CT_I64;
    default: return CT_U64;
    }
}

// Arithmetic is evaluated at the width of the output dtype: narrow integer
// results wrap exactly as the reference's scalar_t arithmetic does once
// stored, and int64/uint64 use their own width.
template <typename CT> __device__ __forceinline__ CT int_pow(CT base, int e)
{
    CT r = (CT)1;
    while (e > 0) {
        if (e & 1) r = r * base;
        base = base * base;
        e >>= 1;
    }
    return r;
}

template <typename CT>
__device__ __forceinline__ CT pow_op(CT a, CT b)
{
    if constexpr (sizeof(CT) == 8 && (CT)0.5 == (CT)0) {
        // integer types: integral exponent path only
        int e = (int)b;
        if (e == 0) return (CT)1;
        if (e == 1) return a;
        if (e == 2) return a * a;
        if (e == 3) return a * a * a;
        if (e < 0) return (CT)0;
        return int_pow(a, e);
    } else {
        if (b == floor(b)) {
            int e = (int)b;
            if (e == 0) return (CT)1;
            if (e == 1) return a;
            if (e == 2) return a * a;
            if (e == 3) return a * a * a;
            if (e < 0) return (CT)1 / int_pow(a, -e);
            return int_pow(a, e);
        }
        if constexpr (sizeof(CT) == 4) return powf(a, b);
        else return pow(a, b);
    }
}

template <typename CT>
__device__ __forceinline__ CT bin_op(int op, CT a, CT b)
{
    switch (op) {
    case PT_OP_ADD: return a + b;
    case PT_OP_SUB: return a - b;
    case PT_OP_MUL: return a * b;
    case PT_OP_DIV:
        if constexpr ((CT)0.5 == (CT)0) return b == (CT)0 ? (CT)0 : a / b;
        else return a / b;
    case PT_OP_POW: return pow_op<CT>(a, b);
    case PT_OP_MAXIMUM: return a > b ? a : b;
    case PT_OP_MINIMUM: return a < b ? a : b;
    case PT_OP_GT: return a > b ? (CT)1 : (CT)0;
    case PT_OP_LT: return a < b ? (CT)1 : (CT)0;
    case PT_OP_EQ: return a == b ? (CT)1 : (CT)0;
    case PT_OP_NE: return a != b ? (CT)1 : (CT)0;
    case PT_OP_GE: return a >= b ? (CT)1 : (CT)0;
    case PT_OP_LE: return a <= b ? (CT)1 : (CT)0;
    default: return (CT)0;
    }
}

// 32-bit integer outputs narrower than 64 bits evaluate in int64/uint64 and
// truncate on store, which equals wrapping arithmetic in the narrow type for
// + - * (modular), and is exact for comparisons / max / min.

template <typename SH, typename IT>
__device__ __forceinline__ IT offset_of(const SH &s, const IT *st, IT i)
{
    IT off = 0;
    for (int d = s.ndims - 1; d >= 0; d--) {
        IT e = s.shape[d];
        IT q = i / e;
        off += (i - q * e) * st[d];
        i = q;
    }
    return off;
}

// SH: EwShape (64-bit indices) or EwShape32.
template <typename CT, typename SH>
__global__ __launch_bounds__(256) void k_binary(const void *__restrict__ a, int dta,
                                                const void *__restrict__ b, int dtb,
                                                void *__restrict__ out, int dto, int op,
                                                SH s, int b_scalar, CT scalar, int reverse)
{
    using IT = decltype(s.total);
    IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x;
    const IT stride = (IT)gridDim.x * blockDim.x;
    for (; i < s.total; i += stride) {
        CT x = ld<CT>(a, dta, offset_of(s, s.sa, i));
        CT y = b_scalar ? scalar : ld<CT>(b, dtb, offset_of(s, s.sb, i));
        st<CT>(out, dto, i, reverse ? bin_op<CT>(op, y, x) : bin_op<CT>(op, x, y));
    }
}

// All-contiguous float32 fast path: 4 elements per thread per step.
__global__ __launch_bounds__(256) void k_binary_f32_contig(const float *__restrict__ a,
                                                           const float *__restrict__ b,
                                                           float *__restrict__ out, int op,
                                                           long long n, int b_scalar, float scalar,
                                                           int reverse)
{
    long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const long long stride = (long long)gridDim.x * blockDim.x * 4;
    for (; i < n; i += stride) {
        if (i + 4 <= n) {
            f32x4 x = ld_stream(a + i);
            f32x4 y = b_scalar ? (f32x4){scalar, scalar, scalar, scalar} : ld_stream(b + i);
            f32x4 r;
            if (reverse) {
                r.x = bin_op<float>(op, y.x, x.x); r.y = bin_op<float>(op, y.y, x.y);
                r.z = bin_op<float>(op, y.z, x.z); r.w = bin_op<float>(op, y.w, x.w);
            } else {
                r.x = bin_op<float>(op, x.x, y.x); r.y = bin_op<float>(op, x.y, y.y);
                r.z = bin_op<float>(op, x.z, y.z); r.w = bin_op<float>(op, x.w, y.w);
            }
            st_stream(out + i, r);
        } else {
            for (long long j = i; j < n; j++) {
                float x = a[j], y = b_scalar ? scalar : b[j];
                out[j] = reverse ? bin_op<float>(op, y, x) : bin_op<float>(op, x, y);
            }
        }
    }
}

// float32 operands over a 2-D [rows, cols] output (cols a multiple of 4):
// each operand either walks the row (column stride 1, 16-byte loads) or
// holds one value per row (column stride 0); its row stride may be 0 (a
// broadcast row).  Operands read once per output element stream past the
// caches (nontemporal); broadcast ones use ordinary loads.
__device__ __forceinline__ f32x4 ld_row4(const float *p, unsigned ro, unsigned c, int inner, bool stream)
{
    if (!inner) {
        const float v = p[ro];
        return (f32x4){v, v, v, v};
    }
    return stream ? ld_stream(p + ro + c) : *(const f32x4 *)(p + ro + c);
}

__global__ __launch_bounds__(256) void k_binary_f32_rows(const float *__restrict__ a, const float *__restrict__ b,
                                                         float *__restrict__ out, int op, unsigned rows,
                                                         unsigned cols4, unsigned ra, int ia, unsigned rb, int ib,
                                                         int reverse)
{
    const unsigned g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= rows * cols4) return;
    const unsigned r = g / cols4, c = (g - r * cols4) * 4;
    const f32x4 x = ld_row4(a, r * ra, c, ia, ia && ra != 0);
    const f32x4 y = ld_row4(b, r * rb, c, ib, ib && rb != 0);
    f32x4 v;
    if (reverse) {
        v.x = bin_op<float>(op, y.x, x.x); v.y = bin_op<float>(op, y.y, x.y);
        v.z = bin_op<float>(op, y.z, x.z); v.w = bin_op<float>(op, y.w, x.w);
    } else {
        v.x = bin_op<float>(op, x.x, y.x); v.y = bin_op<float>(op, x.y, y.y);
        v.z = bin_op<float>(op, x.z, y.z); v.w = bin_op<float>(op, x.w, y.w);
    }
    st_stream(out + (size_t)g * 4, v);
}

// ------------------------------------------------------------------ unary
template <typename CT>
__device__ __forceinline__ CT unary_f(int op, CT v)
{
    constexpr bool F = sizeof(CT) == 4;
    switch (op) {
    case PT_OP_EXP: return F ? expf(v) : exp(v);
    case PT_OP_EXPM1: return F ? expm1f(v) : expm1(v);
    case PT_OP_EXP2: return F ? exp2f(v) : exp2(v);
    case PT_OP_LOG: return F ? logf(v) : log(v);
    case PT_OP_LOG1P: return F ? log1pf(v) : log1p(v);
    case PT_OP_LOG2: return F ? log2f(v) : log2(v);
    case PT_OP_LOG10: return F ? log10f(v) : log10(v);
    case PT_OP_SQRT: return F ? sqrtf(v) : sqrt(v);
    case PT_OP_SIN: return F ? sinf(v) : sin(v);
    case PT_OP_COS: return F ? cosf(v) : cos(v);
    case PT_OP_TAN: return F ? tanf(v) : tan(v);
    case PT_OP_ASIN: return F ? asinf(v) : asin(v);
    case PT_OP_ACOS: return F ? acosf(v) : acos(v);
    case PT_OP_ATAN: return F ? atanf(v) : atan(v);
    case PT_OP_SINH: return F ? sinhf(v) : sinh(v);
    case PT_OP_COSH: return F ? coshf(v) : cosh(v);
    case PT_OP_TANH: return F ? tanhf(v) : tanh(v);
    case PT_OP_ABS: return v < (CT)0 ? -v : v;
    case PT_OP_NEG: return -v;
    case PT_OP_FLOOR: return F ? floorf(v) : floor(v);
    case PT_OP_CEIL: return F ? ceilf(v) : ceil(v);
    case PT_OP_ROUND: return F ? roundf(v) : round(v);
    default: return v;
    }
}

template <typename CT, typename SH>
__global__ __launch_bounds__(256) void k_unary(const void *__restrict__ x, int dt,
                                               void *__restrict__ out, int op, SH s)
{
    using IT = decltype(s.total);
    IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x;
    const IT stride = (IT)gridDim.x * blockDim.x;
    for (; i < s.total; i += stride) {
        IT off = offset_of(s, s.sa, i);
        if constexpr (sizeof(CT) == 8 && (CT)0.5 == (CT)0) {
            // integers: abs/neg exact, floor/ceil/round identity, the rest
            // through float (cuda_op_functors.cuh:153-449)
            CT v = ld<CT>(x, dt, off);
            CT r;
            if (op == PT_OP_ABS) r = v < (CT)0 ? (CT)0 - v : v;
            else if (op == PT_OP_NEG) r = (CT)0 - v;
            else if (op == PT_OP_FLOOR || op == PT_OP_CEIL || op == PT_OP_ROUND) r = v;
            else r = (CT)unary_f<float>(op, (float)v);
            st<CT>(out, dt, i, r);
        } else {
            st<CT>(out, dt, i, unary_f<CT>(op, ld<CT>(x, dt, off)));
        }
    }
}

// OPC >= 0: the op fixed at compile time (the per-element dispatch folds
// away); OPC < 0: the op comes from `op`.
template <int OPC>
__global__ __launch_bounds__(256) void k_unary_f32_contig(const float *__restrict__ x,
                                                          float *__restrict__ out, int op_arg, long long n)
{
    const int op = OPC >= 0 ? OPC : op_arg;
    long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const long long stride = (long long)gridDim.x * blockDim.x * 4;
    for (; i < n; i += stride) {
        if (i + 4 <= n) {
            f32x4 v = ld_stream(x + i);
            f32x4 r;
            r.x = unary_f<float>(op, v.x); r.y = unary_f<float>(op, v.y);
            r.z = unary_f<float>(op, v.z); r.w = unary_f<float>(op, v.w);
            st_stream(out + i, r);
        } else {
            for (long long j = i; j < n; j++) out[j] = unary_f<float>(op, x[j]);
        }
    }
}

// --------------------------------------------------------- cast / where
// Casts follow the reference's converting kernels: to f16/bf16 through
// float with RNE, floats to integers by C conversion, anything to bool by
// != 0 (factory_kernels.cu:128-163).
__device__ __forceinline__ void cast_elem(const void *x, int dti, long long oi, void *out, int dto,
                                          long long i)
{
    if (dti == dto) {
        switch (dtype_size(dti)) {
        case 1: ((uint8_t *)out)[i] = ((const uint8_t *)x)[oi]; return;
        case 2: ((uint16_t *)out)[i] = ((const uint16_t *)x)[oi]; return;
        case 4: ((uint32_t *)out)[i] = ((const uint32_t *)x)[oi]; return;
        default: ((uint64_t *)out)[i] = ((const uint64_t *)x)[oi]; return;
        }
    }
    const bool src_int64 = dti == PT_INT64, src_u64 = dti == PT_UINT64;
    if (src_int64) { st<long long>(out, dto, i, ((const int64_t *)x)[oi]); return; }
    if (src_u64) { st<unsigned long long>(out, dto, i, ((const uint64_t *)x)[oi]); return; }
    if (dto == PT_INT64) { st<long long>(out, dto, i, (long long)ld<double>(x, dti, oi)); return; }
    if (dto == PT_UINT64) { st<unsigned long long>(out, dto, i, (unsigned long long)ld<double>(x, dti, oi)); return; }
    st<double>(out, dto, i, ld<double>(x, dti, oi));
}

template <typename SH>
__global__ __launch_bounds__(256) void k_cast(const void *__restrict__ x, int dti,
                                              void *__restrict__ out, int dto, SH s)
{
    using IT = decltype(s.total);
    IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x;
    const IT stride = (IT)gridDim.x * blockDim.x;
    for (; i < s.total; i += stride) cast_elem(x, dti, (long long)offset_of(s, s.sa, i), out, dto, (long long)i);
}

template <typename SH>
__global__ __launch_bounds__(256) void k_where(const void *__restrict__ c, int dtc,
                                               const void *__restrict__ x, const void *__restrict__ y,
                                               int esz, void *__restrict__ out, SH s)
{
    using IT = decltype(s.total);
    IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x;
    const IT stride = (IT)gridDim.x * blockDim.x;
    for (; i < s.total; i += stride) {
        const IT co = offset_of(s, s.sc, i);
        bool pick = ld<double>(c, dtc, co) != 0.0;
        if (dtc == PT_INT64 || dtc == PT_UINT64) pick = ((const uint64_t *)c)[co] != 0;
        const void *src = pick ? x : y;
        IT o = offset_of(s, pick ? s.sa : s.sb, i);
        switch (esz) {
        case 1: ((uint8_t *)out)[i] = ((const uint8_t *)src)[o]; break;
        case 2: ((uint16_t *)out)[i] = ((const uint16_t *)src)[o]; break;
        case 4: ((uint32_t *)out)[i] = ((const uint32_t *)src)[o]; break;
        default: ((uint64_t *)out)[i] = ((const uint64_t *)src)[o]; break;
        }
    }
}

__global__ __launch_bounds__(256) void k_fill(void *__restrict__ out, int esz, long long n, uint64_t bits)
{
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        switch (esz) {
        case 1: ((uint8_t *)out)[i] = (uint8_t)bits; break;
        case 2: ((uint16_t *)out)[i] = (uint16_t)bits; break;
        case 4: ((uint32_t *)out)[i] = (uint32_t)bits; break;
        default: ((uint64_t *)out)[i] = bits; break;
        }
    }
}

// ------------------------------------------------------------------ host
static unsigned grid_for(long long n, int per_thread = 1)
{
    // one thread per work item: a full grid streams HBM faster on gfx950
    // than a capped grid-stride loop; the loops cover grids above the limit
    long long blocks = (n + 256LL * per_thread - 1) / (256LL * per_thread);
    if (blocks > 0x7fffffffLL) blocks = 0x7fffffffLL;
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

static bool valid_binary_op(int op)
{
    return (op >= PT_OP_ADD && op <= PT_OP_POW) || (op >= PT_OP_GT && op <= PT_OP_LE) ||
           op == PT_OP_MAXIMUM || op == PT_OP_MINIMUM;
}

static bool valid_unary_op(int op)
{
    return (op >= PT_OP_EXP && op <= PT_OP_NEG) || (op >= PT_OP_CEIL && op <= PT_OP_ROUND);
}

// scalar value converted to a compute class
static double scalar_as_double(const pt_scalar_t *s)
{
    switch (s->dtype) {
    case PT_FLOAT32: return s->v.f32;
    case PT_FLOAT64: return s->v.f64;
    case PT_FLOAT16: {
        uint16_t h = s->v.u16;
        _Float16 f;
        memcpy(&f, &h, 2);
        return (double)f;
    }
    case PT_BFLOAT16: {
        uint32_t b = (uint32_t)s->v.u16 << 16;
        float f;
        memcpy(&f, &b, 4);
        return f;
    }
    case PT_UINT8: case PT_UINT16: case PT_UINT32: case PT_UINT64: case PT_BOOL:
        return (double)s->v.u64;
    default: return (double)s->v.i64;
    }
}

static long long scalar_as_i64(const pt_scalar_t *s)
{
    if (dtype_is_floating(s->dtype)) return (long long)scalar_as_double(s);
    return s->v.i64;
}

// The 2-D float32 row kernel applies: 1 or 2 collapsed dims, a column
// count that is a multiple of 4, each operand's column stride 0 or 1, and
// 16-byte aligned rows for the operands that walk them.
static bool rows_f32(const EwShape &s, const void *pa, const void *pb, const void *out)
{
    if (s.ndims < 1 || s.ndims > 2 || s.total > 0x7fffffffLL) return false;
    const long long cols = s.shape[s.ndims - 1];
    if (cols % 4 || ((uintptr_t)out & 15)) return false;
    const long long ia = s.sa[s.ndims - 1], ib = s.sb[s.ndims - 1];
    const long long ra = s.ndims == 2 ? s.sa[0] : 0, rb = s.ndims == 2 ? s.sb[0] : 0;
    if ((ia != 0 && ia != 1) || (ib != 0 && ib != 1)) return false;
    if (ia == 1 && (((uintptr_t)pa & 15) || ra % 4)) return false;
    if (ib == 1 && (((uintptr_t)pb & 15) || rb % 4)) return false;
    const long long rows = s.ndims == 2 ? s.shape[0] : 1;
    // largest offsets stay in 32 bits
    if ((rows - 1) * ra + cols > 0x7fffffffLL || (rows - 1) * rb + cols > 0x7fffffffLL) return false;
    return true;
}

static pt_status binary_impl(const void *a, int dta, const size_t *sa, size_t offa,
                             const void *b, int dtb, const size_t *sb, size_t offb,
                             const pt_scalar_t *scalar, int reverse, void *out, int dto, int op,
                             const int *shape, int ndims, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!dtype_valid(dta) || !dtype_valid(dto) || (!scalar && !dtype_valid(dtb)))
        return fail(PT_ERR_INVALID, "elementwise: unknown dtype");
    if (!valid_binary_op(op)) return fail(PT_ERR_INVALID, "elementwise: unsupported op %d", op);
    if (ndims < 0 || ndims > PT_MAX_DIMS) return fail(PT_ERR_INVALID, "elementwise: rank %d", ndims);
    size_t cstr[PT_MAX_DIMS];
    size_t acc = 1;
    for (int d = ndims - 1; d >= 0; d--) {
        if (shape[d] < 0) return fail(PT_ERR_INVALID, "elementwise: negative extent");
        cstr[d] = acc;
        acc *= (size_t)shape[d];
    }
    EwShape s;
    collapse(shape, ndims, sa, scalar ? nullptr : sb, cstr, s);
    if (s.total == 0) return PT_OK;
    hipStream_t st_ = stream_of(stream);
    const char *pa = (const char *)a + offa * dtype_size(dta);
    const char *pb = scalar ? nullptr : (const char *)b + offb * dtype_size(dtb);
    bool contig = s.ndims <= 1 && (s.ndims == 0 || (s.sa[0] == 1 && (scalar || s.sb[0] == 1)));
    if (contig && dta == PT_FLOAT32 && (scalar || dtb == PT_FLOAT32) && dto == PT_FLOAT32 &&
        ((uintptr_t)pa & 15) == 0 && (scalar || ((uintptr_t)pb & 15) == 0) &&
        ((uintptr_t)out & 15) == 0) {
        float sv = scalar ? (float)scalar_as_double(scalar) : 0.0f;
        k_binary_f32_contig<<<grid_for(s.total, 4), 256, 0, st_>>>(
            (const float *)pa, (const float *)pb, (float *)out, op, s.total, scalar != nullptr, sv, reverse);
    } else if (!scalar && dta == PT_FLOAT32 && dtb == PT_FLOAT32 && dto == PT_FLOAT32 &&
               rows_f32(s, pa, pb, out)) {
        // 2-D row/column broadcasts of float32 (bias adds, row scalings)
        const unsigned rows = s.ndims == 2 ? (unsigned)s.shape[0] : 1u;
        const unsigned cols = (unsigned)s.shape[s.ndims - 1];
        const long long ra = s.ndims == 2 ? s.sa[0] : 0, rb = s.ndims == 2 ? s.sb[0] : 0;
        const unsigned n4 = rows * (cols / 4);
        k_binary_f32_rows<<<(n4 + 255) / 256, 256, 0, st_>>>((const float *)pa, (const float *)pb, (float *)out,
                                                              op, rows, cols / 4, (unsigned)ra,
                                                              (int)s.sa[s.ndims - 1], (unsigned)rb,
                                                              (int)s.sb[s.ndims - 1], reverse);
    } else {
        EwShape32 s32;
        const bool i32 = to32(s, s32);
#define PT_BIN(CT, SV)                                                                                          \
    (i32 ? (k_binary<CT, EwShape32><<<grid_for(s.total), 256, 0, st_>>>(pa, dta, pb, dtb, out, dto, op, s32, \
                                                                          scalar != nullptr, SV, reverse), 0) \
         : (k_binary<CT, EwShape><<<grid_for(s.total), 256, 0, st_>>>(pa, dta, pb, dtb, out, dto, op, s,     \
                                                                        scalar != nullptr, SV, reverse), 0))
        switch (compute_class(dto)) {
        case CT_F32: PT_BIN(float, scalar ? (float)scalar_as_double(scalar) : 0.0f); break;
        case CT_F64: PT_BIN(double, scalar ? scalar_as_double(scalar) : 0.0); break;
        case CT_I64: PT_BIN(long long, scalar ? scalar_as_i64(scalar) : 0LL); break;
        default: PT_BIN(unsigned long long, scalar ? (unsigned long long)scalar_as_i64(scalar) : 0ULL); break;
        }
#undef PT_BIN
    }
    PT_LAUNCH_CHECK("elementwise binary");
    counters().elementwise_calls++;
    return PT_OK;
}

}  // namespace pt

using namespace pt;

extern "C" {

pt_status pt_broadcast(const void *a, int dtype_a, const size_t *strides_a, size_t offset_a,
                       const void *b, int dtype_b, const size_t *strides_b, size_t offset_b,
                       void *out, int dtype_out, int op,
                       const int *shape, int ndims, pt_stream_t stream)
{
    return binary_impl(a, dtype_a, strides_a, offset_a, b, dtype_b, strides_b, offset_b, nullptr,
                       0, out, dtype_out, op, shape, ndims, stream);
}

pt_status pt_scalar(const void *input, int dtype_in, const size_t *strides, size_t offset,
                    const pt_scalar_t *scalar, int reverse, void *out, int dtype_out,
                    int op, const int *shape, int ndims, pt_stream_t stream)
{
    if (!scalar) return fail(PT_ERR_INVALID, "pt_scalar: missing scalar");
    return binary_impl(input, dtype_in, strides, offset, nullptr, dtype_in, nullptr, 0, scalar,
                       reverse, out, dtype_out, op, shape, ndims, stream);
}

pt_status pt_unary(const void *input, int dtype, const size_t *strides, size_t offset,
                   void *out, int op, const int *shape, int ndims, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!dtype_valid(dtype)) return fail(PT_ERR_INVALID, "unary: unknown dtype");
    if (!valid_unary_op(op)) return fail(PT_ERR_INVALID, "unary: unsupported op %d", op);
    if (ndims < 0 || ndims > PT_MAX_DIMS) return fail(PT_ERR_INVALID, "unary: rank %d", ndims);
    size_t cstr[PT_MAX_DIMS], acc = 1;
    for (int d = ndims - 1; d >= 0; d--) { cstr[d] = acc; acc *= (size_t)shape[d]; }
    EwShape s;
    collapse(shape, ndims, strides, nullptr, cstr, s);
    if (s.total == 0) return PT_OK;
    hipStream_t st_ = stream_of(stream);
    const char *px = (const char *)input + offset * dtype_size(dtype);
    bool contig = s.ndims <= 1 && (s.ndims == 0 || s.sa[0] == 1);
    if (contig && dtype == PT_FLOAT32 && ((uintptr_t)px & 15) == 0 && ((uintptr_t)out & 15) == 0) {
        const unsigned g = grid_for(s.total, 4);
        if (op == PT_OP_TANH)
            k_unary_f32_contig<PT_OP_TANH><<<g, 256, 0, st_>>>((const float *)px, (float *)out, op, s.total);
        else if (op == PT_OP_EXP)
            k_unary_f32_contig<PT_OP_EXP><<<g, 256, 0, st_>>>((const float *)px, (float *)out, op, s.total);
        else
            k_unary_f32_contig<-1><<<g, 256, 0, st_>>>((const float *)px, (float *)out, op, s.total);
    } else {
        EwShape32 s32;
        const bool i32 = to32(s, s32);
#define PT_UN(CT)                                                                                     \
    (i32 ? (k_unary<CT, EwShape32><<<grid_for(s.total), 256, 0, st_>>>(px, dtype, out, op, s32), 0) \
         : (k_unary<CT, EwShape><<<grid_for(s.total), 256, 0, st_>>>(px, dtype, out, op, s), 0))
        switch (compute_class(dtype)) {
        case CT_F32: PT_UN(float); break;
        case CT_F64: PT_UN(double); break;
        case CT_I64: PT_UN(long long); break;
        default: PT_UN(unsigned long long); break;
        }
#undef PT_UN
    }
    PT_LAUNCH_CHECK("unary");
    counters().elementwise_calls++;
    return PT_OK;
}

pt_status pt_cast(const void *input, int dtype_in, const size_t *strides, size_t offset,
                  void *out, int dtype_out, const int *shape, int ndims, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!dtype_valid(dtype_in) || !dtype_valid(dtype_out)) return fail(PT_ERR_INVALID, "cast: unknown dtype");
    if (ndims < 0 || ndims > PT_MAX_DIMS) return fail(PT_ERR_INVALID, "cast: rank %d", ndims);
    size_t cstr[PT_MAX_DIMS], acc = 1;
    for (int d = ndims - 1; d >= 0; d--) { cstr[d] = acc; acc *= (size_t)shape[d]; }
    EwShape s;
    collapse(shape, ndims, strides, nullptr, cstr, s);
    if (s.total == 0) return PT_OK;
    hipStream_t st_ = stream_of(stream);
    const char *px = (const char *)input + offset * dtype_size(dtype_in);
    bool contig = s.ndims <= 1 && (s.ndims == 0 || s.sa[0] == 1);
    if (contig && dtype_in == dtype_out) {
        PT_TRY(check_hip(hipMemcpyAsync(out, px, (size_t)s.total * dtype_size(dtype_in),
                                        hipMemcpyDeviceToDevice, st_), "cast copy"));
        return PT_OK;
    }
    EwShape32 s32;
    if (to32(s, s32)) k_cast<EwShape32><<<grid_for(s.total), 256, 0, st_>>>(px, dtype_in, out, dtype_out, s32);
    else k_cast<EwShape><<<grid_for(s.total), 256, 0, st_>>>(px, dtype_in, out, dtype_out, s);
    PT_LAUNCH_CHECK("cast");
    counters().elementwise_calls++;
    return PT_OK;
}

pt_status pt_where(const void *cond, int dtype_cond, const size_t *strides_cond,
                   const void *x, const size_t *strides_x,
                   const void *y, const size_t *strides_y, int dtype_xy,
                   void *out, const int *shape, int ndims, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!dtype_valid(dtype_cond) || !dtype_valid(dtype_xy)) return fail(PT_ERR_INVALID, "where: unknown dtype");
    if (ndims < 0 || ndims > PT_MAX_DIMS) return fail(PT_ERR_INVALID, "where: rank %d", ndims);
    EwShape s;
    collapse(shape, ndims, strides_x, strides_y, strides_cond, s);
    if (s.total == 0) return PT_OK;
    hipStream_t st_ = stream_of(stream);
    EwShape32 s32;
    if (to32(s, s32))
        k_where<EwShape32><<<grid_for(s.total), 256, 0, st_>>>(cond, dtype_cond, x, y, (int)dtype_size(dtype_xy), out,
                                                               s32);
    else
        k_where<EwShape><<<grid_for(s.total), 256, 0, st_>>>(cond, dtype_cond, x, y, (int)dtype_size(dtype_xy), out, s);
    PT_LAUNCH_CHECK("where");
    counters().elementwise_calls++;
    return PT_OK;
}

pt_status pt_fill(void *out, int dtype, size_t n, const pt_scalar_t *value, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!dtype_valid(dtype) || !value) return fail(PT_ERR_INVALID, "fill: bad arguments");
    if (!n) return PT_OK;
    uint64_t bits = 0;
    double d = scalar_as_double(value);
    long long iv = scalar_as_i64(value);
    switch (dtype) {
    case PT_FLOAT32: { float f = (float)d; memcpy(&bits, &f, 4); break; }
    case PT_FLOAT64: memcpy(&bits, &d, 8); break;
    case PT_FLOAT16: { _Float16 h = (_Float16)(float)d; uint16_t u; memcpy(&u, &h, 2); bits = u; break; }
    case PT_BFLOAT16: {
        float f = (float)d;
        uint32_t u;
        memcpy(&u, &f, 4);
        bits = ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) ? ((u >> 16) | 0x40u)
                                                                       : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        break;
    }
    case PT_BOOL: bits = d != 0.0; break;
    default: bits = dtype_is_floating(value->dtype) ? (uint64_t)(long long)d : (uint64_t)iv; break;
    }
    k_fill<<<grid_for((long long)n), 256, 0, stream_of(stream)>>>(out, (int)dtype_size(dtype), (long long)n, bits);
    PT_LAUNCH_CHECK("fill");
    return PT_OK;
}

}  // extern "C"
