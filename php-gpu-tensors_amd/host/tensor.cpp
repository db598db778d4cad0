// Tensor lifecycle, dtype rules, views and transfers of the host runtime.
// Mirrors src/tensor.c, src/data_types.c, src/tensor_shape.h and
// src/cuda_array/tensor_transfer.c of the reference; device memory and
// copies go through the C-ABI (pt_alloc / pt_memcpy_* / pt_cast).
#include "runtime.hpp"

#include <algorithm>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <strings.h>

#include <atomic>

namespace phpt {

// ------------------------------------------------------------------ errors
static thread_local int t_kind = ERR_NONE;
static thread_local char t_msg[1024];

static void vset(int kind, const char *fmt, va_list ap)
{
    t_kind = kind;
    vsnprintf(t_msg, sizeof(t_msg), fmt, ap);
}

void set_invalid(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vset(ERR_INVALID, fmt, ap);
    va_end(ap);
}

void set_runtime(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vset(ERR_RUNTIME, fmt, ap);
    va_end(ap);
}

void clear_error()
{
    t_kind = ERR_NONE;
    t_msg[0] = 0;
}

int error_kind() { return t_kind; }
const char *error_message() { return t_msg; }

static thread_local pt_status t_last_status = PT_OK;
pt_status last_failed_status() { return t_last_status; }
void reset_failed_status() { t_last_status = PT_OK; }

bool check_status(pt_status st, const char *what)
{
    if (st == PT_OK) return true;
    t_last_status = st;
    const char *detail = pt_last_error();
    if (st == PT_ERR_INVALID) set_invalid("%s", detail && *detail ? detail : what);
    else set_runtime("%s: %s", what, detail ? detail : pt_status_string(st));
    return false;
}

// ------------------------------------------------------------------ dtypes
size_t dtype_size(int dt)
{
    switch (dt) {
    case PT_FLOAT32: case PT_INT32: case PT_UINT32: return 4;
    case PT_FLOAT64: case PT_INT64: case PT_UINT64: return 8;
    case PT_INT16: case PT_UINT16: case PT_FLOAT16: case PT_BFLOAT16: return 2;
    case PT_INT8: case PT_UINT8: case PT_BOOL: return 1;
    default: return 0;
    }
}

bool is_valid_dtype(int dt) { return dtype_size(dt) != 0; }
bool is_floating(int dt)
{
    return dt == PT_FLOAT32 || dt == PT_FLOAT64 || dt == PT_FLOAT16 || dt == PT_BFLOAT16;
}
bool is_integer(int dt) { return dt >= PT_INT8 && dt <= PT_UINT64; }
bool is_signed(int dt) { return is_floating(dt) || (dt >= PT_INT8 && dt <= PT_INT64); }

static const char *kNames[] = {"float32", "float64", "int8", "int16", "int32", "int64", "uint8",
                               "uint16", "uint32", "uint64", "bool", "float16", "bfloat16"};

const char *dtype_name(int dt) { return is_valid_dtype(dt) ? kNames[dt] : "unknown"; }

// Accepted spellings follow dtype_from_string (data_types.c:162-248).
int dtype_from_name(const char *name)
{
    if (!name || !*name) return PT_FLOAT32;
    struct Alias { const char *s; int dt; };
    static const Alias aliases[] = {
        {"float32", PT_FLOAT32}, {"float", PT_FLOAT32}, {"f32", PT_FLOAT32}, {"single", PT_FLOAT32},
        {"float64", PT_FLOAT64}, {"double", PT_FLOAT64}, {"f64", PT_FLOAT64},
        {"float16", PT_FLOAT16}, {"half", PT_FLOAT16}, {"f16", PT_FLOAT16},
        {"bfloat16", PT_BFLOAT16}, {"bf16", PT_BFLOAT16},
        {"int8", PT_INT8}, {"char", PT_INT8}, {"i8", PT_INT8},
        {"int16", PT_INT16}, {"short", PT_INT16}, {"i16", PT_INT16},
        {"int32", PT_INT32}, {"int", PT_INT32}, {"i32", PT_INT32},
        {"int64", PT_INT64}, {"long", PT_INT64}, {"i64", PT_INT64},
        {"uint8", PT_UINT8}, {"uchar", PT_UINT8}, {"u8", PT_UINT8},
        {"uint16", PT_UINT16}, {"ushort", PT_UINT16}, {"u16", PT_UINT16},
        {"uint32", PT_UINT32}, {"uint", PT_UINT32}, {"u32", PT_UINT32},
        {"uint64", PT_UINT64}, {"ulong", PT_UINT64}, {"u64", PT_UINT64},
        {"bool", PT_BOOL}, {"boolean", PT_BOOL},
    };
    for (const Alias &a : aliases)
        if (strcasecmp(name, a.s) == 0) return a.dt;
    return -1;
}

long double Scalar::as_ld() const
{
    if (is_floating(dtype)) return f;
    if (dtype == PT_BOOL || (dtype >= PT_UINT8 && dtype <= PT_UINT64)) return (long double)u;
    return (long double)i;
}

Scalar scalar_from_double(double v)
{
    Scalar s;
    s.dtype = PT_FLOAT64;
    s.f = v;
    s.is_neg = v < 0;
    return s;
}

Scalar scalar_from_int(int64_t v)
{
    Scalar s;
    s.dtype = PT_INT64;
    s.i = v;
    s.is_neg = v < 0;
    return s;
}

Scalar scalar_from_bool(bool v)
{
    Scalar s;
    s.dtype = PT_BOOL;
    s.u = v ? 1 : 0;
    return s;
}

static uint16_t f32_to_bf16_bits(float v)
{
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static float bf16_bits_to_f32(uint16_t b)
{
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// binary16 round to nearest even (finite, infinite and NaN inputs), the
// rounding of float_to_float16_bits (data_types.c:46-80).
static uint16_t f32_to_f16_bits(float v)
{
    uint32_t u;
    memcpy(&u, &v, 4);
    uint32_t sign = (u >> 16) & 0x8000u, e = (u >> 23) & 0xffu, m = u & 0x7fffffu;
    if (e == 0xffu) {
        uint32_t payload = m >> 13;
        if (m && !payload) payload = 1;
        return (uint16_t)(sign | 0x7c00u | payload);
    }
    int he = (int)e - 112;
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)sign;
        uint32_t full = m | 0x800000u;
        int shift = 14 - he;
        uint32_t q = full >> shift, rem = full & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)he << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static float f16_bits_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (!e) {
        if (!m) {
            bits = sign;
        } else {
            int ex = -14;
            while (!(m & 0x400u)) {
                m <<= 1;
                ex--;
            }
            bits = sign | ((uint32_t)(ex + 127) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float round_f16(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }

// cast_single_value (data_types.c:373-436): integer targets reject values
// outside [-2^(bits-1), 2^(bits-1)) or [0, 2^bits); float targets round.
bool cast_scalar(const Scalar &in, int target, Scalar &out)
{
    if (!is_valid_dtype(target) || !is_valid_dtype(in.dtype)) return false;
    long double v = in.as_ld();
    if (in.dtype == target) {
        out = in;
        return true;
    }
    if (is_integer(target)) {
        bool sgn = is_signed(target);
        long double limit = ldexpl(1.0L, (int)(8 * dtype_size(target)) - (sgn ? 1 : 0));
        if (!isfinite(v) || v < (sgn ? -limit : 0) || v >= limit) return false;
    }
    Scalar r;
    r.dtype = target;
    switch (target) {
    case PT_FLOAT32: r.f = (float)v; r.is_neg = r.f < 0; break;
    case PT_FLOAT64: r.f = (double)v; r.is_neg = r.f < 0; break;
    case PT_FLOAT16: r.f = round_f16((float)v); r.is_neg = v < 0; break;
    case PT_BFLOAT16: r.f = bf16_bits_to_f32(f32_to_bf16_bits((float)v)); r.is_neg = v < 0; break;
    case PT_BOOL: r.u = v != 0; break;
    case PT_INT8: r.i = (int8_t)v; r.is_neg = r.i < 0; break;
    case PT_INT16: r.i = (int16_t)v; r.is_neg = v < 0; break;
    case PT_INT32: r.i = (int32_t)v; r.is_neg = r.i < 0; break;
    case PT_INT64: r.i = (int64_t)v; r.is_neg = r.i < 0; break;
    case PT_UINT8: r.u = (uint8_t)v; break;
    case PT_UINT16: r.u = (uint16_t)v; break;
    case PT_UINT32: r.u = (uint32_t)v; break;
    case PT_UINT64: r.u = (uint64_t)v; break;
    default: return false;
    }
    out = r;
    return true;
}

pt_scalar_t to_pt_scalar(const Scalar &s)
{
    pt_scalar_t p;
    memset(&p, 0, sizeof(p));
    p.dtype = s.dtype;
    switch (s.dtype) {
    case PT_FLOAT32: p.v.f32 = (float)s.f; break;
    case PT_FLOAT64: p.v.f64 = s.f; break;
    case PT_FLOAT16: p.v.u16 = f32_to_f16_bits((float)s.f); break;
    case PT_BFLOAT16: p.v.u16 = f32_to_bf16_bits((float)s.f); break;
    case PT_BOOL: case PT_UINT8: case PT_UINT16: case PT_UINT32: case PT_UINT64: p.v.u64 = s.u; break;
    default: p.v.i64 = s.i; break;
    }
    return p;
}

// promote_types (data_types.c:301-349)
int promote_types(int a, int b)
{
    if (!is_valid_dtype(a) || !is_valid_dtype(b)) return -1;
    if (a == b) return a;
    bool a_half = a == PT_FLOAT16 || a == PT_BFLOAT16, b_half = b == PT_FLOAT16 || b == PT_BFLOAT16;
    if (is_floating(a) && is_floating(b) && (a_half || b_half)) {
        if (a_half) return b_half ? PT_FLOAT32 : b;
        return a;
    }
    if (a == PT_BOOL) return b;
    if (b == PT_BOOL) return a;
    if (is_floating(a) && is_integer(b)) return a;
    if (is_integer(a) && is_floating(b)) return b;
    if (is_integer(a) && is_integer(b)) {
        bool sa = is_signed(a), sb = is_signed(b);
        if (sa == sb) return dtype_size(a) > dtype_size(b) ? a : b;
        int st = sa ? a : b, ut = sa ? b : a;
        if (dtype_size(st) > dtype_size(ut)) return st;
        switch (ut) {
        case PT_UINT8: return PT_INT16;
        case PT_UINT16: return PT_INT32;
        case PT_UINT32: return PT_INT64;
        default: return -1;
        }
    }
    return (a == PT_FLOAT64 || b == PT_FLOAT64) ? PT_FLOAT64 : PT_FLOAT32;
}

// promote_scalar_for_arithmetic (data_types.c:438-490)
int promote_scalar_for_arithmetic(int t, int s, int op, bool is_neg)
{
    if (!is_valid_dtype(t) || !is_valid_dtype(s)) return -1;
    if (is_integer(t) && is_integer(s) && is_signed(t) != is_signed(s) &&
        (t == PT_UINT64 || s == PT_UINT64))
        return -1;
    if (op == PT_OP_MAXIMUM || op == PT_OP_MINIMUM) return t == s ? t : promote_types(t, s);
    if (op == PT_OP_DIV || (op == PT_OP_POW && is_neg)) {
        if (t == PT_FLOAT64 || t == PT_INT64 || t == PT_UINT64) return PT_FLOAT64;
        return PT_FLOAT32;
    }
    if (t == s) return t;
    if (t == PT_BOOL) return is_floating(s) ? PT_FLOAT32 : PT_INT32;
    if (is_floating(t)) return t;
    if (is_integer(t) && is_floating(s)) return dtype_size(t) == 8 ? PT_FLOAT64 : PT_FLOAT32;
    return t;
}

// promote_types_for_arithmetic (data_types.c:492-516)
int promote_types_for_arithmetic(int a, int b, int op)
{
    int p = promote_types(a, b);
    if (p < 0) return -1;
    if (op == PT_OP_MAXIMUM || op == PT_OP_MINIMUM) return p;
    if (op == PT_OP_DIV || op == PT_OP_POW)
        return (p == PT_FLOAT64 || p == PT_INT64 || p == PT_UINT64) ? PT_FLOAT64 : PT_FLOAT32;
    if (a == PT_BOOL && b == PT_BOOL) return PT_INT32;
    return p;
}

// can_safely_cast_to (data_types.c:565-629)
bool can_safely_cast_to(int from, int to)
{
    if (!is_valid_dtype(from) || !is_valid_dtype(to)) return false;
    if (from == to) return true;
    if (from == PT_FLOAT16 || from == PT_BFLOAT16) return to == PT_FLOAT32 || to == PT_FLOAT64;
    if (to == PT_FLOAT16 || to == PT_BFLOAT16) return false;
    if (from == PT_BOOL) return true;
    if (is_floating(from) && is_integer(to)) return false;
    if (is_integer(from) && is_floating(to)) {
        if (to == PT_FLOAT64) return true;
        return dtype_size(from) <= 4;  // float32 accepts 8-, 16- and 32-bit integers
    }
    if (is_integer(from) && is_integer(to)) {
        size_t fb = dtype_size(from) * 8, tb = dtype_size(to) * 8;
        bool fs = is_signed(from), ts = is_signed(to);
        if (fs == ts) return tb >= fb;
        if (!fs && ts) return tb > fb;
        return false;
    }
    if (is_floating(from) && is_floating(to)) return dtype_size(to) >= dtype_size(from);
    return false;
}

// ------------------------------------------------------------------ shapes
void contiguous_strides(const int *shape, int ndims, size_t *strides)
{
    size_t s = 1;
    for (int d = ndims - 1; d >= 0; d--) {
        strides[d] = s;
        s *= (size_t)shape[d];
    }
}

bool shape_metrics(const int *shape, int ndims, size_t *elements)
{
    if (ndims < 0 || ndims > kMaxDims) return false;
    size_t total = 1;
    for (int d = ndims - 1; d >= 0; d--) {
        if (shape[d] < 0) return false;
        if (shape[d] && total > (size_t)PTRDIFF_MAX / (size_t)shape[d]) return false;
        total *= (size_t)shape[d];
    }
    *elements = total;
    return true;
}

// tensor_broadcast_shape (src/tensor_shape.h:7-21)
bool broadcast_shape(const int *a, int na, const int *b, int nb, int *out, int *nout)
{
    int n = na > nb ? na : nb;
    int oa = n - na, ob = n - nb;
    for (int d = 0; d < n; d++) {
        int ea = d < oa ? 1 : a[d - oa];
        int eb = d < ob ? 1 : b[d - ob];
        if (ea != eb && ea != 1 && eb != 1) return false;
        out[d] = ea == 1 ? eb : ea;
    }
    *nout = n;
    return true;
}

// tensor_matmul_shape (src/tensor_shape.h:46-59)
bool matmul_shape(const int *a, int na, const int *b, int nb, int *out, int *nout)
{
    if (na < 2 || na > kMaxDims || nb < 2 || nb > kMaxDims || a[na - 1] != b[nb - 2]) return false;
    int bd;
    if (!broadcast_shape(a, na - 2, b, nb - 2, out, &bd)) return false;
    out[bd] = a[na - 2];
    out[bd + 1] = b[nb - 1];
    *nout = bd + 2;
    return true;
}

// ----------------------------------------------------------------- tensors
Storage::~Storage()
{
    if (ptr) pt_free(ptr, nullptr);
}

static std::atomic<uint64_t> g_ids{1};
uint64_t next_tensor_id() { return g_ids.fetch_add(1); }

size_t Tensor::numel() const
{
    size_t n = 1;
    for (int d = 0; d < ndims; d++) n *= (size_t)shape[d];
    return n;
}

bool Tensor::contiguous() const
{
    size_t expect = 1;
    for (int d = ndims - 1; d >= 0; d--) {
        if (shape[d] != 1 && strides[d] != expect) return false;
        expect *= (size_t)shape[d];
    }
    return true;
}

void *Tensor::data() const
{
    if (!storage) return nullptr;
    return (char *)storage->ptr + offset * dtype_size(dtype);
}

TensorP make_meta(const int *shape, int ndims, int dtype)
{
    size_t n;
    if (!is_valid_dtype(dtype)) {
        set_invalid("Unknown dtype");
        return nullptr;
    }
    if (!shape_metrics(shape, ndims, &n)) {
        set_invalid("Tensor shape exceeds supported limits");
        return nullptr;
    }
    auto t = std::make_shared<Tensor>();
    t->dtype = dtype;
    t->ndims = ndims;
    for (int d = 0; d < ndims; d++) t->shape[d] = shape[d];
    contiguous_strides(shape, ndims, t->strides);
    t->id = next_tensor_id();
    return t;
}

static thread_local bool t_alloc_forbidden = false;
static thread_local uint64_t t_alloc_refusals = 0;
static thread_local TensorP t_preset;

bool &allocation_forbidden() { return t_alloc_forbidden; }
uint64_t allocation_refusals() { return t_alloc_refusals; }

void preset_output(const TensorP &t) { t_preset = t; }

TensorP output_tensor(const int *shape, int ndims, int dtype)
{
    TensorP p = std::move(t_preset);
    t_preset.reset();
    if (p && p->storage && p->dtype == dtype && p->ndims == ndims && std::equal(shape, shape + ndims, p->shape) &&
        p->contiguous() && p->storage->bytes >= p->numel() * dtype_size(dtype))
        return p;
    return make_empty(shape, ndims, dtype);
}

TensorP make_empty(const int *shape, int ndims, int dtype)
{
    if (t_alloc_forbidden) {
        t_alloc_refusals++;
        set_runtime("Device allocation inside a captured plan");
        return nullptr;
    }
    TensorP t = make_meta(shape, ndims, dtype);
    if (!t) return nullptr;
    auto st = std::make_shared<Storage>();
    size_t bytes = t->numel() * dtype_size(dtype);
    st->bytes = bytes;
    if (!check_status(pt_alloc(&st->ptr, bytes ? bytes : 1, nullptr), "device allocation")) return nullptr;
    t->storage = st;
    return t;
}

TensorP from_host(const void *data, const int *shape, int ndims, int dtype)
{
    TensorP t = make_empty(shape, ndims, dtype);
    if (!t) return nullptr;
    size_t bytes = t->numel() * dtype_size(dtype);
    if (bytes && !check_status(pt_memcpy_h2d(t->storage->ptr, data, bytes, nullptr), "host to device copy"))
        return nullptr;
    return t;
}

TensorP materialize(const TensorP &t)
{
    if (t->contiguous() && t->offset == 0 && !t->lazy()) return t;
    TensorP out = make_empty(t->shape, t->ndims, t->dtype);
    if (!out) return nullptr;
    if (t->numel() &&
        !check_status(pt_cast(t->storage->ptr, t->dtype, t->strides, t->offset, out->storage->ptr,
                              t->dtype, t->shape, t->ndims, nullptr), "pack"))
        return nullptr;
    return out;
}

bool to_host(const TensorP &t, void *out, size_t bytes)
{
    size_t need = t->numel() * dtype_size(t->dtype);
    if (bytes < need) {
        set_invalid("Destination buffer too small");
        return false;
    }
    if (!need) return true;
    TensorP c = (t->contiguous()) ? t : materialize(t);
    if (!c) return false;
    return check_status(pt_memcpy_d2h(out, c->data(), need, nullptr), "device to host copy");
}

TensorP full(const int *shape, int ndims, int dtype, const Scalar &value)
{
    TensorP t = make_empty(shape, ndims, dtype);
    if (!t) return nullptr;
    pt_scalar_t s = to_pt_scalar(value);
    if (!check_status(pt_fill(t->storage->ptr, dtype, t->numel(), &s, nullptr), "fill")) return nullptr;
    return t;
}

// ------------------------------------------------------------------- views
TensorP view(const TensorP &t, const int *shape, const size_t *strides, int ndims, size_t offset)
{
    auto v = std::make_shared<Tensor>();
    v->storage = t->storage;
    v->dtype = t->dtype;
    v->ndims = ndims;
    for (int d = 0; d < ndims; d++) {
        v->shape[d] = shape[d];
        v->strides[d] = strides[d];
    }
    v->offset = offset;
    v->read_only = t->read_only;
    v->is_view = true;
    v->id = next_tensor_id();
    return v;
}

TensorP reshape(const TensorP &t, const int *shape, int ndims)
{
    int sh[kMaxDims];
    int infer = -1;
    size_t known = 1;
    if (ndims < 0 || ndims > kMaxDims) {
        set_invalid("Reshape rank must be between 0 and 10");
        return nullptr;
    }
    for (int d = 0; d < ndims; d++) {
        sh[d] = shape[d];
        if (shape[d] == -1) {
            if (infer >= 0) {
                set_invalid("Only one reshape dimension can be inferred");
                return nullptr;
            }
            infer = d;
        } else if (shape[d] < 0) {
            set_invalid("Invalid reshape dimension");
            return nullptr;
        } else {
            known *= (size_t)shape[d];
        }
    }
    size_t total = t->numel();
    if (infer >= 0) {
        if (!known || total % known) {
            set_invalid("Cannot infer reshape dimension");
            return nullptr;
        }
        sh[infer] = (int)(total / known);
        known *= (size_t)sh[infer];
    }
    if (known != total) {
        set_invalid("Reshape must preserve the number of elements");
        return nullptr;
    }
    TensorP src = t;
    if (!t->contiguous()) {
        src = materialize(t);
        if (!src) return nullptr;
    }
    size_t st[kMaxDims];
    contiguous_strides(sh, ndims, st);
    return view(src, sh, st, ndims, src->offset);
}

TensorP transpose(const TensorP &t, const int *perm, int nperm)
{
    int p[kMaxDims];
    if (nperm == 0) {
        for (int d = 0; d < t->ndims; d++) p[d] = t->ndims - 1 - d;
    } else {
        if (nperm != t->ndims) {
            set_invalid("Transpose axes must match the tensor rank");
            return nullptr;
        }
        int seen[kMaxDims] = {0};
        for (int d = 0; d < nperm; d++) {
            int a = perm[d] < 0 ? perm[d] + t->ndims : perm[d];
            if (a < 0 || a >= t->ndims || seen[a]) {
                set_invalid("Transpose axes must be a permutation of the tensor axes");
                return nullptr;
            }
            seen[a] = 1;
            p[d] = a;
        }
    }
    int sh[kMaxDims];
    size_t st[kMaxDims];
    for (int d = 0; d < t->ndims; d++) {
        sh[d] = t->shape[p[d]];
        st[d] = t->strides[p[d]];
    }
    return view(t, sh, st, t->ndims, t->offset);
}

TensorP broadcast_to(const TensorP &t, const int *shape, int ndims)
{
    if (ndims < t->ndims || ndims > kMaxDims) {
        set_invalid("broadcastTo target rank must be at least the input rank");
        return nullptr;
    }
    size_t st[kMaxDims] = {0};
    int off = ndims - t->ndims;
    for (int d = off; d < ndims; d++) {
        int e = t->shape[d - off];
        if (e != shape[d] && e != 1) {
            set_invalid("Cannot broadcast dimension %d from %d to %d", d - off, e, shape[d]);
            return nullptr;
        }
        st[d] = (e == 1 && shape[d] != 1) ? 0 : t->strides[d - off];
    }
    TensorP v = view(t, shape, st, ndims, t->offset);
    v->read_only = true;
    return v;
}

TensorP slice_axis(const TensorP &t, int axis, int start, int stop, int step)
{
    if (axis < 0 || axis >= t->ndims || step <= 0) {
        set_invalid("Invalid slice");
        return nullptr;
    }
    int n = t->shape[axis];
    if (start < 0) start += n;
    if (stop < 0) stop += n;
    start = start < 0 ? 0 : (start > n ? n : start);
    stop = stop < start ? start : (stop > n ? n : stop);
    int sh[kMaxDims];
    size_t st[kMaxDims];
    for (int d = 0; d < t->ndims; d++) {
        sh[d] = t->shape[d];
        st[d] = t->strides[d];
    }
    sh[axis] = (stop - start + step - 1) / step;
    st[axis] = t->strides[axis] * (size_t)step;
    return view(t, sh, st, t->ndims, t->offset + (size_t)start * t->strides[axis]);
}

TensorP select_index(const TensorP &t, int axis, int index)
{
    if (axis < 0 || axis >= t->ndims) {
        set_invalid("Invalid index axis");
        return nullptr;
    }
    int n = t->shape[axis];
    if (index < 0) index += n;
    if (index < 0 || index >= n) {
        set_invalid("Index %d out of range for dimension of size %d", index, n);
        return nullptr;
    }
    int sh[kMaxDims];
    size_t st[kMaxDims];
    int k = 0;
    for (int d = 0; d < t->ndims; d++) {
        if (d == axis) continue;
        sh[k] = t->shape[d];
        st[k] = t->strides[d];
        k++;
    }
    return view(t, sh, st, k, t->offset + (size_t)index * t->strides[axis]);
}

}  // namespace phpt
