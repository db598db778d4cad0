// Internal header shared by the gfx950 kernels and the C-ABI glue.
// Not part of the public boundary (include/pt_hip.h is).
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/pt_hip.h"

#define PT_MAX_DIMS 10
#define PT_WAVE 64

namespace pt {

// ------------------------------------------------------------ status glue
void set_error(const char *fmt, ...);
pt_status fail(pt_status status, const char *fmt, ...);
pt_status check_hip(hipError_t err, const char *what);
hipStream_t stream_of(pt_stream_t s);
pt_status ensure_init();
pt_status scratch_alloc(void **ptr, size_t bytes, hipStream_t stream);
void scratch_free(void *ptr, hipStream_t stream);
// static scratch of the no-allocation entry points (1 MiB per device);
// begin orders the call's stream after the previous call's work on the
// device, end records the call's own (both on `stream`)
#define PT_STATIC_SCRATCH_BYTES (1u << 20)
pt_status static_scratch_begin(hipStream_t stream);
pt_status static_scratch_end(hipStream_t stream);
pt_backend_info &counters();

#define PT_TRY(expr)                      \
    do {                                  \
        pt_status _s = (expr);            \
        if (_s != PT_OK) return _s;       \
    } while (0)

#define PT_LAUNCH_CHECK(what) PT_TRY(::pt::check_hip(hipGetLastError(), what))

__host__ __device__ inline size_t dtype_size(int dtype)
{
    switch (dtype) {
    case PT_FLOAT32: case PT_INT32: case PT_UINT32: return 4;
    case PT_FLOAT64: case PT_INT64: case PT_UINT64: return 8;
    case PT_INT16: case PT_UINT16: case PT_FLOAT16: case PT_BFLOAT16: return 2;
    case PT_INT8: case PT_UINT8: case PT_BOOL: return 1;
    default: return 0;
    }
}

inline bool dtype_is_floating(int d)
{
    return d == PT_FLOAT32 || d == PT_FLOAT64 || d == PT_FLOAT16 || d == PT_BFLOAT16;
}
inline bool dtype_is_integer(int d) { return d >= PT_INT8 && d <= PT_UINT64; }
inline bool dtype_valid(int d) { return dtype_size(d) != 0; }

// Shape helpers (host side).
struct Layout {
    int ndims = 0;
    int shape[PT_MAX_DIMS] = {0};
    size_t strides[PT_MAX_DIMS] = {0};
};

inline size_t numel(const int *shape, int ndims)
{
    size_t n = 1;
    for (int d = 0; d < ndims; d++) n *= (size_t)shape[d];
    return n;
}

inline bool is_row_major(const int *shape, const size_t *strides, int ndims)
{
    size_t expect = 1;
    for (int d = ndims - 1; d >= 0; d--) {
        if (shape[d] != 1 && strides[d] != expect) return false;
        expect *= (size_t)shape[d];
    }
    return true;
}

// ---------------------------------------------------- device conversions
// bfloat16 and float16 travel as raw uint16_t bit patterns.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_float(uint16_t b)
{
    return __uint_as_float((uint32_t)b << 16);
}

// Round to nearest even with NaN quieting, bit-identical to the reference's
// float_to_bfloat16_bits (src/data_types.c:113-123).
__device__ __forceinline__ uint16_t float_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu))
        return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float f16_to_float(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}

// Hardware RNE for finite/inf values; NaN payload as the reference's
// float_to_float16_bits (src/data_types.c:46-59): top mantissa bits, forced
// non-zero.
__device__ __forceinline__ uint16_t float_to_f16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) {
        uint32_t payload = (u & 0x7fffffu) >> 13;
        if (!payload) payload = 1;
        return (uint16_t)(((u >> 16) & 0x8000u) | 0x7c00u | payload);
    }
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT> struct DType;
template <> struct DType<PT_FLOAT32> {
    using S = float; using C = float;
    __device__ static C to_c(S s) { return s; }
    __device__ static S from_c(C c) { return c; }
};
template <> struct DType<PT_FLOAT64> {
    using S = double; using C = double;
    __device__ static C to_c(S s) { return s; }
    __device__ static S from_c(C c) { return c; }
};
template <> struct DType<PT_BFLOAT16> {
    using S = uint16_t; using C = float;
    __device__ static C to_c(S s) { return bf16_to_float(s); }
    __device__ static S from_c(C c) { return float_to_bf16(c); }
};
template <> struct DType<PT_FLOAT16> {
    using S = uint16_t; using C = float;
    __device__ static C to_c(S s) { return f16_to_float(s); }
    __device__ static S from_c(C c) { return float_to_f16(c); }
};
template <> struct DType<PT_INT8> { using S = int8_t; using C = int8_t; };
template <> struct DType<PT_INT16> { using S = int16_t; using C = int16_t; };
template <> struct DType<PT_INT32> { using S = int32_t; using C = int32_t; };
template <> struct DType<PT_INT64> { using S = int64_t; using C = int64_t; };
template <> struct DType<PT_UINT8> { using S = uint8_t; using C = uint8_t; };
template <> struct DType<PT_UINT16> { using S = uint16_t; using C = uint16_t; };
template <> struct DType<PT_UINT32> { using S = uint32_t; using C = uint32_t; };
template <> struct DType<PT_UINT64> { using S = uint64_t; using C = uint64_t; };
template <> struct DType<PT_BOOL> { using S = uint8_t; using C = uint8_t; };

// Load element i of dtype `dt` from raw memory as double (generic paths).
__device__ __forceinline__ double load_as_double(const void *p, int dt, size_t i)
{
    switch (dt) {
    case PT_FLOAT32: return ((const float *)p)[i];
    case PT_FLOAT64: return ((const double *)p)[i];
    case PT_FLOAT16: return f16_to_float(((const uint16_t *)p)[i]);
    case PT_BFLOAT16: return bf16_to_float(((const uint16_t *)p)[i]);
    case PT_INT8: return ((const int8_t *)p)[i];
    case PT_INT16: return ((const int16_t *)p)[i];
    case PT_INT32: return ((const int32_t *)p)[i];
    case PT_INT64: return (double)((const int64_t *)p)[i];
    case PT_UINT8: return ((const uint8_t *)p)[i];
    case PT_UINT16: return ((const uint16_t *)p)[i];
    case PT_UINT32: return ((const uint32_t *)p)[i];
    case PT_UINT64: return (double)((const uint64_t *)p)[i];
    case PT_BOOL: return ((const uint8_t *)p)[i] != 0;
    default: return 0.0;
    }
}

// ---------------------------------------------------- wave64 reductions
template <typename T, typename F>
__device__ __forceinline__ T wave_reduce(T v, F f)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = f(v, __shfl_xor(v, m, PT_WAVE));
    return v;
}

// Every lane gets the wave's reduction of a 4-byte value, without LDS:
// two DPP quad permutes (lane ^ 1, lane ^ 2) and the half-row and row
// mirrors (lane i with 7 - i and 15 - i) combine each 16-lane row, fused
// into the ALU ops as DPP source modifiers; the four row totals then come
// out through v_readlane and are combined in one fixed order, so the result
// is the same wave-uniform value in every lane.  f must be commutative and
// associative up to the rounding a reduction order may change (add, max,
// min).
template <typename T, typename F>
__device__ __forceinline__ T wave_all(T v, F f)
{
    static_assert(sizeof(T) == 4, "4-byte lanes");
    auto dpp = [](T x, auto CTRL) {
        return __builtin_bit_cast(
            T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(CTRL)::value, 0xF, 0xF, false));
    };
    v = f(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1, 0, 3, 2]
    v = f(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2, 3, 0, 1]
    v = f(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
    v = f(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
    const int iv = __builtin_bit_cast(int, v);
    const T a = __builtin_bit_cast(T, __builtin_amdgcn_readlane(iv, 0));
    const T b = __builtin_bit_cast(T, __builtin_amdgcn_readlane(iv, 16));
    const T c = __builtin_bit_cast(T, __builtin_amdgcn_readlane(iv, 32));
    const T d = __builtin_bit_cast(T, __builtin_amdgcn_readlane(iv, 48));
    return f(f(a, b), f(c, d));
}

struct FAdd { template <typename T> __device__ T operator()(T a, T b) const { return a + b; } };
struct FMax { __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
              __device__ double operator()(double a, double b) const { return fmax(a, b); } };
struct FMin { __device__ float operator()(float a, float b) const { return fminf(a, b); }
              __device__ double operator()(double a, double b) const { return fmin(a, b); } };

}  // namespace pt
