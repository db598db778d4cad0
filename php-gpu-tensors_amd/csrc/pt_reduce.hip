// Axis reductions (sum/mean/max/min/prod, argmax/argmin, var/std) and the
// fused row softmax / layerNorm kernels for gfx950.
//
// Layout classes (chosen on the host from shape/strides/axis):
//   rows    : the reduced axis has stride 1 and the other axes collapse to a
//             single row index with pitch `ld` -> one wave64 per row,
//             16-byte vector loads (global_load_dwordx4), DPP/shuffle
//             wave reduction, no LDS.  This is the HBM-roofline path.
//   columns : contiguous input reduced over a non-last axis -> (outer, n,
//             inner), lanes walk `inner` (coalesced), LDS combine over n.
//   strided : anything else -> one workgroup per output with full stride
//             decode (correct for every view, not a fast path).
//   global  : all elements of a contiguous input -> per-workgroup partials
//             in stream-ordered scratch, then one finishing workgroup.
//
// Semantics follow the reference: reduction_ops.cu:148-311 for op/dtype
// rules, reduction_ops.cuh:319-401 for arg reductions, :86-112 (Welford)
// for var/std, cuda_array_ce.c:1942-2001 (softmax) and :2215-2339
// (layerNorm).  max/min skip NaN like HostArray (contiguous_array_ce.c:
// 1241-1242).
#include "pt_common.h"

#include <math.h>

namespace pt {

enum RedOp { R_SUM = 0, R_MEAN, R_MAX, R_MIN, R_PROD, R_ARGMAX, R_ARGMIN, R_VAR, R_ALL, R_ANY };

// ------------------------------------------------------------------ traits
// Storage type S, compute type C, 16-byte vector width V.
template <int DT> struct RT;
template <> struct RT<PT_FLOAT32> {
    using S = float; using C = float; static constexpr int V = 4;
    __device__ static C cv(S s) { return s; }
};
template <> struct RT<PT_FLOAT64> {
    using S = double; using C = double; static constexpr int V = 2;
    __device__ static C cv(S s) { return s; }
};
template <> struct RT<PT_BFLOAT16> {
    using S = uint16_t; using C = float; static constexpr int V = 8;
    __device__ static C cv(S s) { return bf16_to_float(s); }
};
template <> struct RT<PT_FLOAT16> {
    using S = uint16_t; using C = float; static constexpr int V = 8;
    __device__ static C cv(S s) { return f16_to_float(s); }
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte chunk of a row.  Rows are read exactly once, so the loads are
// nontemporal: on gfx950 that keeps the HBM stream at a higher rate than
// cached loads (no L2 / Infinity Cache retention of dead lines).
template <int DT, int V, bool NT = true>
__device__ __forceinline__ void load_chunk(const typename RT<DT>::S *p, typename RT<DT>::C (&v)[V])
{
    using S = typename RT<DT>::S;
    if constexpr (V * sizeof(S) == 16) {
        union { u32x4 raw; S s[V]; } u;
        if constexpr (NT) u.raw = __builtin_nontemporal_load((const u32x4 *)p);
        else u.raw = *(const u32x4 *)p;
#pragma unroll
        for (int i = 0; i < V; i++) v[i] = RT<DT>::cv(u.s[i]);
    } else {
#pragma unroll
        for (int i = 0; i < V; i++) v[i] = RT<DT>::cv(p[i]);
    }
}

// 16-byte store of a register chunk; NT: nontemporal (streaming output
// that is not read back by this kernel).
template <bool NT = false>
__device__ __forceinline__ void store16(void *dst, const void *src)
{
    u32x4 v;
    memcpy(&v, src, 16);
    if constexpr (NT) __builtin_nontemporal_store(v, (u32x4 *)dst);
    else *(u32x4 *)dst = v;
}

// Row-wide sum / max over the WPR waves of one row (LDS when WPR > 1).
// Every wave of the row returns the same value.
template <typename C, int WPR>
__device__ __forceinline__ C row_sum(C v, C *lds)
{
    if constexpr (sizeof(C) == 4) {
        v = wave_all(v, FAdd{});
    } else {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, PT_WAVE);
    }
    if constexpr (WPR > 1) {
        const int wave = threadIdx.x >> 6, w0 = wave - wave % WPR;
        __syncthreads();
        if ((threadIdx.x & 63) == 0) lds[wave] = v;
        __syncthreads();
        v = lds[w0];
        for (int w = 1; w < WPR; w++) v = v + lds[w0 + w];
    }
    return v;
}

template <typename C> __device__ __forceinline__ C fmax_any(C a, C b);

template <typename C, int WPR>
__device__ __forceinline__ C row_max(C v, C *lds)
{
    if constexpr (sizeof(C) == 4) {
        v = wave_all(v, [](C a, C b) { return fmax_any(a, b); });
    } else {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v = fmax_any(v, __shfl_xor(v, m, PT_WAVE));
    }
    if constexpr (WPR > 1) {
        const int wave = threadIdx.x >> 6, w0 = wave - wave % WPR;
        __syncthreads();
        if ((threadIdx.x & 63) == 0) lds[wave] = v;
        __syncthreads();
        v = lds[w0];
        for (int w = 1; w < WPR; w++) v = fmax_any(v, lds[w0 + w]);
    }
    return v;
}

template <typename C> __device__ __forceinline__ C neg_inf();
template <> __device__ __forceinline__ float neg_inf<float>() { return -INFINITY; }
template <> __device__ __forceinline__ double neg_inf<double>() { return -INFINITY; }

__device__ __forceinline__ float fmax_c(float a, float b) { return fmaxf(a, b); }
template <> __device__ __forceinline__ float fmax_any<float>(float a, float b) { return fmaxf(a, b); }
template <> __device__ __forceinline__ double fmax_any<double>(double a, double b) { return fmax(a, b); }
__device__ __forceinline__ double fmax_c(double a, double b) { return fmax(a, b); }
__device__ __forceinline__ float fmin_c(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ double fmin_c(double a, double b) { return fmin(a, b); }
__device__ __forceinline__ float exp_c(float a) { return expf(a); }
__device__ __forceinline__ double exp_c(double a) { return exp(a); }

// a / b for many a and one b.  fp32: with rb = RN(1 / b) (one true division
// per row), q0 = RN(a rb) is within one ulp of a / b and the fma remainder
// a - b q0 is exact, so RN(q0 + (a - b q0) rb) is the correctly rounded
// quotient (Markstein's theorem): three instructions instead of the ~10 of
// an IEEE division.  The theorem needs a normal quotient, so a quotient at
// or below FLT_MIN (a softmax value more than about 87 below its row's
// maximum) takes the IEEE division; the branch is uniform and skipped
// unless a lane needs it.  Callers take the true division when rb is 0 or
// not finite.
struct RowDiv {
    float b, rb;
    bool fast;
    __device__ __forceinline__ explicit RowDiv(float den) : b(den), rb(1.0f / den)
    {
        fast = __builtin_isfinite(rb) && rb != 0.0f;
    }
    __device__ __forceinline__ float operator()(float a) const
    {
        const float q0 = a * rb;
        if (__builtin_expect(__builtin_fabsf(q0) <= 1.17549435e-38f, 0)) return a / b;
        return __builtin_fmaf(__builtin_fmaf(-q0, b, a), rb, q0);
    }
};
__device__ __forceinline__ float sqrt_c(float a) { return sqrtf(a); }
__device__ __forceinline__ double sqrt_c(double a) { return sqrt(a); }

// Moments state for var/std (Chan et al. parallel combination of Welford
// states, reduction_ops.cuh:97-112).
struct Mom {
    double n, mean, m2;
};

__device__ __forceinline__ Mom mom_combine(Mom a, Mom b)
{
    if (a.n == 0) return b;
    if (b.n == 0) return a;
    double n = a.n + b.n;
    double delta = b.mean - a.mean;
    Mom r;
    r.n = n;
    r.mean = a.mean + delta * (b.n / n);
    r.m2 = a.m2 + b.m2 + delta * delta * (a.n * b.n / n);
    return r;
}

__device__ __forceinline__ Mom mom_shfl(Mom m, int lane_mask)
{
    Mom o;
    o.n = __shfl_xor(m.n, lane_mask, PT_WAVE);
    o.mean = __shfl_xor(m.mean, lane_mask, PT_WAVE);
    o.m2 = __shfl_xor(m.m2, lane_mask, PT_WAVE);
    return o;
}

// Per-lane accumulator for one reduction op over compute type C.
template <typename C, int OP> struct Acc;

template <typename C> struct Acc<C, R_SUM> {
    C s = 0;
    __device__ void add(C v, int) { s = s + v; }
    __device__ void merge_shfl(int m) { s = s + __shfl_xor(s, m, PT_WAVE); }
    __device__ void merge(const Acc &o) { s = s + o.s; }
};
template <typename C> struct Acc<C, R_MEAN> : Acc<C, R_SUM> {};
template <typename C> struct Acc<C, R_PROD> {
    C s = 1;
    __device__ void add(C v, int) { s = s * v; }
    __device__ void merge_shfl(int m) { s = s * __shfl_xor(s, m, PT_WAVE); }
    __device__ void merge(const Acc &o) { s = s * o.s; }
};
template <typename C> struct Acc<C, R_MAX> {
    C s = neg_inf<C>();
    __device__ void add(C v, int) { s = fmax_c(s, v); }
    __device__ void merge_shfl(int m) { s = fmax_c(s, __shfl_xor(s, m, PT_WAVE)); }
    __device__ void merge(const Acc &o) { s = fmax_c(s, o.s); }
};
template <typename C> struct Acc<C, R_MIN> {
    C s = -neg_inf<C>();
    __device__ void add(C v, int) { s = fmin_c(s, v); }
    __device__ void merge_shfl(int m) { s = fmin_c(s, __shfl_xor(s, m, PT_WAVE)); }
    __device__ void merge(const Acc &o) { s = fmin_c(s, o.s); }
};
// Arg reductions: elements arrive in increasing index order per lane, so a
// strict comparison keeps the lowest index; merges break ties by index.
// NaN compares false and is never taken; identity is (+-inf, 0).
template <typename C, bool MAXIMIZE> struct ArgAcc {
    C v = MAXIMIZE ? neg_inf<C>() : -neg_inf<C>();
    int i = 0;
    __device__ void add(C x, int idx)
    {
        if (MAXIMIZE ? x > v : x < v) { v = x; i = idx; }
    }
    __device__ void merge(const ArgAcc &o)
    {
        if ((MAXIMIZE ? o.v > v : o.v < v) || (o.v == v && o.i < i)) { v = o.v; i = o.i; }
    }
    __device__ void merge_shfl(int m)
    {
        ArgAcc o;
        o.v = __shfl_xor(v, m, PT_WAVE);
        o.i = __shfl_xor(i, m, PT_WAVE);
        merge(o);
    }
};
template <typename C> struct Acc<C, R_ARGMAX> : ArgAcc<C, true> {};
template <typename C> struct Acc<C, R_ARGMIN> : ArgAcc<C, false> {};
template <typename C> struct Acc<C, R_VAR> {
    Mom m = {0, 0, 0};
    C cn = 0, cmean = 0, cm2 = 0;  // running per-lane state in compute type
    __device__ void add(C v, int)
    {
        // single-element Welford step; welford_single seeds m2 with v - v so
        // that infinities poison the result (reduction_ops.cuh:86-90)
        C n1 = cn + 1;
        C delta = v - cmean;
        cmean = cmean + delta / n1;
        cm2 = cm2 + (v - v) + delta * (v - cmean);
        cn = n1;
    }
    __device__ Mom lane_state() const { return Mom{(double)cn, (double)cmean, (double)cm2}; }
};

template <typename C, int OP>
__device__ __forceinline__ void wave_merge(Acc<C, OP> &a)
{
    if constexpr (sizeof(C) == 4 && (OP == R_ARGMAX || OP == R_ARGMIN)) {
        // (value, index) pairs over the same DPP pattern as wave_all: the
        // merge keeps the better value and, on ties, the lower index, so it
        // gives the same pair whichever side a lane holds
        auto step = [&](auto CTRL) {
            Acc<C, OP> o;
            o.v = __builtin_bit_cast(C, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a.v),
                                                                     decltype(CTRL)::value, 0xF, 0xF, false));
            o.i = __builtin_amdgcn_update_dpp(0, a.i, decltype(CTRL)::value, 0xF, 0xF, false);
            a.merge(o);
        };
        step(std::integral_constant<int, 0xB1>{});
        step(std::integral_constant<int, 0x4E>{});
        step(std::integral_constant<int, 0x141>{});
        step(std::integral_constant<int, 0x140>{});
        Acc<C, OP> r[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            r[q].v = __builtin_bit_cast(C, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a.v), 16 * q));
            r[q].i = __builtin_amdgcn_readlane(a.i, 16 * q);
        }
        r[0].merge(r[1]);
        r[2].merge(r[3]);
        r[0].merge(r[2]);
        a = r[0];
    } else if constexpr (sizeof(C) == 4 && (OP == R_SUM || OP == R_MEAN || OP == R_PROD || OP == R_MAX || OP == R_MIN)) {
        a.s = wave_all(a.s, [](C x, C y) {
            if constexpr (OP == R_MAX) return fmax_c(x, y);
            else if constexpr (OP == R_MIN) return fmin_c(x, y);
            else if constexpr (OP == R_PROD) return x * y;
            else return x + y;
        });
    } else {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) a.merge_shfl(m);
    }
}

// Chunk-level variance update: V elements at once (exact two-pass on the
// registers of the chunk, then a Chan combine), one division per chunk.
template <typename C, int V>
__device__ __forceinline__ void var_add_chunk(Acc<C, R_VAR> &a, const C (&v)[V], int valid)
{
    if (valid == V) {
        C s = 0;
#pragma unroll
        for (int k = 0; k < V; k++) s = s + v[k];
        C mb = s / (C)V;
        C m2b = 0;
#pragma unroll
        for (int k = 0; k < V; k++) {
            C d = v[k] - mb;
            m2b = m2b + d * d;
        }
        if (a.cn == 0) {
            a.cn = (C)V; a.cmean = mb; a.cm2 = m2b;
        } else {
            C n = a.cn + (C)V;
            C delta = mb - a.cmean;
            C r = (C)V / n;
            a.cmean = a.cmean + delta * r;
            a.cm2 = a.cm2 + m2b + delta * delta * a.cn * r;
            a.cn = n;
        }
    } else {
        for (int k = 0; k < valid; k++) a.add(v[k], 0);
    }
}

// ------------------------------------------------------ output conversion
template <typename C>
__device__ __forceinline__ void store_out(void *out, int out_dt, size_t i, C v)
{
    if (out_dt == PT_FLOAT32) ((float *)out)[i] = (float)v;
    else ((double *)out)[i] = (double)v;
}

// ============================================================ row kernels
// WPR wave64s per row (1 or 4) and 256 / (64 * WPR) rows per 256-thread
// block.  Each wave keeps 4 chunks of VEC elements in flight per lane;
// with WPR = 4 the row's chunks interleave across the block's waves, so one
// block streams a long row with 16 KiB in flight, and the four partial
// states meet in LDS (ordered merge: argmax ties still go to the lowest
// index).  With WPR = 1 there is no LDS and no barrier.
template <typename T> struct LdsSlot {
    __align__(16) unsigned char raw[sizeof(T)];
};

// Block shape of a row kernel with WPR waves per row: WPR = 1 packs four
// rows into a 256-thread block; WPR >= 4 gives each row a block of WPR
// waves (64 * WPR threads).
template <int WPR> struct RowShape {
    static_assert(WPR == 1 || WPR == 4 || WPR == 8, "waves per row");
    static constexpr int BW = WPR > 4 ? WPR : 4;  // waves per block
    static constexpr int RPB = BW / WPR;           // rows per block
};

template <int DT, int OP, int VEC, int WPR>
__global__ __launch_bounds__(64 * RowShape<WPR>::BW) void k_row_reduce(const void *__restrict__ xin, size_t rows,
                                                                        int n, size_t ld, void *__restrict__ out,
                                                                        int out_dt, int correction, int take_sqrt)
{
    using S = typename RT<DT>::S;
    using C = typename RT<DT>::C;
    constexpr int RPB = RowShape<WPR>::RPB, BW = RowShape<WPR>::BW;
    // chunks in flight per lane: 4, or fewer when the row's block is wider
    constexpr int U = WPR >= 8 ? 2 : 4;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave % WPR;                        // wave within its row
    const size_t row = (size_t)blockIdx.x * RPB + wave / WPR;
    if (row >= rows) return;                          // uniform per block when WPR > 1
    const S *x = (const S *)xin + row * ld;
    Acc<C, OP> acc;
    constexpr int STEP = 64 * VEC;                    // one wave-wide chunk
    constexpr int RSTEP = WPR * STEP;                 // one row-wide chunk
    int i = wr * STEP + lane * VEC;
    // main loop: U chunks in flight per lane
    for (; i + (U - 1) * RSTEP + VEC <= n; i += U * RSTEP) {
        C v[U][VEC];
#pragma unroll
        for (int u = 0; u < U; u++) load_chunk<DT, VEC>(x + i + u * RSTEP, v[u]);
#pragma unroll
        for (int u = 0; u < U; u++) {
            if constexpr (OP == R_VAR) {
                var_add_chunk<C, VEC>(acc, v[u], VEC);
            } else {
#pragma unroll
                for (int k = 0; k < VEC; k++) acc.add(v[u][k], i + u * RSTEP + k);
            }
        }
    }
    for (; i < n; i += RSTEP) {
        C v[VEC];
        int valid = n - i < VEC ? n - i : VEC;
        if (valid == VEC) {
            load_chunk<DT, VEC>(x + i, v);
        } else {
            for (int k = 0; k < VEC; k++) v[k] = k < valid ? RT<DT>::cv(x[i + k]) : (C)0;
        }
        if constexpr (OP == R_VAR) {
            var_add_chunk<C, VEC>(acc, v, valid);
        } else {
            for (int k = 0; k < valid; k++) acc.add(v[k], i + k);
        }
    }
    if constexpr (OP == R_VAR) {
        Mom m = acc.lane_state();
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) m = mom_combine(m, mom_shfl(m, s));
        if constexpr (WPR > 1) {
            __shared__ LdsSlot<Mom> part[BW];
            if (lane == 0) *reinterpret_cast<Mom *>(part[wave].raw) = m;
            __syncthreads();
            if (wr != 0) return;
            for (int w = 1; w < WPR; w++) m = mom_combine(m, *reinterpret_cast<const Mom *>(part[wave + w].raw));
        }
        if (lane == 0) {
            double var = m.m2 / (double)(n - correction);
            store_out(out, out_dt, row, take_sqrt ? sqrt(var) : var);
        }
    } else {
        wave_merge(acc);
        if constexpr (WPR > 1) {
            __shared__ LdsSlot<Acc<C, OP>> part[BW];
            if (lane == 0) memcpy(part[wave].raw, &acc, sizeof(acc));
            __syncthreads();
            if (wr != 0) return;
            for (int w = 1; w < WPR; w++) {
                Acc<C, OP> o;
                memcpy(&o, part[wave + w].raw, sizeof(o));
                acc.merge(o);
            }
        }
        if (lane == 0) {
            if constexpr (OP == R_ARGMAX || OP == R_ARGMIN) {
                ((int32_t *)out)[row] = acc.i;
            } else if constexpr (OP == R_MEAN) {
                store_out(out, out_dt, row, acc.s / (C)n);
            } else {
                store_out(out, out_dt, row, acc.s);
            }
        }
    }
}

// ------------------------------------------------ register-resident rows
// A row is split over WPR waves (1 or 4); lane `lane` of wave `wr` holds
// NCH chunks of VEC elements, chunk c starting at element
// ((c * WPR + wr) * 64 + lane) * VEC, so the block's loads of one chunk step
// are contiguous.  Lanes whose last chunk lies inside the row (all lanes of
// a row that is a multiple of the chunk layout) take branch-free paths so
// that their NCH loads issue back to back.
template <int VEC, int WPR>
__device__ __forceinline__ int chunk_start(int c, int wr, int lane)
{
    return ((c * WPR + wr) * 64 + lane) * VEC;
}

// `full`: every lane's last chunk lies inside the row, judged from lane 63
// so that it is uniform over the wave and guards whole rows with one scalar
// branch instead of a lane mask per element.
template <int DT, int VEC, int NCH, int WPR, bool NT, typename CT>
__device__ __forceinline__ bool load_row(const typename RT<DT>::S *x, int n, int wr, int lane, CT pad,
                                         CT (&v)[NCH][VEC])
{
    const bool full = chunk_start<VEC, WPR>(NCH - 1, wr, 63) + VEC <= n;  // wave-uniform
    if (full) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            typename RT<DT>::C t[VEC];
            load_chunk<DT, VEC, NT>(x + chunk_start<VEC, WPR>(c, wr, lane), t);
#pragma unroll
            for (int k = 0; k < VEC; k++) v[c][k] = (CT)t[k];
        }
    } else {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int i = chunk_start<VEC, WPR>(c, wr, lane);
            if (i + VEC <= n) {
                typename RT<DT>::C t[VEC];
                load_chunk<DT, VEC, NT>(x + i, t);
#pragma unroll
                for (int k = 0; k < VEC; k++) v[c][k] = (CT)t[k];
            } else {
#pragma unroll
                for (int k = 0; k < VEC; k++) v[c][k] = i + k < n ? (CT)RT<DT>::cv(x[i + k]) : pad;
            }
        }
    }
    return full;
}

template <int VEC, int NCH, int WPR, bool NT = false, typename OS, typename CT>
__device__ __forceinline__ void store_row(OS *y, int n, int wr, int lane, bool full, const CT (&v)[NCH][VEC])
{
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int i = chunk_start<VEC, WPR>(c, wr, lane);
        OS r[VEC];
#pragma unroll
        for (int k = 0; k < VEC; k++) r[k] = (OS)v[c][k];
        if (full || i + VEC <= n) {
            if constexpr (VEC * sizeof(OS) == 16) {
                store16<NT>(y + i, r);
            } else if constexpr (VEC * sizeof(OS) == 32) {
                store16<NT>(y + i, r);
                store16<NT>((char *)(y + i) + 16, (const char *)r + 16);
            } else {
#pragma unroll
                for (int k = 0; k < VEC; k++) y[i + k] = r[k];
            }
        } else {
            for (int k = 0; k < VEC; k++)
                if (i + k < n) y[i + k] = r[k];
        }
    }
}

// Argmax / argmin of fp32 rows held in registers, in two passes over the
// registers: the row's best value as the max (min) reduction computes it
// (fmaxf / fminf: a NaN is never taken), then the lowest index holding
// that value (each lane scans its elements from the highest index down, so
// its last hit is its lowest; lanes and waves keep the minimum).  The result
// is ArgAcc's: ties go to the lowest index, ±0 compare equal, and a row
// whose best is the identity (every element -inf for argmax, +inf for
// argmin, or NaN) gives index 0, since ArgAcc's strict comparison never
// takes such an element.  Per element this is one max and one compare-select
// against ArgAcc's compare and two selects.
template <int VEC, int NCH, int WPR, bool MAXIMIZE>
__global__ __launch_bounds__(64 * RowShape<WPR>::BW) void k_row_arg2(const void *__restrict__ xin, size_t rows,
                                                                      int n, size_t ld, void *__restrict__ out)
{
    static_assert(WPR > 1, "one row per block");
    constexpr int BW = RowShape<WPR>::BW;
    __shared__ float lds_v[BW];
    __shared__ int lds_i[BW];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, wr = wave;
    const size_t row = blockIdx.x;
    if (row >= rows) return;  // whole block
    const float *x = (const float *)xin + row * ld;
    const float ident = MAXIMIZE ? -INFINITY : INFINITY;
    float v[NCH][VEC];
    load_row<PT_FLOAT32, VEC, NCH, WPR, true>(x, n, wr, lane, ident, v);
    auto best = [](float a, float b) { return MAXIMIZE ? fmaxf(a, b) : fminf(a, b); };
    float m = ident;
#pragma unroll
    for (int c = 0; c < NCH; c++)
#pragma unroll
        for (int k = 0; k < VEC; k++) m = best(m, v[c][k]);
    m = wave_all(m, best);
    if (lane == 0) lds_v[wave] = m;
    __syncthreads();
    m = lds_v[0];
#pragma unroll
    for (int w = 1; w < WPR; w++) m = best(m, lds_v[w]);
    // lowest index holding m (elements past n hold the identity: they can
    // match only when m is the identity, whose result is 0 anyway)
    int idx = 0x7fffffff;
#pragma unroll
    for (int c = NCH - 1; c >= 0; c--)
#pragma unroll
        for (int k = VEC - 1; k >= 0; k--)
            if (v[c][k] == m) idx = chunk_start<VEC, WPR>(c, wr, lane) + k;
    idx = wave_all(idx, [](int a, int b) { return a < b ? a : b; });
    if (lane == 0) lds_i[wave] = idx;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < WPR; w++) idx = min(idx, lds_i[w]);
    ((int32_t *)out)[row] = m == ident ? 0 : idx;
}

// Variance / standard deviation: exact two-pass form (mean, then the sum of
// squared deviations from it) over the values held in registers.  Same
// result definition as the Welford kernels (M2 / (n - correction), sqrt for
// std), one HBM pass.
template <int DT, int VEC, int NCH, int WPR>
__global__ __launch_bounds__(64 * RowShape<WPR>::BW) void k_row_moments(const void *__restrict__ xin, size_t rows,
                                                                         int n, size_t ld, void *__restrict__ out,
                                                                         int out_dt, int correction, int take_sqrt)
{
    using S = typename RT<DT>::S;
    using C = typename RT<DT>::C;
    __shared__ C lds[RowShape<WPR>::BW];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, wr = wave % WPR;
    const size_t row = (size_t)blockIdx.x * RowShape<WPR>::RPB + wave / WPR;
    if (row >= rows) return;  // WPR > 1: one row per block, never taken
    const S *x = (const S *)xin + row * ld;
    C v[NCH][VEC];
    const bool full = load_row<DT, VEC, NCH, WPR, true>(x, n, wr, lane, (C)0, v);
    if (n == NCH * VEC * 64 * WPR) {
        // Every lane holds NCH * VEC elements: exact two-pass over the
        // lane's own values, then Chan's pairwise combination of
        // (mean, M2) states of equal counts over the lanes (butterfly: both
        // partners compute the same sums, so every lane ends with the wave's
        // state) and over the waves, in double, by one lane: one exchange
        // through LDS instead of a row mean followed by a row sum.
        constexpr int NL = NCH * VEC;
        C ls = 0;
#pragma unroll
        for (int c = 0; c < NCH; c++)
#pragma unroll
            for (int k = 0; k < VEC; k++) ls = ls + v[c][k];
        C mean = ls / (C)NL, q = 0;
#pragma unroll
        for (int c = 0; c < NCH; c++)
#pragma unroll
            for (int k = 0; k < VEC; k++) {
                const C d = v[c][k] - mean;
                q = q + d * d;
            }
        C cnt = (C)NL;
        // equal-count combination of the partner's state (om, oq)
        auto chan = [&](C om, C oq) {
            const C d = om - mean;
            q = (q + oq) + d * d * (cnt * (C)0.5);
            mean = (mean + om) * (C)0.5;
            cnt = cnt * 2;
        };
        if constexpr (sizeof(C) == 4) {
            // lanes ^ 1, ^ 2 (DPP quad permutes), then the half-row and row
            // mirrors (as in wave_all), then the four row states in order
            auto dpp = [](C x, auto CTRL) {
                return __builtin_bit_cast(C, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                          decltype(CTRL)::value, 0xF, 0xF, false));
            };
            chan(dpp(mean, std::integral_constant<int, 0xB1>{}), dpp(q, std::integral_constant<int, 0xB1>{}));
            chan(dpp(mean, std::integral_constant<int, 0x4E>{}), dpp(q, std::integral_constant<int, 0x4E>{}));
            chan(dpp(mean, std::integral_constant<int, 0x141>{}), dpp(q, std::integral_constant<int, 0x141>{}));
            chan(dpp(mean, std::integral_constant<int, 0x140>{}), dpp(q, std::integral_constant<int, 0x140>{}));
            auto rl = [](C x, int l) {
                return __builtin_bit_cast(C, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
            };
            const C m16 = rl(mean, 16), q16 = rl(q, 16), m32 = rl(mean, 32), q32 = rl(q, 32);
            const C m48 = rl(mean, 48), q48 = rl(q, 48);
            mean = rl(mean, 0);
            q = rl(q, 0);
            const C c16 = cnt;
            chan(m16, q16);  // rows 0 + 1
            const C ma = mean, qa = q;
            mean = m32;
            q = q32;
            cnt = c16;
            chan(m48, q48);  // rows 2 + 3
            chan(ma, qa);    // (rows 2 + 3) + (rows 0 + 1): equal counts, symmetric
        } else {
#pragma unroll
            for (int sh = 32; sh >= 1; sh >>= 1) chan(__shfl_xor(mean, sh, PT_WAVE), __shfl_xor(q, sh, PT_WAVE));
        }
        if constexpr (WPR > 1) {
            __shared__ C part_m[RowShape<WPR>::BW], part_q[RowShape<WPR>::BW];
            if (lane == 0) {
                part_m[wave] = mean;
                part_q[wave] = q;
            }
            __syncthreads();
            if (wr != 0 || lane != 0) return;
            double dm = (double)mean, dq = (double)q, dn = (double)cnt;
            for (int w = 1; w < WPR; w++) {
                const double om = (double)part_m[wave + w], oq = (double)part_q[wave + w], on = (double)cnt;
                const double nn = dn + on, d = om - dm;
                dm = dm + d * (on / nn);
                dq = dq + oq + d * d * (dn * on / nn);
                dn = nn;
            }
            const double var = dq / (double)(n - correction);
            store_out(out, out_dt, row, take_sqrt ? sqrt(var) : var);
        } else if (lane == 0) {
            const double var = (double)q / (double)(n - correction);
            store_out(out, out_dt, row, take_sqrt ? sqrt(var) : var);
        }
        return;
    }
    C s = 0;
#pragma unroll
    for (int c = 0; c < NCH; c++)
#pragma unroll
        for (int k = 0; k < VEC; k++) s = s + v[c][k];
    const C mean = row_sum<C, WPR>(s, lds) / (C)n;
    C q = 0;
    // Infinities poison the result as in Welford without a per-element term:
    // an infinite element makes the row's mean infinite or NaN, and its own
    // deviation inf - inf is then NaN (a NaN element makes the mean NaN).
    if (full) {  // wave-uniform: no per-element guard on whole rows
#pragma unroll
        for (int c = 0; c < NCH; c++)
#pragma unroll
            for (int k = 0; k < VEC; k++) {
                const C d = v[c][k] - mean;
                q = q + d * d;
            }
    } else {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int i = chunk_start<VEC, WPR>(c, wr, lane);
#pragma unroll
            for (int k = 0; k < VEC; k++) {
                const C d = i + k < n ? v[c][k] - mean : (C)0;
                q = q + d * d;
            }
        }
    }
    q = row_sum<C, WPR>(q, lds);
    if (wr == 0 && lane == 0) {
        double var = (double)q / (double)(n - correction);
        store_out(out, out_dt, row, take_sqrt ? sqrt(var) : var);
    }
}

// Fused softmax: y = exp(x - max) / sum(exp(x - max)), true division as the
// composite's OP_DIV (cuda_array_ce.c:1995).  One HBM read, one write.
// LNT / SNT: nontemporal row loads / stores.  RW: the grid walks the rows
// (rows blockIdx.x, + gridDim.x, ...) and issues the next row's loads before
// the current row's reductions, so HBM stays busy across its two passes.
template <int DT, int VEC, int NCH, int WPR, typename OS, bool LNT = false, bool SNT = false, bool RW = false>
__global__ __launch_bounds__(64 * RowShape<WPR>::BW) void k_row_softmax(const void *__restrict__ xin, size_t rows,
                                                                         int n, size_t ld, OS *__restrict__ out)
{
    using S = typename RT<DT>::S;
    using C = typename RT<DT>::C;
    constexpr int RPB = RowShape<WPR>::RPB;
    __shared__ C lds[RowShape<WPR>::BW];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, wr = wave % WPR;
    size_t row = (size_t)blockIdx.x * RPB + wave / WPR;
    const size_t row_step = RW ? (size_t)gridDim.x * RPB : rows;
    if (row >= rows) return;  // WPR > 1: uniform per block
    const bool full = chunk_start<VEC, WPR>(NCH - 1, wr, 63) + VEC <= n;  // wave-uniform
    C nx[NCH][VEC];
    if constexpr (RW) load_row<DT, VEC, NCH, WPR, LNT>((const S *)xin + row * ld, n, wr, lane, neg_inf<C>(), nx);
    for (; row < rows; row += row_step) {
        OS *y = out + row * (size_t)n;
        C v[NCH][VEC];
        if constexpr (RW) {
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int k = 0; k < VEC; k++) v[c][k] = nx[c][k];
            if (row + row_step < rows)
                load_row<DT, VEC, NCH, WPR, LNT>((const S *)xin + (row + row_step) * ld, n, wr, lane, neg_inf<C>(),
                                                 nx);
        } else {
            load_row<DT, VEC, NCH, WPR, LNT>((const S *)xin + row * ld, n, wr, lane, neg_inf<C>(), v);
        }
        C m = neg_inf<C>();
#pragma unroll
        for (int c = 0; c < NCH; c++)
#pragma unroll
            for (int k = 0; k < VEC; k++) m = fmax_c(m, v[c][k]);
        m = row_max<C, WPR>(m, lds);
        C sum = 0;
        if (full) {  // wave-uniform: no per-element guard on whole rows
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int k = 0; k < VEC; k++) {
                    const C e = exp_c(v[c][k] - m);
                    v[c][k] = e;
                    sum = sum + e;
                }
        } else {
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                const int i = chunk_start<VEC, WPR>(c, wr, lane);
#pragma unroll
                for (int k = 0; k < VEC; k++) {
                    const C e = i + k < n ? exp_c(v[c][k] - m) : (C)0;
                    v[c][k] = e;
                    sum = sum + e;
                }
            }
        }
        sum = row_sum<C, WPR>(sum, lds);
        if constexpr (sizeof(C) == 4) {
            const RowDiv div(sum);
            if (div.fast) {
#pragma unroll
                for (int c = 0; c < NCH; c++)
#pragma unroll
                    for (int k = 0; k < VEC; k++) v[c][k] = div(v[c][k]);
            } else {
#pragma unroll
                for (int c = 0; c < NCH; c++)
#pragma unroll
                    for (int k = 0; k < VEC; k++) v[c][k] = v[c][k] / sum;
            }
        } else {
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int k = 0; k < VEC; k++) v[c][k] = v[c][k] / sum;
        }
        store_row<VEC, NCH, WPR, SNT>(y, n, wr, lane, full, v);
    }
}

// 16-byte-aligned vector load of VEC values (VEC * sizeof(T) a multiple of 16).
template <typename T, int VEC>
__device__ __forceinline__ void load_vec16(const T *p, T (&v)[VEC])
{
    static_assert((VEC * sizeof(T)) % 16 == 0, "vector width");
    constexpr int Q = VEC * sizeof(T) / 16;
    union { uint4 raw[Q]; T t[VEC]; } u;
#pragma unroll
    for (int q = 0; q < Q; q++) u.raw[q] = ((const uint4 *)p)[q];
#pragma unroll
    for (int k = 0; k < VEC; k++) v[k] = u.t[k];
}

// Fused layerNorm (cuda_array_ce.c:2295-2323): mean, centered, biased
// variance of the centered values, eps inside the sqrt, true division, then
// gamma and beta (contiguous [n] arrays).  With WPR = 4 a block walks the
// rows blockIdx.x, blockIdx.x + gridDim.x, ... and keeps its gamma / beta
// chunks in registers across them, so they are read once per block instead
// of once per row.
template <int DT, int VEC, int NCH, int WPR, typename CT, bool LNT = false, bool SNT = false>
__global__ __launch_bounds__(64 * RowShape<WPR>::BW) void k_row_layernorm(const void *__restrict__ xin, size_t rows,
                                                                           int n, CT eps,
                                                                           const CT *__restrict__ gamma,
                                                                           const CT *__restrict__ beta,
                                                                           CT *__restrict__ out)
{
    using S = typename RT<DT>::S;
    __shared__ CT lds[RowShape<WPR>::BW];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, wr = wave % WPR;
    size_t row = (size_t)blockIdx.x * RowShape<WPR>::RPB + wave / WPR;
    const size_t row_step = WPR > 1 ? (size_t)gridDim.x : rows;
    if (row >= rows) return;  // WPR > 1: uniform per block
    const bool full = chunk_start<VEC, WPR>(NCH - 1, wr, 63) + VEC <= n;  // wave-uniform
    CT g[NCH][VEC], b[NCH][VEC];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int i = chunk_start<VEC, WPR>(c, wr, lane);
        if (full || i + VEC <= n) {
            if (gamma) load_vec16<CT, VEC>(gamma + i, g[c]);
            if (beta) load_vec16<CT, VEC>(beta + i, b[c]);
        } else {
            for (int k = 0; k < VEC; k++) {
                g[c][k] = gamma && i + k < n ? gamma[i + k] : (CT)1;
                b[c][k] = beta && i + k < n ? beta[i + k] : (CT)0;
            }
        }
    }
    // the next row's loads are issued before this row's reductions, so its
    // HBM latency overlaps the barriers and stores of the current row (only
    // while two rows and gamma/beta fit the register budget)
    constexpr bool PF = NCH * VEC <= 32;
    // one row: reductions, normalisation, gamma / beta, store
    auto process = [&](CT (&v)[NCH][VEC], size_t r) {
        CT *y = out + r * (size_t)n;
        CT s = 0;
#pragma unroll
        for (int c = 0; c < NCH; c++)
#pragma unroll
            for (int k = 0; k < VEC; k++) s = s + v[c][k];
        const CT mean = row_sum<CT, WPR>(s, lds) / (CT)n;
        CT q = 0;
        if (full) {  // wave-uniform: no per-element guard on whole rows
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int k = 0; k < VEC; k++) {
                    const CT d = v[c][k] - mean;
                    v[c][k] = d;
                    q = q + d * d;
                }
        } else {
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                const int i = chunk_start<VEC, WPR>(c, wr, lane);
#pragma unroll
                for (int k = 0; k < VEC; k++) {
                    const CT d = i + k < n ? v[c][k] - mean : (CT)0;
                    v[c][k] = d;
                    q = q + d * d;
                }
            }
        }
        q = row_sum<CT, WPR>(q, lds);
        const CT dev = sqrt_c(q / (CT)n + eps);
        auto finish = [&](auto quot) {
#pragma unroll
            for (int c = 0; c < NCH; c++) {
#pragma unroll
                for (int k = 0; k < VEC; k++) {
                    CT t = quot(v[c][k]);
                    if (gamma) t = t * g[c][k];
                    if (beta) t = t + b[c][k];
                    v[c][k] = t;
                }
            }
        };
        if constexpr (sizeof(CT) == 4) {
            const RowDiv div(dev);
            if (div.fast) finish(div);
            else finish([&](CT a) { return a / dev; });
        } else {
            finish([&](CT a) { return a / dev; });
        }
        store_row<VEC, NCH, WPR, SNT>(y, n, wr, lane, full, v);
    };
    auto src = [&](size_t r) { return (const S *)xin + r * (size_t)n; };
    if constexpr (PF) {
        // two row buffers used in turn: the next row's loads land in one
        // while the other is reduced, normalised and stored (no register
        // copy between them)
        CT b0[NCH][VEC], b1[NCH][VEC];
        load_row<DT, VEC, NCH, WPR, LNT>(src(row), n, wr, lane, (CT)0, b0);
        for (; row < rows; row += 2 * row_step) {
            const size_t r1 = row + row_step;
            if (r1 < rows) load_row<DT, VEC, NCH, WPR, LNT>(src(r1), n, wr, lane, (CT)0, b1);
            process(b0, row);
            if (r1 >= rows) break;
            if (r1 + row_step < rows) load_row<DT, VEC, NCH, WPR, LNT>(src(r1 + row_step), n, wr, lane, (CT)0, b0);
            process(b1, r1);
        }
    } else {
        for (; row < rows; row += row_step) {
            CT v[NCH][VEC];
            load_row<DT, VEC, NCH, WPR, LNT>(src(row), n, wr, lane, (CT)0, v);
            process(v, row);
        }
    }
}

// Streaming (re-reading) variants for rows too long for registers: one
// 256-thread workgroup per row, LDS combine across its four waves.
template <typename T>
__device__ __forceinline__ T block_allreduce_sum(T v, T *lds)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, PT_WAVE);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[w] = v;
    __syncthreads();
    T r = 0;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) r = r + lds[i];
    return r;
}

template <typename T>
__device__ __forceinline__ T block_allreduce_max(T v, T *lds)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmax_c(v, __shfl_xor(v, m, PT_WAVE));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[w] = v;
    __syncthreads();
    T r = lds[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmax_c(r, lds[i]);
    return r;
}

template <int DT, typename OS>
__global__ __launch_bounds__(256) void k_row_softmax_stream(const void *__restrict__ xin, int n,
                                                            size_t ld, OS *__restrict__ out)
{
    using S = typename RT<DT>::S;
    using C = typename RT<DT>::C;
    __shared__ C lds[4];
    const S *x = (const S *)xin + (size_t)blockIdx.x * ld;
    OS *y = out + (size_t)blockIdx.x * (size_t)n;
    C m = neg_inf<C>();
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmax_c(m, RT<DT>::cv(x[i]));
    m = block_allreduce_max(m, lds);
    C s = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s = s + exp_c(RT<DT>::cv(x[i]) - m);
    s = block_allreduce_sum(s, lds);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = (OS)(exp_c(RT<DT>::cv(x[i]) - m) / s);
}

template <int DT, typename CT>
__global__ __launch_bounds__(256) void k_row_layernorm_stream(const void *__restrict__ xin, int n,
                                                              CT eps, const CT *__restrict__ gamma,
                                                              const CT *__restrict__ beta,
                                                              CT *__restrict__ out)
{
    using S = typename RT<DT>::S;
    __shared__ CT lds[4];
    const S *x = (const S *)xin + (size_t)blockIdx.x * (size_t)n;
    CT *y = out + (size_t)blockIdx.x * (size_t)n;
    CT s = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s = s + (CT)RT<DT>::cv(x[i]);
    const CT mean = block_allreduce_sum(s, lds) / (CT)n;
    CT q = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        CT d = (CT)RT<DT>::cv(x[i]) - mean;
        q = q + d * d;
    }
    const CT dev = sqrt_c(block_allreduce_sum(q, lds) / (CT)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        CT t = ((CT)RT<DT>::cv(x[i]) - mean) / dev;
        if (gamma) t = t * gamma[i];
        if (beta) t = t + beta[i];
        y[i] = t;
    }
}

// ========================================================= generic paths
// Generic element access for every dtype (integer sums wrap: the
// accumulator is uint64 and is truncated on store, matching HostArray's
// modular sums, contiguous_array_ce.c:1149-1161, 1229-1233).
struct GenAcc {
    int op, dt;
    double d;      // float accumulation (sum/mean/prod/max/min of floats, mean of ints)
    uint64_t u;    // integer sum/prod bits
    int64_t si;    // signed integer extremum
    uint64_t ui;   // unsigned integer extremum
    int have;
    Mom m;
    double best; int bi;  // arg reductions (float compare in double; exact for <=32-bit ints)
    int64_t bsi; uint64_t bui;
};

__device__ __forceinline__ bool is_signed_int(int dt) { return dt >= PT_INT8 && dt <= PT_INT64; }
__device__ __forceinline__ bool is_unsigned_int(int dt)
{
    return (dt >= PT_UINT8 && dt <= PT_UINT64) || dt == PT_BOOL;
}
__device__ __forceinline__ bool is_float_dt(int dt)
{
    return dt == PT_FLOAT32 || dt == PT_FLOAT64 || dt == PT_FLOAT16 || dt == PT_BFLOAT16;
}

__device__ __forceinline__ int64_t load_i64(const void *p, int dt, size_t i)
{
    switch (dt) {
    case PT_INT8: return ((const int8_t *)p)[i];
    case PT_INT16: return ((const int16_t *)p)[i];
    case PT_INT32: return ((const int32_t *)p)[i];
    default: return ((const int64_t *)p)[i];
    }
}
__device__ __forceinline__ uint64_t load_u64(const void *p, int dt, size_t i)
{
    switch (dt) {
    case PT_UINT8: return ((const uint8_t *)p)[i];
    case PT_BOOL: return ((const uint8_t *)p)[i] != 0;
    case PT_UINT16: return ((const uint16_t *)p)[i];
    case PT_UINT32: return ((const uint32_t *)p)[i];
    default: return ((const uint64_t *)p)[i];
    }
}

__device__ void gen_init(GenAcc &a, int op, int dt)
{
    a.op = op; a.dt = dt; a.have = 0; a.u = (op == R_PROD || op == R_ALL) ? 1 : 0;
    a.d = op == R_PROD ? 1.0 : (op == R_MAX ? -INFINITY : (op == R_MIN ? INFINITY : 0.0));
    a.si = 0; a.ui = 0; a.m = Mom{0, 0, 0};
    a.best = op == R_ARGMAX ? -INFINITY : INFINITY; a.bi = 0;
    a.bsi = op == R_ARGMAX ? INT64_MIN : INT64_MAX;
    a.bui = op == R_ARGMAX ? 0 : UINT64_MAX;
}

__device__ void gen_add(GenAcc &a, const void *p, size_t off, int idx)
{
    const int dt = a.dt;
    switch (a.op) {
    case R_SUM:
    case R_PROD:
        if (is_float_dt(dt)) {
            double v = load_as_double(p, dt, off);
            if (dt == PT_FLOAT64) a.d = a.op == R_SUM ? a.d + v : a.d * v;
            else a.d = a.op == R_SUM ? (double)((float)a.d + (float)v) : (double)((float)a.d * (float)v);
        } else {
            uint64_t v = is_signed_int(dt) ? (uint64_t)load_i64(p, dt, off) : load_u64(p, dt, off);
            if (dt == PT_BOOL) a.u = a.op == R_SUM ? (a.u || v) : (a.u && v);
            else a.u = a.op == R_SUM ? a.u + v : a.u * v;
        }
        break;
    case R_MEAN: {
        double v = is_float_dt(dt) ? load_as_double(p, dt, off)
                 : is_signed_int(dt) ? (double)load_i64(p, dt, off) : (double)load_u64(p, dt, off);
        if (dt == PT_FLOAT32 || dt == PT_FLOAT16 || dt == PT_BFLOAT16) a.d = (double)((float)a.d + (float)v);
        else a.d = a.d + v;
        break;
    }
    case R_MAX:
    case R_MIN:
        if (is_float_dt(dt)) {
            double v = load_as_double(p, dt, off);
            a.d = a.op == R_MAX ? fmax(a.d, v) : fmin(a.d, v);
        } else if (is_signed_int(dt)) {
            int64_t v = load_i64(p, dt, off);
            if (!a.have || (a.op == R_MAX ? v > a.si : v < a.si)) a.si = v;
            a.have = 1;
        } else {
            uint64_t v = load_u64(p, dt, off);
            if (!a.have || (a.op == R_MAX ? v > a.ui : v < a.ui)) a.ui = v;
            a.have = 1;
        }
        break;
    case R_ARGMAX:
    case R_ARGMIN: {
        bool mx = a.op == R_ARGMAX;
        if (is_float_dt(dt)) {
            double v = load_as_double(p, dt, off);
            if (mx ? v > a.best : v < a.best) { a.best = v; a.bi = idx; }
        } else if (is_signed_int(dt)) {
            int64_t v = load_i64(p, dt, off);
            if (mx ? v > a.bsi : v < a.bsi) { a.bsi = v; a.bi = idx; }
        } else {
            uint64_t v = load_u64(p, dt, off);
            if (mx ? v > a.bui : v < a.bui) { a.bui = v; a.bi = idx; }
        }
        break;
    }
    case R_VAR: {
        double v = is_float_dt(dt) ? load_as_double(p, dt, off)
                 : is_signed_int(dt) ? (double)load_i64(p, dt, off) : (double)load_u64(p, dt, off);
        Mom s = {1.0, v, v - v};
        a.m = mom_combine(a.m, s);
        break;
    }
    case R_ALL:
    case R_ANY: {
        // an element is true when it compares unequal to zero (NaN is true,
        // -0.0 is false), as AllOpT / AnyOpT, cuda_op_functors.cuh:141-151
        bool nz = is_float_dt(dt) ? load_as_double(p, dt, off) != 0.0
                : is_signed_int(dt) ? load_i64(p, dt, off) != 0 : load_u64(p, dt, off) != 0;
        a.u = a.op == R_ALL ? (a.u && nz) : (a.u || nz);
        break;
    }
    }
}

__device__ void gen_merge(GenAcc &a, const GenAcc &b)
{
    const int dt = a.dt;
    switch (a.op) {
    case R_SUM:
    case R_PROD:
        if (is_float_dt(dt)) {
            if (dt == PT_FLOAT64) a.d = a.op == R_SUM ? a.d + b.d : a.d * b.d;
            else a.d = a.op == R_SUM ? (double)((float)a.d + (float)b.d) : (double)((float)a.d * (float)b.d);
        } else if (dt == PT_BOOL) {
            a.u = a.op == R_SUM ? (a.u || b.u) : (a.u && b.u);
        } else {
            a.u = a.op == R_SUM ? a.u + b.u : a.u * b.u;
        }
        break;
    case R_MEAN:
        if (dt == PT_FLOAT32 || dt == PT_FLOAT16 || dt == PT_BFLOAT16) a.d = (double)((float)a.d + (float)b.d);
        else a.d = a.d + b.d;
        break;
    case R_MAX:
    case R_MIN:
        if (is_float_dt(dt)) {
            a.d = a.op == R_MAX ? fmax(a.d, b.d) : fmin(a.d, b.d);
        } else if (b.have) {
            if (is_signed_int(dt)) {
                if (!a.have || (a.op == R_MAX ? b.si > a.si : b.si < a.si)) a.si = b.si;
            } else {
                if (!a.have || (a.op == R_MAX ? b.ui > a.ui : b.ui < a.ui)) a.ui = b.ui;
            }
            a.have = 1;
        }
        break;
    case R_ARGMAX:
    case R_ARGMIN: {
        bool mx = a.op == R_ARGMAX;
        if (is_float_dt(dt)) {
            if ((mx ? b.best > a.best : b.best < a.best) || (b.best == a.best && b.bi < a.bi)) {
                a.best = b.best; a.bi = b.bi;
            }
        } else if (is_signed_int(dt)) {
            if ((mx ? b.bsi > a.bsi : b.bsi < a.bsi) || (b.bsi == a.bsi && b.bi < a.bi)) {
                a.bsi = b.bsi; a.bi = b.bi;
            }
        } else {
            if ((mx ? b.bui > a.bui : b.bui < a.bui) || (b.bui == a.bui && b.bi < a.bi)) {
                a.bui = b.bui; a.bi = b.bi;
            }
        }
        break;
    }
    case R_VAR:
        a.m = mom_combine(a.m, b.m);
        break;
    case R_ALL:
        a.u = a.u && b.u;
        break;
    case R_ANY:
        a.u = a.u || b.u;
        break;
    }
}

__device__ void store_bits_dt(void *out, int dt, size_t i, uint64_t bits)
{
    switch (dt) {
    case PT_BOOL: ((uint8_t *)out)[i] = bits != 0; break;
    case PT_INT8: case PT_UINT8: ((uint8_t *)out)[i] = (uint8_t)bits; break;
    case PT_INT16: case PT_UINT16: ((uint16_t *)out)[i] = (uint16_t)bits; break;
    case PT_INT32: case PT_UINT32: ((uint32_t *)out)[i] = (uint32_t)bits; break;
    default: ((uint64_t *)out)[i] = bits; break;
    }
}

struct GenParams {
    int ndims;
    int axis;          // -1: all elements
    int shape[PT_MAX_DIMS];
    size_t strides[PT_MAX_DIMS];
    size_t count;      // reduced elements per output
    size_t outputs;
    size_t base;
    int out_dt;
    int correction;
    int take_sqrt;
};

__device__ void gen_finish(const GenAcc &a, const GenParams &p, void *out, size_t o)
{
    const int dt = a.dt;
    switch (a.op) {
    case R_SUM:
    case R_PROD:
        if (is_float_dt(dt)) store_out(out, p.out_dt, o, a.d);
        else store_bits_dt(out, p.out_dt, o, a.u);
        break;
    case R_MEAN: {
        double r;
        if (p.count == 0) r = NAN;
        else if (p.out_dt == PT_FLOAT32) r = (double)((float)a.d / (float)p.count);
        else r = a.d / (double)p.count;
        store_out(out, p.out_dt, o, r);
        break;
    }
    case R_MAX:
    case R_MIN:
        if (is_float_dt(dt)) store_out(out, p.out_dt, o, a.d);
        else if (is_signed_int(dt)) store_bits_dt(out, p.out_dt, o, (uint64_t)a.si);
        else store_bits_dt(out, p.out_dt, o, a.ui);
        break;
    case R_ARGMAX:
    case R_ARGMIN:
        ((int32_t *)out)[o] = a.bi;
        break;
    case R_VAR: {
        double var = a.m.m2 / (double)(p.count - (size_t)p.correction);
        store_out(out, p.out_dt, o, p.take_sqrt ? sqrt(var) : var);
        break;
    }
    case R_ALL:
    case R_ANY:
        ((uint8_t *)out)[o] = a.u != 0;
        break;
    }
}

__device__ __forceinline__ size_t gen_offset(const GenParams &p, size_t o, size_t i)
{
    size_t off = p.base;
    if (p.axis >= 0) {
        size_t rem = o;
        for (int d = p.ndims - 1; d >= 0; d--) {
            if (d == p.axis) continue;
            off += (rem % (size_t)p.shape[d]) * p.strides[d];
            rem /= (size_t)p.shape[d];
        }
        off += i * p.strides[p.axis];
    } else {
        size_t rem = i;
        for (int d = p.ndims - 1; d >= 0; d--) {
            off += (rem % (size_t)p.shape[d]) * p.strides[d];
            rem /= (size_t)p.shape[d];
        }
    }
    return off;
}

// Block-cooperative merge of GenAcc through LDS (lane 0 holds the result).
__device__ void gen_block_merge(GenAcc &a, GenAcc *lds)
{
    lds[threadIdx.x] = a;
    __syncthreads();
    for (unsigned s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) gen_merge(lds[threadIdx.x], lds[threadIdx.x + s]);
        __syncthreads();
    }
    a = lds[0];
}

// One workgroup per output, every layout.  Threads take contiguous slices
// of the reduced index range so that sequential per-thread order (and
// therefore the lowest-index tie rule) is preserved.
__global__ __launch_bounds__(128) void k_strided_reduce(const void *__restrict__ x,
                                                        void *__restrict__ out, int op, int dt,
                                                        GenParams p)
{
    __shared__ GenAcc lds[128];
    const size_t o = blockIdx.x;
    if (o >= p.outputs) return;
    GenAcc a;
    gen_init(a, op, dt);
    size_t per = (p.count + blockDim.x - 1) / blockDim.x;
    size_t lo = threadIdx.x * per, hi = lo + per < p.count ? lo + per : p.count;
    for (size_t i = lo; i < hi; i++) gen_add(a, x, gen_offset(p, o, i), (int)i);
    gen_block_merge(a, lds);
    if (threadIdx.x == 0) gen_finish(a, p, out, o);
}

// Contiguous (outer, n, inner) reduction over the middle axis: a 64x4
// workgroup covers 64 consecutive inner positions (coalesced) and splits n
// over its 4 waves in contiguous slices.
__global__ __launch_bounds__(256) void k_column_reduce(const void *__restrict__ x,
                                                       void *__restrict__ out, int op, int dt,
                                                       size_t outer, size_t n, size_t inner,
                                                       GenParams p)
{
    __shared__ GenAcc lds[4][64];
    const int lx = threadIdx.x & 63, ly = threadIdx.x >> 6;
    const size_t col = (size_t)blockIdx.x * 64 + lx;
    const size_t o_outer = blockIdx.y;
    GenAcc a;
    gen_init(a, op, dt);
    if (col < inner) {
        size_t per = (n + 3) / 4;
        size_t lo = ly * per, hi = lo + per < n ? lo + per : n;
        const size_t base = o_outer * n * inner + col;
        for (size_t i = lo; i < hi; i++) gen_add(a, x, base + i * inner, (int)i);
    }
    lds[ly][lx] = a;
    __syncthreads();
    if (ly == 0 && col < inner) {
        for (int k = 1; k < 4; k++) gen_merge(a, lds[k][lx]);
        gen_finish(a, p, out, o_outer * inner + col);
    }
}

// Split column reduction for short outer / long middle axes: workgroup
// (cx, split, o) reduces 64 columns over its contiguous slice of the middle
// axis into partial[(o * splits + split) * inner + col]; the final pass
// merges the slices of each column in order (index ties resolve to the
// lowest index as in the single-pass kernel).
__global__ __launch_bounds__(256) void k_column_partial(const void *__restrict__ x, int op, int dt,
                                                        size_t n, size_t inner, size_t slice,
                                                        GenAcc *__restrict__ partial)
{
    __shared__ GenAcc lds[4][64];
    const int lx = threadIdx.x & 63, ly = threadIdx.x >> 6;
    const size_t col = (size_t)blockIdx.x * 64 + lx;
    const size_t split = blockIdx.y, o_outer = blockIdx.z;
    GenAcc a;
    gen_init(a, op, dt);
    const size_t s_lo = split * slice;
    const size_t s_hi = s_lo + slice < n ? s_lo + slice : n;
    if (col < inner && s_lo < s_hi) {
        size_t per = (s_hi - s_lo + 3) / 4;
        size_t lo = s_lo + ly * per, hi = lo + per < s_hi ? lo + per : s_hi;
        const size_t base = o_outer * n * inner + col;
        for (size_t i = lo; i < hi; i++) gen_add(a, x, base + i * inner, (int)i);
    }
    lds[ly][lx] = a;
    __syncthreads();
    if (ly == 0 && col < inner) {
        for (int k = 1; k < 4; k++) gen_merge(a, lds[k][lx]);
        partial[(o_outer * gridDim.y + split) * inner + col] = a;
    }
}

__global__ __launch_bounds__(256) void k_column_final(const GenAcc *__restrict__ partial, size_t outer,
                                                      size_t splits, size_t inner, void *__restrict__ out,
                                                      GenParams p)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= outer * inner) return;
    const size_t o = i / inner, col = i % inner;
    GenAcc a = partial[(o * splits) * inner + col];
    for (size_t k = 1; k < splits; k++) gen_merge(a, partial[(o * splits + k) * inner + col]);
    gen_finish(a, p, out, i);
}

// Typed column reductions (floating inputs; sum, mean, prod, max, min) of a
// contiguous [outer, n, inner] input along n.  A 256-thread block owns
// 64 * V adjacent columns; its four waves take interleaved rows of the
// block's row slice (adjacent rows in flight together), each lane keeping V
// columns in registers, and meet in LDS in wave order.  With one slice per
// column the block writes the result; otherwise it writes a partial per
// slice and k_col_final_t merges them in slice order.
template <int DT, int OP, int V>
__global__ __launch_bounds__(256) void k_col_reduce_t(const void *__restrict__ xin, size_t n, size_t inner,
                                                      size_t slice, void *__restrict__ out, int out_dt,
                                                      typename RT<DT>::C *__restrict__ partial)
{
    using S = typename RT<DT>::S;
    using C = typename RT<DT>::C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t col = ((size_t)blockIdx.x * 64 + lane) * V;
    const size_t split = blockIdx.y, o = blockIdx.z;
    const size_t lo = split * slice;
    const size_t hi = lo + slice < n ? lo + slice : n;
    Acc<C, OP> acc[V];
    if (col < inner) {
        const S *x = (const S *)xin + o * n * inner + col;
        size_t r = lo + wave;
        for (; r + 12 < hi; r += 16) {
            C v[4][V];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if constexpr (V > 1) load_chunk<DT, V>(x + (r + 4 * u) * inner, v[u]);
                else v[u][0] = RT<DT>::cv(x[(r + 4 * u) * inner]);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int k = 0; k < V; k++) acc[k].add(v[u][k], 0);
        }
        for (; r < hi; r += 4) {
            C v[V];
            if constexpr (V > 1) load_chunk<DT, V>(x + r * inner, v);
            else v[0] = RT<DT>::cv(x[r * inner]);
#pragma unroll
            for (int k = 0; k < V; k++) acc[k].add(v[k], 0);
        }
    }
    __shared__ C part[3][64 * V];
    if (wave > 0)
#pragma unroll
        for (int k = 0; k < V; k++) part[wave - 1][lane * V + k] = acc[k].s;
    __syncthreads();
    if (wave != 0 || col >= inner) return;
#pragma unroll
    for (int w = 0; w < 3; w++)
#pragma unroll
        for (int k = 0; k < V; k++) {
            Acc<C, OP> b;
            b.s = part[w][lane * V + k];
            acc[k].merge(b);
        }
#pragma unroll
    for (int k = 0; k < V; k++) {
        if (partial) {
            partial[(o * gridDim.y + split) * inner + col + k] = acc[k].s;
        } else {
            C r = OP == R_MEAN ? acc[k].s / (C)n : acc[k].s;
            store_out(out, out_dt, o * inner + col + k, r);
        }
    }
}

// Merge of the per-slice partials [outer][splits][inner]: wave w of a block
// merges a contiguous quarter of the slices for 64 columns, then wave 0
// merges the quarters in order.
template <int DT, int OP>
__global__ __launch_bounds__(256) void k_col_final_t(const typename RT<DT>::C *__restrict__ partial,
                                                     size_t splits, size_t inner, size_t n,
                                                     void *__restrict__ out, int out_dt)
{
    using C = typename RT<DT>::C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t col = (size_t)blockIdx.x * 64 + lane, o = blockIdx.y;
    const size_t q = (splits + 3) / 4;
    const size_t lo = wave * q, hi = lo + q < splits ? lo + q : splits;
    Acc<C, OP> acc;
    if (col < inner) {
        const C *p = partial + o * splits * inner + col;
        size_t k = lo;
        for (; k + 3 < hi; k += 4) {
            C v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = p[(k + u) * inner];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                Acc<C, OP> b;
                b.s = v[u];
                acc.merge(b);
            }
        }
        for (; k < hi; k++) {
            Acc<C, OP> b;
            b.s = p[k * inner];
            acc.merge(b);
        }
    }
    __shared__ C part[3][64];
    if (wave > 0) part[wave - 1][lane] = acc.s;
    __syncthreads();
    if (wave != 0 || col >= inner) return;
    for (int w = 0; w < 3; w++) {
        Acc<C, OP> b;
        b.s = part[w][lane];
        acc.merge(b);
    }
    C r = OP == R_MEAN ? acc.s / (C)n : acc.s;
    store_out(out, out_dt, o * inner + col, r);
}

// Global reduction of a contiguous input: stage 1 writes one GenAcc per
// workgroup (each takes a contiguous slice, so index ties resolve to the
// lowest index), stage 2 merges them in order.
__global__ __launch_bounds__(256) void k_global_partial(const void *__restrict__ x, int op, int dt,
                                                        size_t count, size_t base,
                                                        GenAcc *__restrict__ partials)
{
    __shared__ GenAcc lds[256];
    size_t per_block = (count + gridDim.x - 1) / gridDim.x;
    size_t blo = blockIdx.x * per_block;
    size_t bhi = blo + per_block < count ? blo + per_block : count;
    GenAcc a;
    gen_init(a, op, dt);
    if (blo < bhi) {
        size_t len = bhi - blo;
        size_t per = (len + blockDim.x - 1) / blockDim.x;
        size_t lo = blo + threadIdx.x * per;
        size_t hi = lo + per < bhi ? lo + per : bhi;
        for (size_t i = lo; i < hi; i++) gen_add(a, x, base + i, (int)i);
    }
    gen_block_merge(a, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = a;
}

__global__ __launch_bounds__(256) void k_global_final(const GenAcc *__restrict__ partials, int nparts,
                                                      void *__restrict__ out, GenParams p)
{
    __shared__ GenAcc lds[256];
    GenAcc a;
    int per = (nparts + blockDim.x - 1) / blockDim.x;
    int lo = threadIdx.x * per, hi = lo + per < nparts ? lo + per : nparts;
    if (lo < hi) {
        a = partials[lo];
        for (int i = lo + 1; i < hi; i++) gen_merge(a, partials[i]);
    } else {
        gen_init(a, partials[0].op, partials[0].dt);
    }
    gen_block_merge(a, lds);
    if (threadIdx.x == 0) gen_finish(a, p, out, 0);
}

// Fill used for empty-axis identities (sum 0, prod 1, mean NaN).
__global__ void k_fill_identity(void *out, int out_dt, size_t n, double value)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (out_dt == PT_FLOAT32) ((float *)out)[i] = (float)value;
    else if (out_dt == PT_FLOAT64) ((double *)out)[i] = value;
    else store_bits_dt(out, out_dt, i, (uint64_t)(int64_t)value);
}

// ================================================================== host
static int red_op_of(int op)
{
    switch (op) {
    case PT_OP_REDUCE_SUM: return R_SUM;
    case PT_OP_REDUCE_MEAN: return R_MEAN;
    case PT_OP_REDUCE_MAX: return R_MAX;
    case PT_OP_REDUCE_MIN: return R_MIN;
    case PT_OP_REDUCE_PROD: return R_PROD;
    case PT_OP_ARG_MAX: return R_ARGMAX;
    case PT_OP_ARG_MIN: return R_ARGMIN;
    case PT_OP_REDUCE_ALL: return R_ALL;
    case PT_OP_REDUCE_ANY: return R_ANY;
    default: return -1;
    }
}

// Collapse the non-axis dims into rows with a uniform pitch; true if the
// reduced axis is unit-stride and rows are equally spaced.
static bool as_rows(const int *shape, const size_t *strides, int ndims, int axis,
                    size_t *rows, size_t *ld)
{
    if (axis < 0 || (strides[axis] != 1 && shape[axis] != 1)) return false;
    size_t r = 1, pitch = 0, expect = 0;
    bool first = true;
    for (int d = ndims - 1; d >= 0; d--) {
        if (d == axis || shape[d] == 1) continue;
        if (first) {
            pitch = strides[d];
            expect = strides[d] * (size_t)shape[d];
            first = false;
        } else {
            if (strides[d] != expect) return false;
            expect = strides[d] * (size_t)shape[d];
        }
        r *= (size_t)shape[d];
    }
    *rows = r;
    // pitch may be below n (zero-stride broadcast rows): reads may overlap
    *ld = first ? (size_t)shape[axis] : pitch;
    return true;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Waves per row of the block-per-row kernels on fp32 rows of 5 to 16
// chunks of 16 bytes per wave-row step (up to 4096 floats): 8 for every op.
// On config 2 (X[8192, 4096]) against 4 waves: sum 20.5 against 20.8 us,
// softmax 41.6 against 42.9 us, layerNorm 43.4 against 43.9 us, variance
// (single-exchange Chan merge) 20.9-21.0 against 21.1; argmax / argmin with
// the two-pass k_row_arg2 20.4-20.5 against 21.3-21.4 us for the 4-wave
// (value, index) kernel (8 waves of that kernel took 22.8 us).  16 waves
// (1024-thread blocks) ran 30-60 % slower for every op, and nontemporal row
// loads or stores slowed softmax and layerNorm at every width.  PT_ROW_WAVES
// (4 or 8) overrides the choice, a tuning knob read once from the
// environment.
static int row_waves()
{
    static const int w = [] {
        const char *e = getenv("PT_ROW_WAVES");
        const int v = e && *e ? atoi(e) : 0;
        return (v == 4 || v == 8) ? v : 8;
    }();
    return w;
}

template <int DT, int OP>
static void launch_rows_t(const void *x, size_t rows, int n, size_t ld, void *out, int out_dt,
                          int correction, int take_sqrt, hipStream_t s)
{
    constexpr int V = RT<DT>::V;
    dim3 block(256);
    if constexpr (DT == PT_FLOAT32) {
        const int chunks = (n + 64 * V - 1) / (64 * V);
        if (row_waves() == 8 && n % V == 0 && ld % V == 0 && aligned16(x) &&
            chunks > 4 && chunks <= 16) {
            dim3 grid1((unsigned)rows), block8(512);
            if constexpr (OP == R_VAR)
                k_row_moments<DT, V, 2, 8><<<grid1, block8, 0, s>>>(x, rows, n, ld, out, out_dt, correction, take_sqrt);
            else if constexpr (OP == R_ARGMAX || OP == R_ARGMIN)
                k_row_arg2<V, 2, 8, OP == R_ARGMAX><<<grid1, block8, 0, s>>>(x, rows, n, ld, out);
            else
                k_row_reduce<DT, OP, V, 8><<<grid1, block8, 0, s>>>(x, rows, n, ld, out, out_dt, 0, 0);
            return;
        }
    }
    if constexpr (OP == R_VAR) {
        // rows that fit in registers: two-pass moments, one block per row
        int chunks = (n + 64 * V - 1) / (64 * V);
        if (n % V == 0 && ld % V == 0 && aligned16(x) && chunks > 4) {
            dim3 grid1((unsigned)rows);
            if (chunks <= 8) {
                k_row_moments<DT, V, 2, 4><<<grid1, block, 0, s>>>(x, rows, n, ld, out, out_dt, correction, take_sqrt);
                return;
            }
            if (chunks <= 16) {
                k_row_moments<DT, V, 4, 4><<<grid1, block, 0, s>>>(x, rows, n, ld, out, out_dt, correction, take_sqrt);
                return;
            }
            if (chunks <= 32) {
                k_row_moments<DT, V, 8, 4><<<grid1, block, 0, s>>>(x, rows, n, ld, out, out_dt, correction, take_sqrt);
                return;
            }
        }
    }
    if (n % V == 0 && ld % V == 0 && aligned16(x)) {
        // long rows: a block per row (16 chunks of 16 B in flight per row)
        if (n >= 4 * 64 * V * 2)
            k_row_reduce<DT, OP, V, 4><<<dim3((unsigned)rows), block, 0, s>>>(x, rows, n, ld, out, out_dt,
                                                                              correction, take_sqrt);
        else
            k_row_reduce<DT, OP, V, 1><<<dim3((unsigned)((rows + 3) / 4)), block, 0, s>>>(
                x, rows, n, ld, out, out_dt, correction, take_sqrt);
    } else {
        k_row_reduce<DT, OP, 1, 1><<<dim3((unsigned)((rows + 3) / 4)), block, 0, s>>>(x, rows, n, ld, out, out_dt,
                                                                                       correction, take_sqrt);
    }
}

template <int DT>
static bool launch_rows_dt(int rop, const void *x, size_t rows, int n, size_t ld, void *out,
                           int out_dt, int correction, int take_sqrt, hipStream_t s)
{
    switch (rop) {
    case R_SUM: launch_rows_t<DT, R_SUM>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_MEAN: launch_rows_t<DT, R_MEAN>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_MAX: launch_rows_t<DT, R_MAX>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_MIN: launch_rows_t<DT, R_MIN>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_PROD: launch_rows_t<DT, R_PROD>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_ARGMAX: launch_rows_t<DT, R_ARGMAX>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_ARGMIN: launch_rows_t<DT, R_ARGMIN>(x, rows, n, ld, out, out_dt, 0, 0, s); return true;
    case R_VAR: launch_rows_t<DT, R_VAR>(x, rows, n, ld, out, out_dt, correction, take_sqrt, s); return true;
    }
    return false;
}

static bool launch_rows(int dt, int rop, const void *x, size_t rows, int n, size_t ld, void *out,
                        int out_dt, int correction, int take_sqrt, hipStream_t s)
{
    switch (dt) {
    case PT_FLOAT32: return launch_rows_dt<PT_FLOAT32>(rop, x, rows, n, ld, out, out_dt, correction, take_sqrt, s);
    case PT_FLOAT64: return launch_rows_dt<PT_FLOAT64>(rop, x, rows, n, ld, out, out_dt, correction, take_sqrt, s);
    case PT_BFLOAT16: return launch_rows_dt<PT_BFLOAT16>(rop, x, rows, n, ld, out, out_dt, correction, take_sqrt, s);
    case PT_FLOAT16: return launch_rows_dt<PT_FLOAT16>(rop, x, rows, n, ld, out, out_dt, correction, take_sqrt, s);
    default: return false;
    }
}

static int result_dtype(int dtype, int rop)
{
    if (rop == R_ARGMAX || rop == R_ARGMIN) return PT_INT32;
    if (rop == R_ALL || rop == R_ANY) return PT_BOOL;
    if (rop == R_VAR) return (dtype == PT_FLOAT32 || dtype == PT_FLOAT16 || dtype == PT_BFLOAT16)
                          ? PT_FLOAT32 : PT_FLOAT64;
    if (rop == R_MEAN) return (dtype == PT_FLOAT32 || dtype == PT_FLOAT16 || dtype == PT_BFLOAT16)
                           ? PT_FLOAT32 : PT_FLOAT64;
    if (dtype == PT_FLOAT16 || dtype == PT_BFLOAT16) return PT_FLOAT32;
    return dtype;
}

// Column launcher of k_col_reduce_t: whole-16-byte column packs when the
// row pitch and base keep them aligned; when the column blocks cannot fill
// the GPU the rows are split into slices (at least 64 rows each, at most
// 128 slices) merged by k_col_final_t.
template <int DT, int OP>
static pt_status launch_cols_t(const void *x, size_t outer, size_t n, size_t inner, void *out, int out_dt,
                               hipStream_t s)
{
    using C = typename RT<DT>::C;
    constexpr int V = RT<DT>::V;
    const bool vec = inner % V == 0 && aligned16(x);
    const size_t cols_per_block = vec ? 64 * V : 64;
    const size_t col_blocks = (inner + cols_per_block - 1) / cols_per_block;
    size_t splits = 1;
    if (col_blocks * outer < 1024) {
        splits = (2048 + col_blocks * outer - 1) / (col_blocks * outer);
        size_t max_splits = n / 64;
        if (splits > max_splits) splits = max_splits;
        if (splits > 128) splits = 128;
        if (splits < 1) splits = 1;
    }
    const size_t slice = (n + splits - 1) / splits;
    splits = (n + slice - 1) / slice;
    C *partial = nullptr;
    if (splits > 1) PT_TRY(scratch_alloc((void **)&partial, sizeof(C) * outer * splits * inner, s));
    dim3 grid((unsigned)col_blocks, (unsigned)splits, (unsigned)outer);
    if (vec) k_col_reduce_t<DT, OP, V><<<grid, 256, 0, s>>>(x, n, inner, slice, out, out_dt, partial);
    else k_col_reduce_t<DT, OP, 1><<<grid, 256, 0, s>>>(x, n, inner, slice, out, out_dt, partial);
    hipError_t e1 = hipGetLastError(), e2 = hipSuccess;
    if (splits > 1) {
        k_col_final_t<DT, OP><<<dim3((unsigned)((inner + 63) / 64), (unsigned)outer), 256, 0, s>>>(
            partial, splits, inner, n, out, out_dt);
        e2 = hipGetLastError();
        scratch_free(partial, s);
    }
    PT_TRY(check_hip(e1, "column reduction"));
    PT_TRY(check_hip(e2, "column reduction (merge)"));
    return PT_OK;
}

template <int DT>
static int launch_cols_dt(int rop, const void *x, size_t outer, size_t n, size_t inner, void *out, int out_dt,
                          hipStream_t s)
{
    switch (rop) {
    case R_SUM: return launch_cols_t<DT, R_SUM>(x, outer, n, inner, out, out_dt, s);
    case R_MEAN: return launch_cols_t<DT, R_MEAN>(x, outer, n, inner, out, out_dt, s);
    case R_PROD: return launch_cols_t<DT, R_PROD>(x, outer, n, inner, out, out_dt, s);
    case R_MAX: return launch_cols_t<DT, R_MAX>(x, outer, n, inner, out, out_dt, s);
    case R_MIN: return launch_cols_t<DT, R_MIN>(x, outer, n, inner, out, out_dt, s);
    }
    return -1;
}

// Returns -1 when the typed column path does not cover (dtype, op).
static int launch_cols(int dt, int rop, const void *x, size_t outer, size_t n, size_t inner, void *out,
                       int out_dt, hipStream_t s)
{
    switch (dt) {
    case PT_FLOAT32: return launch_cols_dt<PT_FLOAT32>(rop, x, outer, n, inner, out, out_dt, s);
    case PT_FLOAT64: return launch_cols_dt<PT_FLOAT64>(rop, x, outer, n, inner, out, out_dt, s);
    case PT_BFLOAT16: return launch_cols_dt<PT_BFLOAT16>(rop, x, outer, n, inner, out, out_dt, s);
    case PT_FLOAT16: return launch_cols_dt<PT_FLOAT16>(rop, x, outer, n, inner, out, out_dt, s);
    }
    return -1;
}

// Shared driver of pt_reduce / pt_arg_reduce / pt_moments.
static pt_status reduce_driver(const void *input, void *output, int dtype, int rop, int out_dt,
                               const int *shape, const size_t *strides, int ndims, int axis,
                               size_t base_offset, int correction, int take_sqrt,
                               pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!dtype_valid(dtype)) return fail(PT_ERR_INVALID, "reduction: unknown dtype %d", dtype);
    if (ndims < 0 || ndims > PT_MAX_DIMS) return fail(PT_ERR_INVALID, "reduction: rank %d outside [0, 10]", ndims);
    if (axis >= ndims) return fail(PT_ERR_INVALID, "reduction axis %d outside rank %d", axis, ndims);
    for (int d = 0; d < ndims; d++)
        if (shape[d] < 0) return fail(PT_ERR_INVALID, "reduction: negative extent");
    hipStream_t s = stream_of(stream);
    size_t total = numel(shape, ndims);
    size_t count = axis < 0 ? total : (size_t)shape[axis];
    size_t outputs = 1;
    if (axis >= 0)
        for (int d = 0; d < ndims; d++)
            if (d != axis) outputs *= (size_t)shape[d];
    if (outputs == 0) return PT_OK;
    if (rop == R_VAR && (correction < 0 || (size_t)correction >= count))
        return fail(PT_ERR_INVALID, "Variance correction must be non-negative and smaller than the reduced dimension");
    if (count == 0) {
        if (rop == R_MAX || rop == R_MIN)
            return fail(PT_ERR_INVALID, "Min/max reduction has no identity for an empty axis");
        if (rop == R_ARGMAX || rop == R_ARGMIN)
            return fail(PT_ERR_INVALID, "Arg reduction has no identity for an empty axis");
        double ident = (rop == R_PROD || rop == R_ALL) ? 1.0 : (rop == R_MEAN ? NAN : 0.0);
        k_fill_identity<<<(unsigned)((outputs + 255) / 256), 256, 0, s>>>(output, out_dt, outputs, ident);
        PT_LAUNCH_CHECK("reduction identity fill");
        return PT_OK;
    }
    if (count > (size_t)INT32_MAX && (rop == R_ARGMAX || rop == R_ARGMIN))
        return fail(PT_ERR_INVALID, "arg reduction index exceeds int32");

    GenParams p = {};
    p.ndims = ndims;
    p.axis = axis;
    for (int d = 0; d < ndims; d++) {
        p.shape[d] = shape[d];
        p.strides[d] = strides[d];
    }
    p.count = count;
    p.outputs = outputs;
    p.base = base_offset;
    p.out_dt = out_dt;
    p.correction = correction;
    p.take_sqrt = take_sqrt;

    const size_t esz = dtype_size(dtype);
    const char *xb = (const char *)input + base_offset * esz;

    // rows: fast wave-per-row path (floating dtypes)
    size_t rows = 0, ld = 0;
    if (axis >= 0 && dtype_is_floating(dtype) && count <= (size_t)INT32_MAX &&
        as_rows(shape, strides, ndims, axis, &rows, &ld)) {
        if (launch_rows(dtype, rop, xb, rows, (int)count, ld, output, out_dt, correction, take_sqrt, s)) {
            PT_LAUNCH_CHECK("row reduction");
            counters().row_reduce_calls++;
            return PT_OK;
        }
    }
    bool contiguous = is_row_major(shape, strides, ndims);
    if (axis < 0 && contiguous) {
        int parts = (int)((total + 8191) / 8192);
        if (parts > 1024) parts = 1024;
        if (parts < 1) parts = 1;
        GenAcc *partials = nullptr;
        PT_TRY(scratch_alloc((void **)&partials, sizeof(GenAcc) * (size_t)parts, s));
        k_global_partial<<<parts, 256, 0, s>>>(input, rop, dtype, total, base_offset, partials);
        hipError_t e1 = hipGetLastError();
        k_global_final<<<1, 256, 0, s>>>(partials, parts, output, p);
        hipError_t e2 = hipGetLastError();
        scratch_free(partials, s);
        PT_TRY(check_hip(e1, "global reduction (partials)"));
        PT_TRY(check_hip(e2, "global reduction (final)"));
        counters().global_reduce_calls++;
        return PT_OK;
    }
    if (axis >= 0 && contiguous && axis < ndims - 1) {
        size_t outer = 1, inner = 1;
        for (int d = 0; d < axis; d++) outer *= (size_t)shape[d];
        for (int d = axis + 1; d < ndims; d++) inner *= (size_t)shape[d];
        if (outer <= 65535 && count <= (size_t)INT32_MAX) {
            int st = launch_cols(dtype, rop, xb, outer, count, inner, output, out_dt, s);
            if (st >= 0) {
                PT_TRY((pt_status)st);
                counters().column_reduce_calls++;
                return PT_OK;
            }
        }
        const size_t col_blocks = (inner + 63) / 64;
        // too few workgroups for the GPU: split the reduced axis as well
        if (outer <= 65535 && col_blocks * outer < 1024 && count >= 256) {
            size_t splits = (2048 + col_blocks * outer - 1) / (col_blocks * outer);
            const size_t max_splits = (count + 63) / 64;  // at least 64 rows per slice
            if (splits > max_splits) splits = max_splits;
            if (splits > 65535) splits = 65535;
            const size_t slice = (count + splits - 1) / splits;
            GenAcc *partial = nullptr;
            PT_TRY(scratch_alloc((void **)&partial, sizeof(GenAcc) * outer * splits * inner, s));
            k_column_partial<<<dim3((unsigned)col_blocks, (unsigned)splits, (unsigned)outer), 256, 0, s>>>(
                xb, rop, dtype, count, inner, slice, partial);
            hipError_t e1 = hipGetLastError();
            k_column_final<<<(unsigned)((outer * inner + 255) / 256), 256, 0, s>>>(partial, outer, splits, inner,
                                                                                  output, p);
            hipError_t e2 = hipGetLastError();
            scratch_free(partial, s);
            PT_TRY(check_hip(e1, "column reduction (partials)"));
            PT_TRY(check_hip(e2, "column reduction (final)"));
            counters().column_reduce_calls++;
            return PT_OK;
        }
        if (outer <= 65535) {
            dim3 grid((unsigned)((inner + 63) / 64), (unsigned)outer);
            k_column_reduce<<<grid, 256, 0, s>>>(xb, output, rop, dtype,
                                                 outer, count, inner, p);
            PT_LAUNCH_CHECK("column reduction");
            counters().column_reduce_calls++;
            return PT_OK;
        }
    }
    if (outputs > 0x7fffffffu)
        return fail(PT_ERR_INVALID, "reduction: too many outputs");
    k_strided_reduce<<<(unsigned)outputs, 128, 0, s>>>(input, output, rop, dtype, p);
    PT_LAUNCH_CHECK("strided reduction");
    counters().strided_reduce_calls++;
    return PT_OK;
}

// ---------------------------------------------------- fused row launchers
// Register-resident row kernels: rows of up to 4 chunks per lane run one
// wave per row (4 rows per block); longer rows run one block of 4 waves per
// row (more waves in flight per CU, and rows up to 64 * VEC * 16 * 4
// elements stay in registers); beyond that the streaming kernels re-read.
template <int DT, typename OS>
static void launch_softmax_rows(const void *x, size_t rows, int n, size_t ld, OS *y, hipStream_t s)
{
    constexpr int V = RT<DT>::V;
    constexpr bool narrow = sizeof(typename RT<DT>::C) == 4;
    dim3 block(256), grid4((unsigned)((rows + 3) / 4)), grid1((unsigned)rows);
    bool vec = n % V == 0 && ld % V == 0 && aligned16(x) && aligned16(y);
    int chunks = (n + 64 * V - 1) / (64 * V);
    if constexpr (DT == PT_FLOAT32) {
        if (vec && chunks > 4 && chunks <= 16 && row_waves() == 8) {
            k_row_softmax<DT, V, 2, 8, OS><<<grid1, dim3(512), 0, s>>>(x, rows, n, ld, y);
            return;
        }
    }
    if (vec) {
        switch (chunks) {
        case 1: k_row_softmax<DT, V, 1, 1, OS><<<grid4, block, 0, s>>>(x, rows, n, ld, y); return;
        case 2: k_row_softmax<DT, V, 2, 1, OS><<<grid4, block, 0, s>>>(x, rows, n, ld, y); return;
        case 3: case 4: k_row_softmax<DT, V, 4, 1, OS><<<grid4, block, 0, s>>>(x, rows, n, ld, y); return;
        default:
            if (chunks <= 8) { k_row_softmax<DT, V, 2, 4, OS><<<grid1, block, 0, s>>>(x, rows, n, ld, y); return; }
            if (chunks <= 16) { k_row_softmax<DT, V, 4, 4, OS><<<grid1, block, 0, s>>>(x, rows, n, ld, y); return; }
            if (chunks <= 32) { k_row_softmax<DT, V, 8, 4, OS><<<grid1, block, 0, s>>>(x, rows, n, ld, y); return; }
            if constexpr (narrow) {
                if (chunks <= 64) { k_row_softmax<DT, V, 16, 4, OS><<<grid1, block, 0, s>>>(x, rows, n, ld, y); return; }
            }
            break;
        }
    }
    k_row_softmax_stream<DT, OS><<<(unsigned)rows, 256, 0, s>>>(x, n, ld, y);
}

// Grid of a row-walking kernel: two whole generations of the blocks that
// fit on the device at once.  A partial last generation leaves CUs idle
// while its blocks walk their rows: on config 2 the layerNorm walk took
// 44.3-44.4 us with 2048 blocks (768 resident) and 43.3-43.4 us with 768,
// 1536 or 3072.  The count is taken once per kernel, on the first device
// that launches it (every device of a host is the same model here).
template <auto K, int THREADS = 256>
static unsigned walk_grid(size_t rows)
{
    static const unsigned resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, K, THREADS, 0) != hipSuccess || per_cu < 1)
            per_cu = 1;
        (void)hipGetLastError();  // a failed query is not the launch's error
        return (unsigned)(per_cu * cus);
    }();
    const size_t b = 2 * (size_t)resident;
    return (unsigned)(rows < b ? rows : b);
}

template <int DT, typename CT>
static void launch_layernorm_rows(const void *x, size_t rows, int n, CT eps, const CT *g,
                                  const CT *b, CT *y, hipStream_t s)
{
    constexpr int V = RT<DT>::V;
    dim3 block(256), grid4((unsigned)((rows + 3) / 4)), grid1((unsigned)rows);
    bool vec = n % V == 0 && aligned16(x) && aligned16(y) && (!g || aligned16(g)) &&
               (!b || aligned16(b));
    int chunks = (n + 64 * V - 1) / (64 * V);
    if constexpr (DT == PT_FLOAT32 && sizeof(CT) == 4) {
        if (vec && chunks > 4 && chunks <= 16 && row_waves() == 8) {
            constexpr auto k = k_row_layernorm<DT, V, 2, 8, CT>;
            k<<<walk_grid<k, 512>(rows), dim3(512), 0, s>>>(x, rows, n, eps, g, b, y);
            return;
        }
    }
    if (vec) {
        switch (chunks) {
        case 1: k_row_layernorm<DT, V, 1, 1, CT><<<grid4, block, 0, s>>>(x, rows, n, eps, g, b, y); return;
        case 2: k_row_layernorm<DT, V, 2, 1, CT><<<grid4, block, 0, s>>>(x, rows, n, eps, g, b, y); return;
        case 3: case 4: k_row_layernorm<DT, V, 4, 1, CT><<<grid4, block, 0, s>>>(x, rows, n, eps, g, b, y); return;
        default:
            // block-per-row kernels walk the rows (walk_grid blocks)
            if (chunks <= 8) {
                constexpr auto k = k_row_layernorm<DT, V, 2, 4, CT>;
                k<<<walk_grid<k>(rows), block, 0, s>>>(x, rows, n, eps, g, b, y);
                return;
            }
            if (chunks <= 16) {
                constexpr auto k = k_row_layernorm<DT, V, 4, 4, CT>;
                k<<<walk_grid<k>(rows), block, 0, s>>>(x, rows, n, eps, g, b, y);
                return;
            }
            // (gamma and beta stay in registers too: 8 chunks per lane at most)
            if (chunks <= 32) {
                constexpr auto k = k_row_layernorm<DT, V, 8, 4, CT>;
                k<<<walk_grid<k>(rows), block, 0, s>>>(x, rows, n, eps, g, b, y);
                return;
            }
            break;
        }
    }
    k_row_layernorm_stream<DT, CT><<<(unsigned)rows, 256, 0, s>>>(x, n, eps, g, b, y);
}

// Strided -> contiguous permuted copy used to move the softmax axis last.
__global__ void k_permute_copy(const void *__restrict__ x, void *__restrict__ y, int esz,
                               GenParams p, size_t total)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    size_t rem = i, off = p.base;
    for (int d = p.ndims - 1; d >= 0; d--) {
        off += (rem % (size_t)p.shape[d]) * p.strides[d];
        rem /= (size_t)p.shape[d];
    }
    switch (esz) {
    case 1: ((uint8_t *)y)[i] = ((const uint8_t *)x)[off]; break;
    case 2: ((uint16_t *)y)[i] = ((const uint16_t *)x)[off]; break;
    case 4: ((uint32_t *)y)[i] = ((const uint32_t *)x)[off]; break;
    default: ((uint64_t *)y)[i] = ((const uint64_t *)x)[off]; break;
    }
}

static pt_status permute_copy(const void *x, void *y, int esz, const int *shape, const size_t *strides,
                              int ndims, hipStream_t s)
{
    GenParams p = {};
    p.ndims = ndims;
    for (int d = 0; d < ndims; d++) {
        p.shape[d] = shape[d];
        p.strides[d] = strides[d];
    }
    size_t total = numel(shape, ndims);
    if (!total) return PT_OK;
    k_permute_copy<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(x, y, esz, p, total);
    PT_LAUNCH_CHECK("permute copy");
    return PT_OK;
}

}  // namespace pt

using namespace pt;

extern "C" {

int pt_reduce_result_dtype(int dtype, int op)
{
    int rop = red_op_of(op);
    if (rop < 0 || !dtype_valid(dtype)) return -1;
    return result_dtype(dtype, rop);
}

pt_status pt_reduce(const void *input, void *output, int dtype, int op,
                    const int *shape, const size_t *strides, int ndims, int axis,
                    size_t base_offset, pt_stream_t stream)
{
    int rop = red_op_of(op);
    if (rop < 0 || rop == R_ARGMAX || rop == R_ARGMIN)
        return fail(PT_ERR_INVALID, "pt_reduce: unsupported op %d", op);
    return reduce_driver(input, output, dtype, rop, result_dtype(dtype, rop), shape, strides, ndims,
                         axis, base_offset, 0, 0, stream);
}

pt_status pt_reduce_noalloc(const void *input, void *output, int dtype, int op,
                            const int *shape, const size_t *strides, int ndims, int axis,
                            size_t base_offset, pt_stream_t stream)
{
    int rop = red_op_of(op);
    if (rop < 0 || rop == R_ARGMAX || rop == R_ARGMIN)
        return fail(PT_ERR_INVALID, "pt_reduce_noalloc: unsupported op %d", op);
    PT_TRY(ensure_init());
    hipStream_t s = stream_of(stream);
    PT_TRY(static_scratch_begin(s));
    pt_status st = reduce_driver(input, output, dtype, rop, result_dtype(dtype, rop), shape, strides, ndims,
                                 axis, base_offset, 0, 0, s);
    const pt_status end = static_scratch_end(s);
    return st != PT_OK ? st : end;
}

pt_status pt_arg_reduce(const void *input, int32_t *output, int dtype, int op,
                        const int *shape, const size_t *strides, int ndims, int axis,
                        size_t base_offset, pt_stream_t stream)
{
    int rop = red_op_of(op);
    if (rop != R_ARGMAX && rop != R_ARGMIN)
        return fail(PT_ERR_INVALID, "pt_arg_reduce: op %d is not argmax/argmin", op);
    return reduce_driver(input, output, dtype, rop, PT_INT32, shape, strides, ndims, axis,
                         base_offset, 0, 0, stream);
}

pt_status pt_moments(const void *input, void *output, int input_dtype, int result_dtype_,
                     const int *shape, const size_t *strides, int ndims, int axis,
                     int correction, int standard_deviation, pt_stream_t stream)
{
    int expect = result_dtype(input_dtype, R_VAR);
    if (result_dtype_ != expect)
        return fail(PT_ERR_INVALID, "pt_moments: result dtype must be %s",
                    expect == PT_FLOAT32 ? "float32" : "float64");
    return reduce_driver(input, output, input_dtype, R_VAR, expect, shape, strides, ndims, axis, 0,
                         correction, standard_deviation ? 1 : 0, stream);
}

pt_status pt_softmax(const void *input, void *output, int input_dtype, int output_dtype,
                     const int *shape, const size_t *strides, int ndims, int axis,
                     pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (ndims < 1 || ndims > PT_MAX_DIMS || axis < 0 || axis >= ndims)
        return fail(PT_ERR_INVALID, "Softmax axis is out of range for tensor rank %d", ndims);
    int expect = (input_dtype == PT_FLOAT32 || input_dtype == PT_FLOAT16 || input_dtype == PT_BFLOAT16)
                 ? PT_FLOAT32 : PT_FLOAT64;
    if (output_dtype != expect)
        return fail(PT_ERR_INVALID, "softmax output dtype must be %s", expect == PT_FLOAT32 ? "float32" : "float64");
    if (!dtype_is_floating(input_dtype))
        return fail(PT_ERR_UNSUPPORTED, "pt_softmax takes floating input; cast integers to float64 first");
    hipStream_t s = stream_of(stream);
    size_t total = numel(shape, ndims);
    int n = shape[axis];
    if (total == 0) {
        if (n == 0) {
            size_t others = 1;
            for (int d = 0; d < ndims; d++) if (d != axis) others *= (size_t)shape[d];
            if (others) return fail(PT_ERR_INVALID, "Min/max reduction has no identity for an empty axis");
        }
        return PT_OK;
    }
    // Move the axis last (contiguous) when the input is not already rows.
    size_t rows = 0, ld = 0;
    const void *src = input;
    void *tmp_in = nullptr;
    void *dst = output;
    void *tmp_out = nullptr;
    int perm_shape[PT_MAX_DIMS];
    size_t perm_strides[PT_MAX_DIMS];
    bool rowform = as_rows(shape, strides, ndims, axis, &rows, &ld) &&
                   (axis == ndims - 1 || rows == 1);
    // rows of the output must coincide with the contiguous output layout:
    // only true when the axis is the last one (or the tensor is one row).
    if (!rowform) {
        int k = 0;
        for (int d = 0; d < ndims; d++)
            if (d != axis) { perm_shape[k] = shape[d]; perm_strides[k] = strides[d]; k++; }
        perm_shape[k] = shape[axis];
        perm_strides[k] = strides[axis];
        size_t esz = dtype_size(input_dtype);
        PT_TRY(scratch_alloc(&tmp_in, total * esz, s));
        pt_status st = permute_copy(input, tmp_in, (int)esz, perm_shape, perm_strides, ndims, s);
        if (st != PT_OK) { scratch_free(tmp_in, s); return st; }
        src = tmp_in;
        rows = total / (size_t)n;
        ld = (size_t)n;
        if (axis != ndims - 1) {
            st = scratch_alloc(&tmp_out, total * dtype_size(output_dtype), s);
            if (st != PT_OK) { scratch_free(tmp_in, s); return st; }
            dst = tmp_out;
        }
    }
    if (n > 0) {
        switch (input_dtype) {
        case PT_FLOAT32: launch_softmax_rows<PT_FLOAT32, float>(src, rows, n, ld, (float *)dst, s); break;
        case PT_BFLOAT16: launch_softmax_rows<PT_BFLOAT16, float>(src, rows, n, ld, (float *)dst, s); break;
        case PT_FLOAT16: launch_softmax_rows<PT_FLOAT16, float>(src, rows, n, ld, (float *)dst, s); break;
        case PT_FLOAT64: launch_softmax_rows<PT_FLOAT64, double>(src, rows, n, ld, (double *)dst, s); break;
        }
    }
    hipError_t err = hipGetLastError();
    if (err == hipSuccess && tmp_out) {
        // scatter rows back: output[..., axis, ...] from the permuted buffer
        // the permuted buffer is contiguous over (others..., axis); build the
        // strides that read it in the output's order
        size_t pstr[PT_MAX_DIMS];
        size_t pacc = (size_t)n;
        pstr[axis] = 1;
        for (int d = ndims - 1; d >= 0; d--) {
            if (d == axis) continue;
            pstr[d] = pacc;
            pacc *= (size_t)shape[d];
        }
        pt_status st = permute_copy(tmp_out, output, (int)dtype_size(output_dtype), shape, pstr, ndims, s);
        if (st != PT_OK) err = hipErrorLaunchFailure;
    }
    scratch_free(tmp_in, s);
    scratch_free(tmp_out, s);
    PT_TRY(check_hip(err, "softmax"));
    counters().fused_row_calls++;
    return PT_OK;
}

pt_status pt_layernorm(const void *input, void *output, int input_dtype, int compute_dtype,
                       size_t rows, size_t n, double eps,
                       const void *gamma, const void *beta, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!(eps > 0.0) || !isfinite(eps))
        return fail(PT_ERR_INVALID, "LayerNorm epsilon must be finite and greater than zero");
    if (compute_dtype != PT_FLOAT32 && compute_dtype != PT_FLOAT64)
        return fail(PT_ERR_INVALID, "LayerNorm compute dtype must be float32 or float64");
    if (compute_dtype == PT_FLOAT32 && (!isfinite((float)eps) || (float)eps <= 0.0f))
        return fail(PT_ERR_INVALID, "LayerNorm epsilon is not representable as float32");
    if (n == 0 && rows) return fail(PT_ERR_INVALID, "LayerNorm cannot normalize an empty dimension");
    if (n > (size_t)INT32_MAX) return fail(PT_ERR_INVALID, "LayerNorm row too long");
    if (!rows) return PT_OK;
    hipStream_t s = stream_of(stream);
    int ni = (int)n;
    if (compute_dtype == PT_FLOAT32) {
        float e = (float)eps;
        const float *g = (const float *)gamma, *b = (const float *)beta;
        float *y = (float *)output;
        switch (input_dtype) {
        case PT_FLOAT32: launch_layernorm_rows<PT_FLOAT32, float>(input, rows, ni, e, g, b, y, s); break;
        case PT_BFLOAT16: launch_layernorm_rows<PT_BFLOAT16, float>(input, rows, ni, e, g, b, y, s); break;
        case PT_FLOAT16: launch_layernorm_rows<PT_FLOAT16, float>(input, rows, ni, e, g, b, y, s); break;
        default: return fail(PT_ERR_INVALID, "float32 layerNorm takes f32/f16/bf16 input");
        }
    } else {
        const double *g = (const double *)gamma, *b = (const double *)beta;
        double *y = (double *)output;
        switch (input_dtype) {
        case PT_FLOAT64: launch_layernorm_rows<PT_FLOAT64, double>(input, rows, ni, eps, g, b, y, s); break;
        case PT_FLOAT32: launch_layernorm_rows<PT_FLOAT32, double>(input, rows, ni, eps, g, b, y, s); break;
        default: return fail(PT_ERR_INVALID, "float64 layerNorm takes f64/f32 input");
        }
    }
    PT_LAUNCH_CHECK("layernorm");
    counters().fused_row_calls++;
    return PT_OK;
}

}  // extern "C"
