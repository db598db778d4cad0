// Internal header of the GEMM kernels (pt_gemm.hip, pt_gemm_ring.hip,
// pt_gemm_f32ring.hip, pt_gemm_smalln.hip):
// argument block, element traits, MFMA fragment types and helpers shared by
// the kernels.  Not part of the public boundary (include/pt_hip.h is).
#pragma once

#include "pt_common.h"

namespace pt {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define GEMM_MAX_BATCH_DIMS 8

struct GemmArgs {
    const void *a;
    const void *b;
    void *c;
    int M, N, K;
    long long a_sm, a_sk;  // A(m,k) = a[m * a_sm + k * a_sk]
    long long b_sk, b_sn;  // B(k,n) = b[k * b_sk + n * b_sn]
    int tiles_m, tiles_n;
    int batch;
    int nbd;               // batch dims
    int bshape[GEMM_MAX_BATCH_DIMS];
    long long bsa[GEMM_MAX_BATCH_DIMS];
    long long bsb[GEMM_MAX_BATCH_DIMS];
    int remap;             // total tiles divisible by 8: XCD remap on
    int vec_a, vec_b;      // 16-byte aligned packs: the checked kernel loads in-range packs whole
    int ksplit, k_chunk;   // split-K: blockIdx.y = K chunk of k_chunk (a multiple of BK)
    float *partial;        // split-K fp32 partials [ksplit][batch][M][N]
};

// Element traits: storage type and elements per 16-byte pack.
template <int DT> struct GE;
template <> struct GE<PT_BFLOAT16> { using S = uint16_t; static constexpr int PK = 8; };
template <> struct GE<PT_FLOAT16> { using S = uint16_t; static constexpr int PK = 8; };
template <> struct GE<PT_FLOAT32> { using S = float; static constexpr int PK = 4; };

template <int DT>
__device__ __forceinline__ void store_c(void *c, size_t idx, float v)
{
    if constexpr (DT == PT_FLOAT32) ((float *)c)[idx] = v;
    else if constexpr (DT == PT_BFLOAT16) ((uint16_t *)c)[idx] = float_to_bf16(v);
    else ((uint16_t *)c)[idx] = float_to_f16(v);
}

template <int DT> struct FragT;
template <> struct FragT<PT_BFLOAT16> { using type = bf16x8_t; };
template <> struct FragT<PT_FLOAT16> { using type = f16x8_t; };
template <> struct FragT<PT_FLOAT32> { using type = floatx4; };

// acc[i][j] += A-fragment i x B-fragment j for one k-slice.
template <int DT, int TM, int TN>
__device__ __forceinline__ void mfma_block(floatx16 (&acc)[TM][TN],
                                           const typename FragT<DT>::type (&fa)[TM],
                                           const typename FragT<DT>::type (&fb)[TN])
{
    if constexpr (DT == PT_FLOAT32) {
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][e], fb[j][e], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (DT == PT_BFLOAT16)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
            }
    }
}

__device__ __forceinline__ void batch_offsets(const GemmArgs &g, int b, long long &oa, long long &ob)
{
    oa = 0;
    ob = 0;
    for (int d = g.nbd - 1; d >= 0; d--) {
        int c = b % g.bshape[d];
        b /= g.bshape[d];
        oa += (long long)c * g.bsa[d];
        ob += (long long)c * g.bsb[d];
    }
}

#define PT_LDS_AS __attribute__((address_space(3)))
typedef short s16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int swz_k(int row, int cpr)
{
    return cpr == 8 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

// ---- helpers of the LDS-ring kernels (pt_gemm_ring.hip, pt_gemm_f32ring.hip)
template <int I> struct IC { static constexpr int value = I; };
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (B < E) {
        f(IC<B>{});
        static_for<B + 1, E>(f);
    }
}

// Wait until at most VM vector-memory operations of this wave are in
// flight and all of its LDS reads have returned (gfx9 s_waitcnt fields:
// vmcnt[3:0] bits 3:0, expcnt 6:4, lgkmcnt 11:8, vmcnt[5:4] 15:14).
template <int VM>
__device__ __forceinline__ void ring_wait()
{
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (0 << 8) | ((VM >> 4) << 14));
}

// Workgroup barrier without the memory-model fence of __syncthreads (which
// would wait for every load in flight); the waits that make LDS data
// visible are the explicit ring_wait before it.
__device__ __forceinline__ void ring_barrier()
{
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// LDS reads issued as inline asm (instruction offset OFF bytes).
template <int OFF, typename T>
__device__ __forceinline__ void lds_read_b128(T &dst, uint32_t addr)
{
    static_assert(sizeof(T) == 16 && OFF >= 0 && OFF < 65536, "ds_read_b128 operand");
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF));
}
// One load of 16 bytes per lane into LDS: the wave-uniform base address in
// a scalar raw-buffer resource (stride 0), the lane's byte offset in a
// register, the LDS destination (wave-uniform) in M0.  Unlike
// global_load_lds with a per-lane 64-bit address, a load then needs no
// vector instruction of its own.  `range`: bytes from `base` that may be
// read; the buffer unit returns zeros for a lane's bytes past it instead of
// reading them.
__device__ __forceinline__ void buffer_load_lds16(const void *base, uint32_t lane_off, PT_LDS_AS void *lds,
                                                  uint32_t range = 0xffffffffu)
{
    constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)range, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, lane_off, 0, 0, 0);
}

typedef float f32x2v_t __attribute__((ext_vector_type(2)));
template <int OFF>
__device__ __forceinline__ void lds_read_b64(f32x2v_t &dst, uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds_read_b64 offset");
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF));
}
template <int OFF>
__device__ __forceinline__ void lds_read_tr16(s16x4_t &dst, uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds_read_b64_tr_b16 offset");
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF));
}

// LDS-ring kernels for 16-bit operands (pt_gemm_ring.hip).  A variant is a
// (K step, stages, tile width, workgroups per CU, schedule, waves, kind)
// shape; every variant needs M % 256 == 0, N % tile width == 0 and K a
// multiple of gemm_ring_kmul.
// b_row: B is n-contiguous (else k-contiguous).
int gemm_ring_variants();
int gemm_ring_kind(int variant);  // 0 k_gemm_ring, 1 k_gemm_pp, 2 k_gemm_wl
int gemm_ring_bn(int variant);
int gemm_ring_bk(int variant);
int gemm_ring_kmul(int variant);
void launch_gemm_ring(const GemmArgs &g, int dtype, bool b_row, int variant, dim3 grid, hipStream_t s);

// fp32 LDS-ring kernel for 128x128 tiles (pt_gemm_f32ring.hip); a_kc / b_kc:
// the operand's K index is its contiguous one (else M / N is).  stages: 4
// (128 KiB of LDS, one workgroup per CU) or 2 (64 KiB, two per CU).
bool gemm_f32r_eligible(const GemmArgs &g, bool a_kc, bool b_kc);
void launch_gemm_f32r(const GemmArgs &g, bool a_kc, bool b_kc, int stages, hipStream_t s);

// fp32 products with N <= 16 and k-contiguous A (pt_gemm_smalln.hip).
bool gemm_smalln_eligible(const GemmArgs &g);
void launch_gemm_smalln(const GemmArgs &g, hipStream_t s);

}  // namespace pt
