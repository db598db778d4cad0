// LDS-ring GEMM kernel for bf16 / fp16 on gfx950, 4 or 8 waves per 256-row
// tile (see the comment blocks below).  Launched by pt_matmul (pt_gemm.hip)
// through launch_gemm_ring.
#include "pt_gemm.h"

namespace pt {

// ------------------------------------------------ LDS-ring 16-bit kernel
// bf16 / fp16 GEMM for whole 256x256 tiles, K a multiple of BK * NST,
// k-contiguous A, B k- or n-contiguous.  Four waves in a 2 x 2 grid (the
// 8-wave form is described at the template), each
// owning a 128 x 128 sub-tile: 4 x 4 blocks of 32 x 32, i.e. 256 fp32
// accumulators per lane.  At one workgroup per CU a wave has its SIMD's
// whole register file, so the accumulators live in the accumulation
// registers and the fragments, addresses and staging in the others.  Per
// 16-wide k-slice a wave reads 8 fragments for 16 MFMAs (512 B of LDS per
// MFMA).
//
// K runs in steps of BK through a ring of NST LDS stages filled by
// global_load_lds (same swizzled layouts as k_gemm_direct).  Each step has
// one barrier, placed after the step's last fragment reads and before the
// next step's first:
//   * each wave first waits for its own loads of step k+1 only (vmcnt lets
//     the loads of steps k+2 .. k+NST-1 stay in flight), so after the
//     barrier step k+1's stage is complete for every wave;
//   * every wave has read all of step k's fragments, so step k's stage is
//     free and the loads of step k+NST go into it right after the barrier;
//   * the MFMAs of step k's last slice run after the barrier, over the LDS
//     latency of step k+1's first fragment reads.
// Loads thus have NST-1 steps to land.  Loads past the last step re-read
// the last K step (in bounds, never consumed), so every step waits for the
// same count.
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
template <int OFF>
__device__ __forceinline__ void lds_read_tr16(s16x4_t &dst, uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds_read_b64_tr_b16 offset");
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF));
}

// Two fp32 values rounded to the 16-bit dtype, packed low | high << 16.
// bf16: v_cvt_pk_bf16_f32 rounds to nearest even and quiets NaN exactly as
// float_to_bf16 does (checked bit for bit over every exponent / top-mantissa
// pattern with tie, NaN-payload and subnormal low halves).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi)
{
    if constexpr (DT == PT_BFLOAT16) {
        const f32x2_t v = {lo, hi};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    } else {
        return (uint32_t)float_to_f16(lo) | ((uint32_t)float_to_f16(hi) << 16);
    }
}

// Number of ring stages whose instruction offsets (stage * stage_bytes +
// the largest in-stage offset) fit the 16-bit LDS offset field.
constexpr int stages_per_base(int stage_bytes, int max_inner)
{
    int s = 0;
    while (s * stage_bytes + max_inner < 65536) s++;
    return s;
}

// BN: 256 (4 x 4 blocks per wave, one workgroup per CU) or 128 (4 x 2
// blocks per wave, WGS = 2 workgroups per CU, whose barriers and load
// waits then overlap each other's MFMAs).
// ILV 1: one fragment read (and, after the barrier, one load-to-LDS) between
// consecutive MFMAs instead of each group in one burst, so that a read
// waiting for the LDS queue never holds back the MFMAs behind it.
// ILV 2: as 1, and the loads of step k + NST - 1 are spread evenly over all
// of step k's MFMAs (into the stage freed by step k-1's barrier) rather
// than issued together after a barrier: four waves issuing their loads at
// once fill the CU's address queue, and in-order issue then holds every
// MFMA behind a load (needs NST >= 3 for the loads to land in time).
// NW: 4 waves (2 x 2, 128 x 128 each) or 8 waves (2 x 4, 128 x 64 each: two
// waves per SIMD with 128 accumulators apiece, so that one wave's MFMAs run
// while the other waits to issue a load or at a barrier; 6 fragment reads
// per 8 MFMAs instead of 8 per 16).
template <int DT, bool B_KC, int BK, int NST, int BN, int WGS, int ILV, int NW>
__global__ __launch_bounds__(64 * NW, WGS) void k_gemm_ring(GemmArgs g)
{
    using S = uint16_t;
    constexpr int WGN = NW / 2;            // wave grid: 2 x WGN
    constexpr int BM = 256, WTM = 128, WTN = BN / WGN, TM = 4, TN = WTN / 32;
    constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    constexpr int CPR = BK / 8;            // 16-byte chunks per k-contiguous row
    constexpr int RPI = 64 / CPR;          // such rows per load instruction (64 lanes x 16 B)
    constexpr int CPB = BN / 8;            // 16-byte chunks per k-row of row-major B
    constexpr int KPI = 64 / CPB;          // k-rows of row-major B per load instruction
    constexpr int NQA = A_ELEMS / 512 / NW; // load instructions per wave and step: A
    constexpr int NQB = B_ELEMS / 512 / NW; // ... and B
    constexpr int PER = NQA + NQB;         // vmcnt units per step
    constexpr int NS = BK / 16;            // MFMA k-slices per step
    constexpr int GROUP_M = 4;
    constexpr bool kGuard = (NST & (NST - 1)) != 0;
    static_assert(NS % 2 == 0 && NST >= 2 && NST <= 8 && (NST - 1) * PER < 64, "pipeline shape");
    static_assert(ILV != 2 || (NST >= 3 && (NS * TM * TN) % PER == 0), "spread loads need three stages");
    static_assert(NQA >= 1 && NQB >= 1 && (BN == 256 || BN == 128), "load split");
    static_assert((NW == 4 || NW == 8) && (TN == 2 || TN == 4), "wave grid");
    // All stages of an operand in one array.  Fragment reads are inline asm
    // from a per-lane base register plus an instruction offset (16 bits), so
    // the compiler neither sees them as LDS reads (it would make them wait
    // for every load-to-LDS in flight) nor waits for them: the waits are
    // explicit (frag_wait, ring_wait).  Stages beyond the offset field's
    // reach use a second base register.
    constexpr int SPA = stages_per_base(A_ELEMS * 2, (TM - 1) * 32 * BK * 2);
    constexpr int SPB = B_KC ? stages_per_base(B_ELEMS * 2, (TN - 1) * 32 * BK * 2)
                             : stages_per_base(B_ELEMS * 2, ((NS - 1) * 16 + 4) * BN * 2);
    static_assert(SPA >= 1 && SPB >= 1 && 2 * SPA >= NST && 2 * SPB >= NST, "two bases cover the ring");
    __shared__ __attribute__((aligned(1024))) S lds_a[NST * A_ELEMS];
    __shared__ __attribute__((aligned(1024))) S lds_b[NST * B_ELEMS];

    const int ntile = g.tiles_m * g.tiles_n;
    long long lin = blockIdx.x;
    if (g.remap) {
        long long total = (long long)ntile * g.batch;
        long long per = total / 8;
        lin = (lin % 8) * per + lin / 8;
    }
    const int bidx = (int)(lin / ntile);
    if (bidx >= g.batch) return;  // whole workgroup
    const int t = (int)(lin % ntile);
    const int group = t / (GROUP_M * g.tiles_n);
    const int first_m = group * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int tm = first_m + (t % (GROUP_M * g.tiles_n)) % gsz;
    const int tn = (t % (GROUP_M * g.tiles_n)) / gsz;
    const int m0 = tm * BM, n0 = tn * BN;
    long long oa, ob;
    batch_offsets(g, bidx, oa, ob);
    const S *A = (const S *)g.a + oa + (long long)m0 * g.a_sm;
    const S *B = (const S *)g.b + ob + (B_KC ? (long long)n0 * g.b_sn : (long long)n0);
    const long long lda = g.a_sm, ldb = B_KC ? g.b_sn : g.b_sk;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    // per-lane source offsets of each load instruction, without the k step
    long long offa[NQA], offb[NQB];
#pragma unroll
    for (int q4 = 0; q4 < NQA; q4++) {
        const int q = wave * NQA + q4;
        const int row = q * RPI + lane / CPR, pc = lane % CPR;
        offa[q4] = (long long)row * lda + (pc ^ swz_k(row, CPR)) * 8;
    }
#pragma unroll
    for (int q4 = 0; q4 < NQB; q4++) {
        const int q = wave * NQB + q4;
        if constexpr (B_KC) {
            const int row = q * RPI + lane / CPR, pc = lane % CPR;
            offb[q4] = (long long)row * ldb + (pc ^ swz_k(row, CPR)) * 8;
        } else {
            const int krow = q * KPI + lane / CPB, pcb = lane % CPB;
            offb[q4] = (long long)krow * ldb + (pcb ^ ((krow & 3) << 2)) * 8;
        }
    }
    const long long bstep = B_KC ? (long long)BK : (long long)BK * ldb;
    // one load instruction of step kt into stage ST: A for idx < NQA, else B
    auto issue_one = [&](int kt, auto ST, auto IDX) {
        constexpr int st = decltype(ST)::value % NST, idx = decltype(IDX)::value;
        if constexpr (idx < NQA) {
            __builtin_amdgcn_global_load_lds((const void *)(A + (long long)kt * BK + offa[idx]),
                                             (PT_LDS_AS void *)(lds_a + st * A_ELEMS + (wave * NQA + idx) * 512),
                                             16, 0, 0);
        } else {
            constexpr int q4 = idx - NQA;
            __builtin_amdgcn_global_load_lds((const void *)(B + (long long)kt * bstep + offb[q4]),
                                             (PT_LDS_AS void *)(lds_b + st * B_ELEMS + (wave * NQB + q4) * 512),
                                             16, 0, 0);
        }
    };
    auto issue = [&](int kt, auto ST) {
        constexpr int st = decltype(ST)::value % NST;
        const S *a = A + (long long)kt * BK;
        const S *b = B + (long long)kt * bstep;
#pragma unroll
        for (int q4 = 0; q4 < NQA; q4++)
            __builtin_amdgcn_global_load_lds((const void *)(a + offa[q4]),
                                             (PT_LDS_AS void *)(lds_a + st * A_ELEMS + (wave * NQA + q4) * 512),
                                             16, 0, 0);
#pragma unroll
        for (int q4 = 0; q4 < NQB; q4++)
            __builtin_amdgcn_global_load_lds((const void *)(b + offb[q4]),
                                             (PT_LDS_AS void *)(lds_b + st * B_ELEMS + (wave * NQB + q4) * 512),
                                             16, 0, 0);
    };

    // Read addresses.  k-contiguous operand (A, and B when B_KC), fragment
    // i of slice sl: row r = w*WT + i*32 + lane%32, 16-byte chunk
    // (2*sl + lane/32) ^ swz_k(r); swz_k does not depend on i, so one base
    // per slice serves every i (offset i * 32 rows).  Row-major B fragment
    // j: two transposing reads, k rows sl*16 + 8*(lane/32) + lane%16/4 (+4);
    // the swizzle of a k-row depends on k % 4 = lane%16/4 only, so one base
    // per j serves every slice (offset sl * 16 rows).  Index [h] of each
    // base: stages h*SP .. (h+1)*SP - 1.
    uint32_t abase[2][NS], kbase_b[2][NS], bbase[2][TN];
    {
        const uint32_t la = (uint32_t)(size_t)(PT_LDS_AS const S *)lds_a;
        const uint32_t lb = (uint32_t)(size_t)(PT_LDS_AS const S *)lds_b;
        const int ra = wm * WTM + (lane & 31), rb = wn * WTN + (lane & 31);
#pragma unroll
        for (int sl = 0; sl < NS; sl++) {
            const int kc = sl * 2 + (lane >> 5);
            abase[0][sl] = la + (uint32_t)(ra * BK + ((kc ^ swz_k(ra, CPR)) << 3)) * 2u;
            abase[1][sl] = abase[0][sl] + (uint32_t)(SPA * A_ELEMS * 2);
            kbase_b[0][sl] = lb + (uint32_t)(rb * BK + ((kc ^ swz_k(rb, CPR)) << 3)) * 2u;
            kbase_b[1][sl] = kbase_b[0][sl] + (uint32_t)(SPB * B_ELEMS * 2);
        }
        const int grp = lane >> 4, s = lane & 15;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = wn * WTN + j * 32 + (grp & 1) * 16 + 4 * (s & 3);
            const int kk = (grp >> 1) * 8 + (s >> 2);
            bbase[0][j] = lb + (uint32_t)(kk * BN + (((n >> 3) ^ ((kk & 3) << 2)) << 3) + (n & 7)) * 2u;
            bbase[1][j] = bbase[0][j] + (uint32_t)(SPB * B_ELEMS * 2);
        }
    }

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    using Frag = typename FragT<DT>::type;
    auto read_frags = [&](auto ST, auto SL, Frag (&fa)[TM], Frag (&fb)[TN]) {
        constexpr int st = decltype(ST)::value % NST, sl = decltype(SL)::value;
        constexpr int ha = st / SPA, sa = st % SPA, hb = st / SPB, sb = st % SPB;
        static_for<0, TM>([&](auto I) {
            constexpr int i = decltype(I)::value;
            lds_read_b128<(sa * A_ELEMS + i * 32 * BK) * 2>(fa[i], abase[ha][sl]);
        });
        static_for<0, TN>([&](auto J) {
            constexpr int j = decltype(J)::value;
            if constexpr (B_KC) {
                lds_read_b128<(sb * B_ELEMS + j * 32 * BK) * 2>(fb[j], kbase_b[hb][sl]);
            } else {
                s16x4_t h0, h1;
                lds_read_tr16<(sb * B_ELEMS + (sl * 16) * BN) * 2>(h0, bbase[hb][j]);
                lds_read_tr16<(sb * B_ELEMS + (sl * 16 + 4) * BN) * 2>(h1, bbase[hb][j]);
                fb[j] = __builtin_bit_cast(Frag, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        });
    };
    // fragment q of a slice: A fragment q for q < TM, else B fragment q - TM
    auto read_one = [&](auto ST, auto SL, auto Q, Frag (&fa)[TM], Frag (&fb)[TN]) {
        constexpr int st = decltype(ST)::value % NST, sl = decltype(SL)::value, q = decltype(Q)::value;
        constexpr int ha = st / SPA, sa = st % SPA, hb = st / SPB, sb = st % SPB;
        if constexpr (q < TM) {
            lds_read_b128<(sa * A_ELEMS + q * 32 * BK) * 2>(fa[q], abase[ha][sl]);
        } else if constexpr (B_KC) {
            constexpr int j = q - TM;
            lds_read_b128<(sb * B_ELEMS + j * 32 * BK) * 2>(fb[j], kbase_b[hb][sl]);
        } else {
            constexpr int j = q - TM;
            s16x4_t h0, h1;
            lds_read_tr16<(sb * B_ELEMS + (sl * 16) * BN) * 2>(h0, bbase[hb][j]);
            lds_read_tr16<(sb * B_ELEMS + (sl * 16 + 4) * BN) * 2>(h1, bbase[hb][j]);
            fb[j] = __builtin_bit_cast(Frag, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    auto mfma_one = [&](auto Q, const Frag (&fa)[TM], const Frag (&fb)[TN]) {
        constexpr int q = decltype(Q)::value, i = q / TN, j = q % TN;
        if constexpr (DT == PT_BFLOAT16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    };
    // every LDS read of the wave has returned before fa / fb are used
    auto frag_wait = [&](Frag (&fa)[TM], Frag (&fb)[TN]) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (TN == 4)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]),
                           "+v"(fb[0]), "+v"(fb[1]), "+v"(fb[2]), "+v"(fb[3])::"memory");
        else
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1])::"memory");
    };

    const int KT = g.K / BK;
    // the ring starts with steps 0 .. NST-1 (spread schedule: 0 .. NST-2,
    // step NST-1 follows during step 0); step 0 is needed first
    constexpr int PRO = ILV == 2 ? NST - 1 : NST;
    static_for<0, PRO>([&](auto P) { issue(min((int)decltype(P)::value, KT - 1), P); });
    ring_wait<(PRO - 1) * PER>();
    ring_barrier();
    // spread schedule: the load issued at MFMA q of slice sl of step kt
    constexpr int SPREAD = ILV == 2 ? NS * TM * TN / PER : 1;
    // loads issued after step kt+1's when step kt's barrier is reached: steps
    // kt+2 .. kt+NST-1 whole, or (spread) steps kt+2 .. kt+NST-2 whole plus the
    // loads of step kt+NST-1 placed in slices 0 .. NS-2 of step kt
    constexpr int WAIT_STEP = ILV == 2 ? (NST - 3) * PER + (NS - 1) * TM * TN / SPREAD : (NST - 2) * PER;
    auto spread_load = [&](int kt, auto J, auto SL, auto Q) {
        if constexpr (ILV == 2) {
            constexpr int slot = decltype(SL)::value * TM * TN + decltype(Q)::value;
            if constexpr (slot % SPREAD == 0)
                issue_one(min(kt + NST - 1, KT - 1), IC<decltype(J)::value + NST - 1>{}, IC<slot / SPREAD>{});
        }
    };
    Frag fa[2][TM], fb[2][TN];
    read_frags(IC<0>{}, IC<0>{}, fa[0], fb[0]);
    frag_wait(fa[0], fb[0]);
    for (int kt0 = 0; kt0 < KT; kt0 += NST) {
        static_for<0, NST>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const int kt = kt0 + j;
            // a power-of-two ring runs whole rounds (host check); other rings
            // skip the steps past the last one (uniform branch)
            if (kGuard ? kt < KT : true) {
                static_for<0, NS - 1>([&](auto SL) {
                    constexpr int sl = decltype(SL)::value, c = sl & 1, n = (sl + 1) & 1;
                    if constexpr (ILV) {
                        static_for<0, TM * TN>([&](auto Q) {
                            mfma_one(Q, fa[c], fb[c]);
                            if constexpr (decltype(Q)::value < TM + TN) read_one(J, IC<sl + 1>{}, Q, fa[n], fb[n]);
                            spread_load(kt, J, SL, Q);
                            __builtin_amdgcn_sched_barrier(0);
                        });
                    } else {
                        read_frags(J, IC<sl + 1>{}, fa[n], fb[n]);
                        __builtin_amdgcn_sched_barrier(0);  // reads first: they overlap the MFMAs
                        mfma_block<DT, TM, TN>(acc, fa[c], fb[c]);
                    }
                    frag_wait(fa[n], fb[n]);
                });
                ring_wait<WAIT_STEP>();  // this wave's loads of step kt+1 landed
                ring_barrier();                // ... everyone's; step kt's stage is free
                const int knext = min(kt + NST, KT - 1);
                if constexpr (ILV == 2) {
                    static_for<0, TM * TN>([&](auto Q) {
                        mfma_one(Q, fa[1], fb[1]);
                        if constexpr (decltype(Q)::value < TM + TN) read_one(IC<j + 1>{}, IC<0>{}, Q, fa[0], fb[0]);
                        spread_load(kt, J, IC<NS - 1>{}, Q);
                        __builtin_amdgcn_sched_barrier(0);
                    });
                } else if constexpr (ILV) {
                    constexpr int QN = TM * TN > PER ? TM * TN : PER;
                    static_for<0, QN>([&](auto Q) {
                        constexpr int q = decltype(Q)::value;
                        if constexpr (q < TM * TN) mfma_one(Q, fa[1], fb[1]);
                        if constexpr (q < TM + TN) read_one(IC<j + 1>{}, IC<0>{}, Q, fa[0], fb[0]);
                        if constexpr (q < PER) issue_one(knext, J, Q);
                        __builtin_amdgcn_sched_barrier(0);
                    });
                } else {
                    read_frags(IC<j + 1>{}, IC<0>{}, fa[0], fb[0]);
                    __builtin_amdgcn_sched_barrier(0);
                    issue(knext, J);
                    mfma_block<DT, TM, TN>(acc, fa[1], fb[1]);
                }
                frag_wait(fa[0], fb[0]);
            }
        });
    }
    ring_wait<0>();  // no load may still target LDS when the workgroup ends

    // ---- epilogue: in a 32x32 block lane l holds column l%32 and rows
    // 8*(e/4) + 4*(l/32) + e%4.  Lane pairs (l, l^1) swap halves so that
    // each lane stores two adjacent columns of two rows as 4-byte words:
    // the even lane rows r, r+1, the odd lane rows r+2, r+3.
    S *Cb = (S *)g.c + (size_t)bidx * (size_t)g.M * (size_t)g.N;
    const bool odd = lane & 1;
    const int col_l = (lane & 31) & ~1;
    const int row_l = (lane >> 5) * 4 + (odd ? 2 : 0);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * WTN + j * 32 + col_l;
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++) {
                const uint32_t p01 = pack2<DT>(acc[i][j][4 * e4 + 0], acc[i][j][4 * e4 + 1]);
                const uint32_t p23 = pack2<DT>(acc[i][j][4 * e4 + 2], acc[i][j][4 * e4 + 3]);
                const uint32_t send = odd ? p01 : p23;
                const uint32_t recv = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send, 0xB1, 0xF, 0xF, false);
                const uint32_t x = odd ? recv : p01, y = odd ? p23 : recv;
                const uint32_t w0 = (x & 0xffffu) | (y << 16);
                const uint32_t w1 = (x >> 16) | (y & 0xffff0000u);
                const int m = m0 + wm * WTM + i * 32 + e4 * 8 + row_l;
                *(uint32_t *)(Cb + (size_t)m * g.N + n) = w0;
                *(uint32_t *)(Cb + (size_t)(m + 1) * g.N + n) = w1;
            }
        }
}

// Ring shapes: {BK, stages, BN, workgroups per CU, schedule, waves}
static const int kRing[][6] = {{32, 4, 256, 1, 0, 4}, {64, 2, 256, 1, 0, 4}, {32, 2, 256, 1, 0, 4},
                               {32, 3, 256, 1, 0, 4}, {32, 5, 256, 1, 0, 4}, {32, 3, 128, 2, 0, 4},
                               {32, 2, 128, 2, 0, 4}, {64, 2, 256, 1, 1, 4}, {32, 4, 256, 1, 1, 4},
                               {32, 3, 128, 2, 1, 4}, {32, 4, 256, 1, 2, 4}, {32, 3, 256, 1, 2, 4},
                               {32, 5, 256, 1, 2, 4}, {32, 4, 256, 1, 1, 8}, {64, 2, 256, 1, 1, 8},
                               {32, 4, 256, 1, 2, 8}, {32, 5, 256, 1, 2, 8}, {32, 3, 256, 1, 2, 8}};

int gemm_ring_variants() { return (int)(sizeof(kRing) / sizeof(kRing[0])); }
int gemm_ring_bn(int variant) { return kRing[variant][2]; }
int gemm_ring_bk(int variant) { return kRing[variant][0]; }
// K must be a multiple of this: BK x stages for power-of-two rings, BK otherwise
int gemm_ring_kmul(int variant)
{
    const int st = kRing[variant][1];
    return (st & (st - 1)) ? kRing[variant][0] : kRing[variant][0] * st;
}

void launch_gemm_ring(const GemmArgs &g, int dtype, bool b_row, int variant, dim3 grid, hipStream_t s)
{
    const dim3 block(64 * kRing[variant][5]);
#define PT_RING(DTV, BKV, STV, BNV, WGV, ILVV, NWV)                                                    \
    do {                                                                                               \
        if (b_row) k_gemm_ring<DTV, false, BKV, STV, BNV, WGV, ILVV, NWV><<<grid, block, 0, s>>>(g);   \
        else k_gemm_ring<DTV, true, BKV, STV, BNV, WGV, ILVV, NWV><<<grid, block, 0, s>>>(g);          \
    } while (0)
#define PT_RING_DT(DTV)                                                                        \
    do {                                                                                       \
        switch (variant) {                                                                     \
        case 0: PT_RING(DTV, 32, 4, 256, 1, 0, 4); break;                                      \
        case 1: PT_RING(DTV, 64, 2, 256, 1, 0, 4); break;                                      \
        case 2: PT_RING(DTV, 32, 2, 256, 1, 0, 4); break;                                      \
        case 3: PT_RING(DTV, 32, 3, 256, 1, 0, 4); break;                                      \
        case 4: PT_RING(DTV, 32, 5, 256, 1, 0, 4); break;                                      \
        case 5: PT_RING(DTV, 32, 3, 128, 2, 0, 4); break;                                      \
        case 6: PT_RING(DTV, 32, 2, 128, 2, 0, 4); break;                                      \
        case 7: PT_RING(DTV, 64, 2, 256, 1, 1, 4); break;                                      \
        case 8: PT_RING(DTV, 32, 4, 256, 1, 1, 4); break;                                      \
        case 9: PT_RING(DTV, 32, 3, 128, 2, 1, 4); break;                                      \
        case 10: PT_RING(DTV, 32, 4, 256, 1, 2, 4); break;                                     \
        case 11: PT_RING(DTV, 32, 3, 256, 1, 2, 4); break;                                     \
        case 12: PT_RING(DTV, 32, 5, 256, 1, 2, 4); break;                                     \
        case 13: PT_RING(DTV, 32, 4, 256, 1, 1, 8); break;                                     \
        case 14: PT_RING(DTV, 64, 2, 256, 1, 1, 8); break;                                     \
        case 15: PT_RING(DTV, 32, 4, 256, 1, 2, 8); break;                                     \
        case 16: PT_RING(DTV, 32, 5, 256, 1, 2, 8); break;                                     \
        default: PT_RING(DTV, 32, 3, 256, 1, 2, 8); break;                                      \
        }                                                                                      \
    } while (0)
    if (dtype == PT_BFLOAT16) PT_RING_DT(PT_BFLOAT16);
    else PT_RING_DT(PT_FLOAT16);
#undef PT_RING_DT
#undef PT_RING
}

} // namespace pt
