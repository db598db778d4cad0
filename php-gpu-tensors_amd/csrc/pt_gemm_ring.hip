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
// Two fp32 values rounded to the 16-bit dtype, packed low | high << 16.
// bf16: v_cvt_pk_bf16_f32 rounds to nearest even and quiets NaN exactly as
// float_to_bf16 does (checked bit for bit over every exponent / top-mantissa
// pattern with tie, NaN-payload and subnormal low halves).
// fp16: v_cvt_pk_f16_f32 gives v_cvt_f16_f32's result for every fp32 bit
// pattern but NaN (checked over all 2^32); a pair holding a NaN, which only
// a NaN or infinite operand produces, takes float_to_f16's payload rule
// off the common path.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi)
{
    const f32x2_t v = {lo, hi};
    if constexpr (DT == PT_BFLOAT16) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    } else {
        uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
        if (__builtin_expect(__builtin_isnan(lo) || __builtin_isnan(hi), 0))
            h = (uint32_t)float_to_f16(lo) | ((uint32_t)float_to_f16(hi) << 16);
        return h;
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

// ------------------------------------------------ ping-pong 16-bit kernel
// 256 x 256 tiles, 8 waves, the LDS ring and load layouts of k_gemm_ring
// (BK 32).  Wave w owns rows 128 * (w / 4) .. +127 and columns
// 64 * (w % 4) .. +63 (4 x 2 blocks of 32 x 32).  Waves are placed on the
// SIMDs round-robin, so waves 0-3 (group 0) and 4-7 (group 1) put one wave
// of each group on every SIMD.  The groups run half a K step apart and
// alternate two phases, each closed by a workgroup barrier:
//   memory phase of step t: read all of step t's fragments (both slices)
//     into registers, issue this wave's share of the loads of step
//     t + NST - 1 into the stage step t - 1 used, then wait for the
//     fragments and for this wave's own loads of step t + 1;
//   compute phase of step t: the step's 16 MFMAs back to back (at raised
//     wave priority when PRIO is set).
// While one group computes, the other runs its memory phase, so each SIMD's
// matrix core is fed by one wave whose instruction stream holds nothing but
// MFMAs, and the load-issue stalls of the address unit fall on the other.
// Global phase p: group 0 runs memory(p / 2) for even p, compute((p-1) / 2)
// for odd p; group 1 runs compute(p / 2 - 1) for even p, memory((p-1) / 2)
// for odd p.  Hence:
//   * step t's stage is complete at phase 2t: every wave waited for its own
//     loads of step t at the end of its memory phase of step t - 1 (phase
//     2t - 2 or 2t - 1), before a barrier that precedes phase 2t;
//   * step t - 1's stage is free at phase 2t: its last reader is group 1's
//     memory phase of step t - 1 (phase 2t - 1), which ends with its LDS
//     reads returned, before the barrier;
//   * group 1 passes one extra barrier before its first phase and skips the
//     one after its last compute phase, so both groups pass 2 KT + 1.
// A load issued at phase 2t is awaited at the end of phase 2(t + NST - 2)
// or one later: 2 (NST - 2) phases of latency.
template <int DT, bool B_KC, int NST, bool PRIO>
__global__ __launch_bounds__(512, 1) void k_gemm_pp(GemmArgs g)
{
    using S = uint16_t;
    constexpr int NW = 8, WGN = 4, BK = 32, BN = 256;
    constexpr int BM = 256, WTM = 128, WTN = 64, TM = 4, TN = 2;
    constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    constexpr int CPR = BK / 8, RPI = 64 / CPR, CPB = BN / 8, KPI = 64 / CPB;
    constexpr int NQA = A_ELEMS / 512 / NW, NQB = B_ELEMS / 512 / NW, PER = NQA + NQB;
    constexpr int NS = BK / 16;
    constexpr int NR = NS * (TM + TN);     // fragment reads per memory phase
    constexpr int GROUP_M = 4;
    constexpr bool kGuard = (NST & (NST - 1)) != 0;
    static_assert(NST >= 3 && NST <= 5 && NR % PER == 0, "pipeline shape");
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

    const int lane = threadIdx.x & 63;
    // wave index in a scalar register: the group branches below are uniform
    // branches, so every barrier is passed by whole waves
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wm = wave / WGN, wn = wave % WGN;  // wm is the wave's group

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

    // fragment read addresses (as in k_gemm_ring)
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
    Frag fa[NS][TM], fb[NS][TN];
    // fragment r of the step at stage ST: slice r / (TM + TN), then A
    // fragments before B fragments
    auto read_one = [&](auto ST, auto R) {
        constexpr int st = decltype(ST)::value % NST, r = decltype(R)::value;
        constexpr int sl = r / (TM + TN), q = r % (TM + TN);
        constexpr int ha = st / SPA, sa = st % SPA, hb = st / SPB, sb = st % SPB;
        if constexpr (q < TM) {
            lds_read_b128<(sa * A_ELEMS + q * 32 * BK) * 2>(fa[sl][q], abase[ha][sl]);
        } else if constexpr (B_KC) {
            constexpr int j = q - TM;
            lds_read_b128<(sb * B_ELEMS + j * 32 * BK) * 2>(fb[sl][j], kbase_b[hb][sl]);
        } else {
            constexpr int j = q - TM;
            s16x4_t h0, h1;
            lds_read_tr16<(sb * B_ELEMS + (sl * 16) * BN) * 2>(h0, bbase[hb][j]);
            lds_read_tr16<(sb * B_ELEMS + (sl * 16 + 4) * BN) * 2>(h1, bbase[hb][j]);
            fb[sl][j] = __builtin_bit_cast(Frag, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    // every LDS read of the wave has returned before a fragment is used
    auto frag_wait = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        static_assert(NS == 2 && TM == 4 && TN == 2, "fragment set");
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(fa[0][0]), "+v"(fa[0][1]), "+v"(fa[0][2]), "+v"(fa[0][3]), "+v"(fb[0][0]),
                       "+v"(fb[0][1]), "+v"(fa[1][0]), "+v"(fa[1][1]), "+v"(fa[1][2]), "+v"(fa[1][3]),
                       "+v"(fb[1][0]), "+v"(fb[1][1])::"memory");
    };
    const int KT = g.K / BK;
    // memory phase of step kt (stage J): the loads of step kt + NST - 1 go
    // one per NR / PER fragment reads
    auto memory_phase = [&](int kt, auto J) {
        constexpr int j = decltype(J)::value;
        const int kl = min(kt + NST - 1, KT - 1);
        static_for<0, NR>([&](auto R) {
            constexpr int r = decltype(R)::value;
            read_one(J, R);
            if constexpr (r % (NR / PER) == 0) issue_one(kl, IC<j + NST - 1>{}, IC<r / (NR / PER)>{});
        });
        frag_wait();
        ring_wait<(NST - 2) * PER>();  // this wave's loads of step kt + 1 landed
        ring_barrier();
    };
    auto compute_phase = [&]() {
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
        static_for<0, NS>([&](auto SL) {
            constexpr int sl = decltype(SL)::value;
            static_for<0, TM * TN>([&](auto Q) {
                constexpr int q = decltype(Q)::value, i = q / TN, jj = q % TN;
                if constexpr (DT == PT_BFLOAT16)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[sl][i], fb[sl][jj], acc[i][jj], 0, 0, 0);
                else
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[sl][i], fb[sl][jj], acc[i][jj], 0, 0, 0);
            });
        });
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    };

    // prologue: steps 0 .. NST-2 in flight, step 0 landed for everyone
    static_for<0, NST - 1>([&](auto P) {
        constexpr int p = decltype(P)::value;
        const int kt = min(p, KT - 1);
        static_for<0, PER>([&](auto Q) { issue_one(kt, P, Q); });
    });
    ring_wait<(NST - 2) * PER>();
    ring_barrier();
    if (wm == 1) ring_barrier();  // group 1 starts half a step later
    for (int kt0 = 0; kt0 < KT; kt0 += NST) {
        static_for<0, NST>([&](auto J) {
            const int kt = kt0 + decltype(J)::value;
            // a power-of-two ring runs whole rounds (host check); other rings
            // skip the steps past the last one (uniform branch)
            if (kGuard ? kt < KT : true) {
                memory_phase(kt, J);
                compute_phase();
                if (wm == 0 || kt + 1 < KT) ring_barrier();
            }
        });
    }
    ring_wait<0>();  // no load may still target LDS when the workgroup ends

    // epilogue (the layout of k_gemm_ring's)
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

// ------------------------------------------------ whole-line 16-bit kernel
// The 8-wave k_gemm_ring (2 x 4 waves of 128 x 64, K steps of 32, one
// barrier per step, loads spread one per four MFMAs) with A staged in whole
// 128-byte lines.  With 32-k steps a k-contiguous A row contributes 64 bytes
// per step, half a cache line, and the L2 -> CU request path, not the matrix
// cores, bounds the kernel: the GEMM's load stream alone (no MFMAs) ran at
// 12.3 TB/s over the device with half-line A rows and at 15.1 TB/s with
// whole lines.
//   * A lives in NSA = 3 superstages of 64 k (256 rows x 128 B = 32 KiB),
//     B in NSB = 4 stages of 32 k (16 KiB): 160 KiB of LDS.
//   * Issue step u (during K step u) loads A rows 128 * (u % 2) .. +127 of
//     superstage (u + 4) / 2 and B of step u + 3.  Superstage S is read by
//     steps 2S and 2S + 1 and its slot is free after step 2S - 5's barrier
//     (the last reader of superstage S - 3), so both halves have at least
//     three steps to land.
//   * A superstage row keeps its eight 16-byte chunks XOR-swizzled by
//     (row / 2) % 8, so a fragment read of 32 rows x 16 bytes hits every
//     LDS bank once.  The load-to-LDS DMA writes a lane's 16 bytes at lane
//     position, so lane L of an A load fetches the chunk that belongs at
//     position L % 8 of its row.
//   * The step loop is unrolled over 12 steps, the period of the two rings
//     (superstage slot (t / 2) % 3, B stage t % 4), so every LDS offset is
//     an instruction immediate.  K must be a multiple of 64.
// At the barrier of step t a wave has issued all loads of issue step t - 1
// and the two A loads of issue step t that precede it (B's two follow it):
// at most 6 may be in flight, and every load of issue step t - 2 or earlier
// (B of step t + 1, both halves of superstage (t + 1) / 2) has landed.
template <int DT, bool B_KC>
__global__ __launch_bounds__(512, 1) void k_gemm_wl(GemmArgs g)
{
    using S = uint16_t;
    constexpr int NW = 8, WGN = 4, BK = 32, BN = 256, BM = 256, WTM = 128, WTN = 64, TM = 4, TN = 2;
    constexpr int NSA = 3, NSB = 4, PERIOD = 12;
    constexpr int SA_ELEMS = BM * 2 * BK;  // superstage: 256 rows x 64 k
    constexpr int B_ELEMS = BN * BK;
    constexpr int CPR = BK / 8, RPI = 64 / CPR, CPB = BN / 8, KPI = 64 / CPB;
    constexpr int NQA = 2;                 // A loads per wave and step (128 rows x 128 B / 8 waves / 1 KiB)
    constexpr int NQB = B_ELEMS / 512 / NW;
    constexpr int PER = NQA + NQB;
    constexpr int NS = BK / 16;
    constexpr int GROUP_M = 4;
    constexpr int SPREAD = NS * TM * TN / PER;
    constexpr int WAIT_STEP = PER + (NS - 1) * TM * TN / SPREAD;
    static_assert(NS == 2 && NQB == 2 && SPREAD == 4 && NQA * SPREAD == TM * TN, "load spread");
    constexpr int SPA = stages_per_base(SA_ELEMS * 2, (TM - 1) * 32 * 2 * BK * 2);
    constexpr int SPB = B_KC ? stages_per_base(B_ELEMS * 2, (TN - 1) * 32 * BK * 2)
                             : stages_per_base(B_ELEMS * 2, ((NS - 1) * 16 + 4) * BN * 2);
    static_assert(2 * SPA >= NSA && 2 * SPB >= NSB, "two bases cover the rings");
    __shared__ __attribute__((aligned(1024))) S lds_a[NSA * SA_ELEMS];
    __shared__ __attribute__((aligned(1024))) S lds_b[NSB * B_ELEMS];

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

    const int lane = threadIdx.x & 63;
    // the wave index as a uniform value (the loads' LDS destinations are
    // scalar arithmetic)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    // A load (half h, instruction q4 of the wave): rows h*128 + 8q .. +7,
    // lane L at row 8q + L/8, LDS position L % 8 holding chunk (L%8) ^ swizzle.
    // Offsets are the lane's bytes from the step's base (the host keeps the
    // pitches below 2^22 elements, so they fit 32 bits): each load is one
    // buffer load to LDS with a scalar base.
    uint32_t offa[2][NQA], offb[NQB];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int q4 = 0; q4 < NQA; q4++) {
            const int q = wave * NQA + q4;
            const int row = h * 128 + q * 8 + lane / 8, p = lane % 8;
            offa[h][q4] = (uint32_t)(((long long)row * lda + ((p ^ swz_k(row, 8)) << 3)) * 2);
        }
#pragma unroll
    for (int q4 = 0; q4 < NQB; q4++) {
        const int q = wave * NQB + q4;
        if constexpr (B_KC) {
            const int row = q * RPI + lane / CPR, pc = lane % CPR;
            offb[q4] = (uint32_t)(((long long)row * ldb + (pc ^ swz_k(row, CPR)) * 8) * 2);
        } else {
            const int krow = q * KPI + lane / CPB, pcb = lane % CPB;
            offb[q4] = (uint32_t)(((long long)krow * ldb + (pcb ^ ((krow & 3) << 2)) * 8) * 2);
        }
    }
    const long long bstep = B_KC ? (long long)BK : (long long)BK * ldb;
    const int KT = g.K / BK, KS = KT / 2;
    // load IDX of issue step u, whose position in the period is J (u = J mod
    // 12; the prologue's u = -4 .. -1 are positions 8 .. 11).  Loads past
    // the end re-read the last superstage / step, in bounds and never used.
    auto issue_one = [&](int u, auto J, auto IDX) {
        constexpr int j = decltype(J)::value, idx = decltype(IDX)::value;
        if constexpr (idx < NQA) {
            constexpr int h = j & 1, slot = ((j + 4) >> 1) % NSA;
            const int s = min((u + 4) >> 1, KS - 1);
            buffer_load_lds16(A + (long long)s * 2 * BK, offa[h][idx],
                              (PT_LDS_AS void *)(lds_a + slot * SA_ELEMS + (h * 128 + (wave * NQA + idx) * 8) * 2 * BK));
        } else {
            constexpr int q4 = idx - NQA, slot = (j + 3) % NSB;
            const int kb = min(u + 3, KT - 1);
            buffer_load_lds16(B + (long long)kb * bstep, offb[q4],
                              (PT_LDS_AS void *)(lds_b + slot * B_ELEMS + (wave * NQB + q4) * 512));
        }
    };

    // fragment read bases.  A: [base][parity of the step][slice]: row
    // ra = wm*128 + lane%32 (+32 i by offset), chunk
    // (4 * parity + 2 * slice + lane/32) ^ swizzle(ra), which does not
    // depend on i.  B as in k_gemm_ring.
    uint32_t abase[2][2][NS], kbase_b[2][NS], bbase[2][TN];
    {
        const uint32_t la = (uint32_t)(size_t)(PT_LDS_AS const S *)lds_a;
        const uint32_t lb = (uint32_t)(size_t)(PT_LDS_AS const S *)lds_b;
        const int ra = wm * WTM + (lane & 31), rb = wn * WTN + (lane & 31);
#pragma unroll
        for (int p = 0; p < 2; p++)
#pragma unroll
            for (int sl = 0; sl < NS; sl++) {
                const int kc = p * 4 + sl * 2 + (lane >> 5);
                abase[0][p][sl] = la + (uint32_t)(ra * 2 * BK + ((kc ^ swz_k(ra, 8)) << 3)) * 2u;
                abase[1][p][sl] = abase[0][p][sl] + (uint32_t)(SPA * SA_ELEMS * 2);
            }
#pragma unroll
        for (int sl = 0; sl < NS; sl++) {
            const int kc = sl * 2 + (lane >> 5);
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
    // fragment q of slice SL of the step at period position J
    auto read_one = [&](auto J, auto SL, auto Q, Frag (&fa)[TM], Frag (&fb)[TN]) {
        constexpr int j = decltype(J)::value % PERIOD, sl = decltype(SL)::value, q = decltype(Q)::value;
        constexpr int slot = (j >> 1) % NSA, par = j & 1, ha = slot / SPA, sa = slot % SPA;
        constexpr int stb = j % NSB, hb = stb / SPB, sb = stb % SPB;
        if constexpr (q < TM) {
            lds_read_b128<(sa * SA_ELEMS + q * 32 * 2 * BK) * 2>(fa[q], abase[ha][par][sl]);
        } else if constexpr (B_KC) {
            constexpr int jj = q - TM;
            lds_read_b128<(sb * B_ELEMS + jj * 32 * BK) * 2>(fb[jj], kbase_b[hb][sl]);
        } else {
            constexpr int jj = q - TM;
            s16x4_t h0, h1;
            lds_read_tr16<(sb * B_ELEMS + (sl * 16) * BN) * 2>(h0, bbase[hb][jj]);
            lds_read_tr16<(sb * B_ELEMS + (sl * 16 + 4) * BN) * 2>(h1, bbase[hb][jj]);
            fb[jj] = __builtin_bit_cast(Frag, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    auto mfma_one = [&](auto Q, const Frag (&fa)[TM], const Frag (&fb)[TN]) {
        constexpr int q = decltype(Q)::value, i = q / TN, j = q % TN;
        if constexpr (DT == PT_BFLOAT16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    };
    auto frag_wait = [&](Frag (&fa)[TM], Frag (&fb)[TN]) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1])::"memory");
    };
    // the load issued at MFMA Q of slice SL of step kt: A loads in slice 0,
    // B loads in slice 1 (after the step's barrier)
    auto spread_load = [&](int kt, auto J, auto SL, auto Q) {
        constexpr int slot = decltype(SL)::value * TM * TN + decltype(Q)::value;
        if constexpr (slot % SPREAD == 0) issue_one(kt, J, IC<slot / SPREAD>{});
    };

    // prologue: issue steps -4 .. -1 (A of superstages 0 and 1, B of steps
    // 0 .. 2); superstage 0 and B step 0 landed for everyone
    static_for<0, NQA>([&](auto Q) { issue_one(-4, IC<8>{}, Q); });
    static_for<0, PER>([&](auto Q) { issue_one(-3, IC<9>{}, Q); });
    static_for<0, PER>([&](auto Q) { issue_one(-2, IC<10>{}, Q); });
    static_for<0, PER>([&](auto Q) { issue_one(-1, IC<11>{}, Q); });
    ring_wait<2 * PER>();
    ring_barrier();
    Frag fa[2][TM], fb[2][TN];
    static_for<0, TM + TN>([&](auto Q) { read_one(IC<0>{}, IC<0>{}, Q, fa[0], fb[0]); });
    frag_wait(fa[0], fb[0]);
    for (int kt0 = 0; kt0 < KT; kt0 += PERIOD) {
        static_for<0, PERIOD>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const int kt = kt0 + j;
            if (kt < KT) {  // uniform branch
                static_for<0, TM * TN>([&](auto Q) {
                    mfma_one(Q, fa[0], fb[0]);
                    if constexpr (decltype(Q)::value < TM + TN) read_one(J, IC<1>{}, Q, fa[1], fb[1]);
                    spread_load(kt, J, IC<0>{}, Q);
                    __builtin_amdgcn_sched_barrier(0);
                });
                frag_wait(fa[1], fb[1]);
                ring_wait<WAIT_STEP>();  // issue step kt - 2 landed
                ring_barrier();          // ... for everyone; step kt's stages are free
                static_for<0, TM * TN>([&](auto Q) {
                    mfma_one(Q, fa[1], fb[1]);
                    if constexpr (decltype(Q)::value < TM + TN) read_one(IC<j + 1>{}, IC<0>{}, Q, fa[0], fb[0]);
                    spread_load(kt, J, IC<1>{}, Q);
                    __builtin_amdgcn_sched_barrier(0);
                });
                frag_wait(fa[0], fb[0]);
            }
        });
    }
    ring_wait<0>();  // no load may still target LDS when the workgroup ends

    // epilogue (the layout of k_gemm_ring's)
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

// Ring shapes: {BK, stages, BN, workgroups per CU, schedule, waves, kind}.
// kind 0: k_gemm_ring; kind 1: k_gemm_pp (BK 32, BN 256, 8 waves; schedule
// 1 = raised priority in the compute phase); kind 2: k_gemm_wl (BK 32, B
// stages, A superstages of 64 k, K a multiple of 64).
static const int kRing[][7] = {
    {32, 4, 256, 1, 0, 4, 0}, {64, 2, 256, 1, 0, 4, 0}, {32, 2, 256, 1, 0, 4, 0}, {32, 3, 256, 1, 0, 4, 0},
    {32, 5, 256, 1, 0, 4, 0}, {32, 3, 128, 2, 0, 4, 0}, {32, 2, 128, 2, 0, 4, 0}, {64, 2, 256, 1, 1, 4, 0},
    {32, 4, 256, 1, 1, 4, 0}, {32, 3, 128, 2, 1, 4, 0}, {32, 4, 256, 1, 2, 4, 0}, {32, 3, 256, 1, 2, 4, 0},
    {32, 5, 256, 1, 2, 4, 0}, {32, 4, 256, 1, 1, 8, 0}, {64, 2, 256, 1, 1, 8, 0}, {32, 4, 256, 1, 2, 8, 0},
    {32, 5, 256, 1, 2, 8, 0}, {32, 3, 256, 1, 2, 8, 0}, {32, 4, 256, 1, 1, 8, 1}, {32, 5, 256, 1, 1, 8, 1},
    {32, 3, 256, 1, 1, 8, 1}, {32, 4, 256, 1, 0, 8, 1}, {32, 5, 256, 1, 0, 8, 1}, {32, 4, 256, 1, 2, 8, 2}};

int gemm_ring_variants() { return (int)(sizeof(kRing) / sizeof(kRing[0])); }
int gemm_ring_kind(int variant) { return kRing[variant][6]; }
int gemm_ring_bn(int variant) { return kRing[variant][2]; }
int gemm_ring_bk(int variant) { return kRing[variant][0]; }
// K must be a multiple of this: BK x stages for power-of-two rings, BK otherwise
int gemm_ring_kmul(int variant)
{
    if (kRing[variant][6] == 2) return 64;
    const int st = kRing[variant][1];
    return (st & (st - 1)) ? kRing[variant][0] : kRing[variant][0] * st;
}

void launch_gemm_ring(const GemmArgs &g, int dtype, bool b_row, int variant, dim3 grid, hipStream_t s)
{
    const dim3 block(64 * kRing[variant][5]);
#define PT_PP(DTV, STV, PRV)                                                                   \
    do {                                                                                       \
        if (b_row) k_gemm_pp<DTV, false, STV, PRV><<<grid, block, 0, s>>>(g);                  \
        else k_gemm_pp<DTV, true, STV, PRV><<<grid, block, 0, s>>>(g);                         \
    } while (0)
    if (kRing[variant][6] == 2) {
        if (dtype == PT_BFLOAT16) {
            if (b_row) k_gemm_wl<PT_BFLOAT16, false><<<grid, block, 0, s>>>(g);
            else k_gemm_wl<PT_BFLOAT16, true><<<grid, block, 0, s>>>(g);
        } else {
            if (b_row) k_gemm_wl<PT_FLOAT16, false><<<grid, block, 0, s>>>(g);
            else k_gemm_wl<PT_FLOAT16, true><<<grid, block, 0, s>>>(g);
        }
        return;
    }
    if (kRing[variant][6] == 1) {
        const int st = kRing[variant][1];
        const bool prio = kRing[variant][4] == 1;
        auto go = [&](auto DTC) {
            constexpr int D = decltype(DTC)::value;
            if (st == 4) { if (prio) PT_PP(D, 4, true); else PT_PP(D, 4, false); }
            else if (st == 5) { if (prio) PT_PP(D, 5, true); else PT_PP(D, 5, false); }
            else PT_PP(D, 3, true);
        };
        if (dtype == PT_BFLOAT16) go(IC<PT_BFLOAT16>{});
        else go(IC<PT_FLOAT16>{});
        return;
    }
#undef PT_PP
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
