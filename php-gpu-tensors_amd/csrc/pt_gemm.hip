// Batched GEMM for gfx950 on the MFMA matrix cores.
//
//   C[b] = A[b] @ B[b],  A: M x K, B: K x N, C: M x N row-major contiguous.
//
// bf16 / fp16: v_mfma_f32_32x32x16_{bf16,f16} (fp32 accumulate, RNE store
// to the operand dtype, as __float2bfloat16_rn in the reference's
// low_precision_matmul_nd_kernel, matmul_kernels.cu:738-791).
// fp32: v_mfma_f32_32x32x2f32 (true fp32 products and accumulation; the
// reference's strict-fp32 policy, matmul_kernels.cu:294-296).
//
// Tiling: a workgroup owns a BM x BN tile of C; its waves form a WM x WN
// grid, each wave a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks held in
// accumulator registers.  K advances in BK steps through two LDS stages
// (global loads of step k+1 are in flight while step k runs on the matrix
// cores).  Both operands are stored in LDS k-contiguous ([row][k], rows
// padded by 16 bytes) so that every lane reads one 16-byte pack per MFMA
// operand.  An operand whose k is not its contiguous dimension (row-major B,
// or a transposed view of A) is transposed in registers between the global
// load and the LDS store.
//
// Workgroup -> tile mapping is XCD-aware: dispatch places consecutive
// workgroups on the 8 XCDs round-robin, so the linear id is remapped to give
// each XCD a contiguous range of tiles, and tiles are walked in groups of
// GROUP_M row-blocks so that co-resident workgroups share A and B panels in
// their XCD's L2.
#include "pt_common.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>

#include "pt_gemm.h"

namespace pt {

// 16-byte pack type for register staging.
typedef uint32_t Pack __attribute__((ext_vector_type(4)));

// Gather PK k rows of VR consecutive r elements (raw[k][dword]) and emit VR
// k-contiguous packs.
template <int DT, int VR, int DW>
__device__ __forceinline__ void transpose_to_packs(const uint32_t (&raw)[GE<DT>::PK][DW],
                                                   Pack (&out)[VR])
{
    if constexpr (sizeof(typename GE<DT>::S) == 2) {
        // 16-bit: dword d holds r = 2d (low half) and r = 2d+1 (high half)
#pragma unroll
        for (int r = 0; r < VR; r++) {
            const int d = r >> 1;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint32_t lo = raw[2 * q][d], hi = raw[2 * q + 1][d];
                out[r][q] = (r & 1) ? ((lo >> 16) | (hi & 0xffff0000u))
                                      : ((lo & 0xffffu) | (hi << 16));
            }
        }
    } else {
        // fp32: raw[k][r] -> out[r].w[k]
#pragma unroll
        for (int r = 0; r < VR; r++)
#pragma unroll
            for (int q = 0; q < 4; q++) out[r][q] = raw[q][r];
    }
}

template <int DT, int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool CHECK>
struct GemmCfg {
    using S = typename GE<DT>::S;
    static constexpr int PK = GE<DT>::PK;
    static constexpr int T = 64 * WM * WN;
    static constexpr int LDK = BK + PK;      // padded LDS row (elements)
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int TM = WTM / 32, TN = WTN / 32;
    // k-contiguous loads: 16-byte packs per thread
    static constexpr int A_P = BM * BK / PK / T;
    static constexpr int B_P = BN * BK / PK / T;
    // r-contiguous loads: r elements per thread per k row
    static constexpr int A_VR = BM * BK / (T * PK);
    static constexpr int B_VR = BN * BK / (T * PK);
    static_assert(BM % (32 * WM) == 0 && BN % (32 * WN) == 0, "wave tiling");
    static_assert(BK % (2 * PK) == 0 || PK == 4, "k slices");
    static_assert(A_P >= 1 && B_P >= 1, "load split");
};

// Load helpers ------------------------------------------------------------

__device__ __forceinline__ uint32_t to_bits(uint16_t v) { return v; }
__device__ __forceinline__ uint32_t to_bits(float v) { return __float_as_uint(v); }

template <typename S>
__device__ __forceinline__ S load_elem_checked(const S *p, long long off, bool ok)
{
    return ok ? p[off] : (S)0;
}

// Stage one operand tile (R rows x BK k) from global memory into registers.
// KC: k is the contiguous dimension of the source.  KM (r-contiguous
// sources only): the tile goes to LDS k-major, [k][r], as 16-byte packs of
// r loaded and stored whole; fragment reads then gather their k values.
template <int DT, int R, int BK, int T, bool KC, bool CHECK, bool KM = false, bool CLAMP = false>
struct TileLoader {
    using S = typename GE<DT>::S;
    static constexpr int PK = GE<DT>::PK;
    static constexpr int P = R * BK / PK / T;         // packs per thread (KC, KM)
    static constexpr int VR = R * BK / (T * PK);      // r per thread (RC)
    static constexpr int DW = (VR * (int)sizeof(S) + 3) / 4;  // dwords per RC row load
    static_assert(!KM || (!KC && P >= 1 && (R / PK) * BK % T == 0), "k-major staging");
    // CLAMP (unchecked loads on an edge tile): rows past r_total read the
    // last whole row or pack instead; they only feed outputs that are not
    // stored
    static_assert(!CLAMP || (!CHECK && (KC || KM)), "clamped staging");
    Pack kc[(KC || KM) ? P : 1];
    uint32_t rc[(KC || KM) ? 1 : PK][(KC || KM) ? 1 : (DW > 0 ? DW : 1)];

    // src(r, k) = base[r * s_r + k * s_k]; rows [r0, r0+R) of r_total,
    // k in [k0, k0+BK) of K.
    __device__ __forceinline__ void load(const S *base, long long s_r, long long s_k, int r0,
                                         int r_total, int k0, int K, int tid, int vec = 0)
    {
        if constexpr (KM) {
            // pack p: k row p / (R / PK), r pack p % (R / PK); a wave reads
            // whole rows of r
#pragma unroll
            for (int j = 0; j < P; j++) {
                int p = tid + j * T;
                int k = p / (R / PK), rp = p % (R / PK);
                int gr = r0 + rp * PK, gk = k0 + k;
                if constexpr (CLAMP) gr = min(gr, r_total - PK);
                if (!CHECK || (vec && gk < K && gr + PK <= r_total)) {
                    kc[j] = *(const Pack *)(base + (long long)gk * s_k + gr);
                } else {
                    Pack pk = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (int e = 0; e < PK; e++) {
                        S v = load_elem_checked(base, (long long)gk * s_k + (long long)(gr + e) * s_r,
                                                gk < K && gr + e < r_total);
                        pk[e * sizeof(S) / 4] |= to_bits(v) << (8 * ((e * sizeof(S)) % 4));
                    }
                    kc[j] = pk;
                }
            }
        } else if constexpr (KC) {
#pragma unroll
            for (int j = 0; j < P; j++) {
                int p = tid + j * T;
                int r = p / (BK / PK), kp = p % (BK / PK);
                int gr = r0 + r, gk = k0 + kp * PK;
                if constexpr (CLAMP) gr = min(gr, r_total - 1);
                if (!CHECK || (vec && gr < r_total && gk + PK <= K)) {
                    kc[j] = *(const Pack *)(base + (long long)gr * s_r + gk);
                } else {
                    Pack pk = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (int e = 0; e < PK; e++) {
                        S v = load_elem_checked(base, (long long)gr * s_r + (long long)(gk + e) * s_k,
                                                gr < r_total && gk + e < K);
                        pk[e * sizeof(S) / 4] |= to_bits(v) << (8 * ((e * sizeof(S)) % 4));
                    }
                    kc[j] = pk;
                }
            }
        } else {
            constexpr int RG = R / VR;  // r groups
            int rg = tid % RG, kg = tid / RG;
            int gr = r0 + rg * VR;
#pragma unroll
            for (int e = 0; e < PK; e++) {
                int gk = k0 + kg * PK + e;
                if (!CHECK || (vec && gk < K && gr + VR <= r_total)) {
                    const S *p = base + (long long)gk * s_k + gr;
                    if constexpr (VR * sizeof(S) == 16) {
                        uint4 v = *(const uint4 *)p;
                        rc[e][0] = v.x; rc[e][1] = v.y; rc[e][2] = v.z; rc[e][3] = v.w;
                    } else if constexpr (VR * sizeof(S) == 8) {
                        uint2 v = *(const uint2 *)p;
                        rc[e][0] = v.x; rc[e][1] = v.y;
                    } else if constexpr (VR * sizeof(S) == 4) {
                        rc[e][0] = *(const uint32_t *)p;
                    } else {
                        rc[e][0] = *(const uint16_t *)p;
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < DW; q++) rc[e][q] = 0u;
#pragma unroll
                    for (int q = 0; q < VR; q++) {
                        S v = load_elem_checked(base, (long long)gk * s_k + (long long)(gr + q) * s_r,
                                                gk < K && gr + q < r_total);
                        rc[e][q * sizeof(S) / 4] |= to_bits(v) << (8 * ((q * sizeof(S)) % 4));
                    }
                }
            }
        }
    }

    // Write the staged tile to LDS laid out [r][k] with row pitch LDK (or,
    // KM, [k][r] with row pitch LDK).
    template <int LDK>
    __device__ __forceinline__ void store(S *lds, int tid)
    {
        if constexpr (KM) {
#pragma unroll
            for (int j = 0; j < P; j++) {
                int p = tid + j * T;
                int k = p / (R / PK), rp = p % (R / PK);
                *(Pack *)(lds + k * LDK + rp * PK) = kc[j];
            }
        } else if constexpr (KC) {
#pragma unroll
            for (int j = 0; j < P; j++) {
                int p = tid + j * T;
                int r = p / (BK / PK), kp = p % (BK / PK);
                *(Pack *)(lds + r * LDK + kp * PK) = kc[j];
            }
        } else {
            constexpr int RG = R / VR;
            int rg = tid % RG, kg = tid / RG;
            Pack out[VR];
            transpose_to_packs<DT, VR, DW>(rc, out);
#pragma unroll
            for (int q = 0; q < VR; q++)
                *(Pack *)(lds + (rg * VR + q) * LDK + kg * PK) = out[q];
        }
    }
};

// LDS layout of one stage.  fp32 operands whose r is contiguous in memory
// stay k-major in LDS ([k][r], row pitch r + 8: the two half-waves of a
// fragment read, four k rows apart, fall on different banks); the others
// are [r][k] with the row padded by one pack.
template <int DT, int BM, int BN, int BK, bool A_KC, bool B_KC>
struct GemmLds {
    static constexpr int PK = GE<DT>::PK;
    static constexpr int LDK = BK + PK;
    static constexpr bool AKM = DT == PT_FLOAT32 && !A_KC;
    static constexpr bool BKM = DT == PT_FLOAT32 && !B_KC;
    static constexpr int LDA = AKM ? BM + 8 : LDK, LDB = BKM ? BN + 8 : LDK;
    static constexpr int SA = AKM ? BK * LDA : BM * LDK;
    static constexpr int SB = BKM ? BK * LDB : BN * LDK;
};

template <int DT, int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool CHECK, int SCHED,
          bool CLAMP = false>
__device__ __forceinline__ void gemm_core(const GemmArgs &g,
                                          typename GE<DT>::S (&lds_a)[2][GemmLds<DT, BM, BN, BK, A_KC, B_KC>::SA],
                                          typename GE<DT>::S (&lds_b)[2][GemmLds<DT, BM, BN, BK, A_KC, B_KC>::SB],
                                          const typename GE<DT>::S *A, const typename GE<DT>::S *B, int Kl,
                                          int bidx, int split, int m0, int n0)
{
    using C = GemmCfg<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK>;
    using S = typename C::S;
    using L = GemmLds<DT, BM, BN, BK, A_KC, B_KC>;
    constexpr int T = C::T, PK = C::PK, LDK = C::LDK, TM = C::TM, TN = C::TN;
    constexpr bool AKM = L::AKM, BKM = L::BKM;
    constexpr int LDA = L::LDA, LDB = L::LDB;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // Two register staging sets: the global loads of tile k+2 are issued
    // while tile k runs on the matrix cores and tile k+1 waits in the other
    // set, giving the loads two K steps of MFMA work to arrive.
    using LoaderA = TileLoader<DT, BM, BK, T, A_KC, CHECK, AKM, CLAMP>;
    using LoaderB = TileLoader<DT, BN, BK, T, B_KC, CHECK, BKM, CLAMP>;
    LoaderA la[2];
    LoaderB lb[2];

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    const int KT = (Kl + BK - 1) / BK;
    // Loads past the last K step re-read the last one (in bounds, never
    // stored to LDS as a step's data): with no branch around the loads the
    // compiler knows exactly which loads are in flight, and waits for the
    // staged step only, never for the one issued after it.
    // A(m, k): r = m, s_r = a_sm, s_k = a_sk.  B(k, n): r = n, s_r = b_sn, s_k = b_sk.
    la[0].load(A, g.a_sm, g.a_sk, m0, g.M, 0, Kl, tid, g.vec_a);
    lb[0].load(B, g.b_sn, g.b_sk, n0, g.N, 0, Kl, tid, g.vec_b);
    la[1].load(A, g.a_sm, g.a_sk, m0, g.M, min(1, KT - 1) * BK, Kl, tid, g.vec_a);
    lb[1].load(B, g.b_sn, g.b_sk, n0, g.N, min(1, KT - 1) * BK, Kl, tid, g.vec_b);
    la[0].template store<LDA>(lds_a[0], tid);
    lb[0].template store<LDB>(lds_b[0], tid);
    __syncthreads();

    const int arow = wm * C::WTM + (lane & 31);
    const int brow = wn * C::WTN + (lane & 31);
    // k-major A with two or four row blocks per wave: block i's row r is the
    // wave's local row TM * r + i, so that one lane's values of all blocks at
    // one k sit side by side in LDS and load as one 8- or 16-byte read
    constexpr bool AIL = AKM && (TM == 2 || TM == 4);
    const int arow_il = wm * C::WTM + TM * (lane & 31);
    const int khalf = (lane >> 5) * PK;
    // One k-slice feeds one MFMA per (i, j) block: 16 k for 16-bit operands,
    // 8 k (four 32x32x2 MFMAs) for fp32.  Fragments of slice s+1 are read
    // from LDS into the second register set while slice s runs on the
    // matrix cores, so LDS latency overlaps MFMA execution.
    constexpr int KS = 2 * PK;
    constexpr int NS = BK / KS;
    using Frag = typename FragT<DT>::type;
    Frag fa[2][TM], fb[2][TN];
    auto read_frags = [&](const S *sa, const S *sb, int slice, Frag (&ra)[TM], Frag (&rb)[TN]) {
        if constexpr (AIL) {
#pragma unroll
            for (int e = 0; e < PK; e++) {
                const S *src = sa + (slice * KS + khalf + e) * LDA + arow_il;
                if constexpr (TM == 2) {
                    const float2 t = *(const float2 *)src;
                    ra[0][e] = t.x;
                    ra[1][e] = t.y;
                } else {
                    const float4 t = *(const float4 *)src;
                    ra[0][e] = t.x;
                    ra[1][e] = t.y;
                    ra[2][e] = t.z;
                    ra[3][e] = t.w;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if constexpr (AIL) {
            } else if constexpr (AKM) {
#pragma unroll
                for (int e = 0; e < PK; e++) ra[i][e] = sa[(slice * KS + khalf + e) * LDA + arow + i * 32];
            } else {
                ra[i] = *(const Frag *)(sa + (arow + i * 32) * LDK + slice * KS + khalf);
            }
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (BKM) {
#pragma unroll
                for (int e = 0; e < PK; e++) rb[j][e] = sb[(slice * KS + khalf + e) * LDB + brow + j * 32];
            } else {
                rb[j] = *(const Frag *)(sb + (brow + j * 32) * LDK + slice * KS + khalf);
            }
        }
    };
    read_frags(lds_a[0], lds_b[0], 0, fa[0], fb[0]);

    // step kt: W holds tile kt+1 (to LDS after the MFMAs), L receives tile kt+2
    auto step = [&](int kt, LoaderA &wa, LoaderB &wb, LoaderA &la_, LoaderB &lb_) {
        const int cur = kt & 1;
        const int kload = min(kt + 2, KT - 1) * BK;
        la_.load(A, g.a_sm, g.a_sk, m0, g.M, kload, Kl, tid, g.vec_a);
        lb_.load(B, g.b_sn, g.b_sk, n0, g.N, kload, Kl, tid, g.vec_b);
#pragma unroll
        for (int sl = 0; sl < NS; sl++) {
            if (sl + 1 < NS)
                read_frags(lds_a[cur], lds_b[cur], sl + 1, fa[(sl + 1) & 1], fb[(sl + 1) & 1]);
            mfma_block<DT, TM, TN>(acc, fa[sl & 1], fb[sl & 1]);
            if constexpr (SCHED == 1) {
                __builtin_amdgcn_iglp_opt(0);
            } else if constexpr (SCHED == 2) {
                __builtin_amdgcn_iglp_opt(1);
            } else if constexpr (SCHED == 3) {
                // interleave: one MFMA, then one LDS read, for the reads of
                // the next slice; remaining MFMAs follow
#pragma unroll
                for (int q = 0; q < TM + TN; q++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                }
                __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
            }
        }
        // the last step stores and reads a re-read copy that no MFMA uses
        wa.template store<LDA>(lds_a[cur ^ 1], tid);
        wb.template store<LDB>(lds_b[cur ^ 1], tid);
        __syncthreads();
        read_frags(lds_a[cur ^ 1], lds_b[cur ^ 1], 0, fa[0], fb[0]);
    };
    for (int kt = 0; kt < KT; kt += 2) {
        step(kt, la[1], lb[1], la[0], lb[0]);
        if (kt + 1 < KT) step(kt + 1, la[0], lb[0], la[1], lb[1]);
    }

    // ---- epilogue: lane holds column n = lane%32 and rows
    // 8*(e/4) + 4*(lane/32) + e%4 of each 32x32 block.
    const size_t mn = (size_t)g.M * (size_t)g.N;
    char *Cb = (char *)g.c + (size_t)bidx * mn * sizeof(S);
    float *Pb = g.ksplit > 1 ? g.partial + ((size_t)split * g.batch + bidx) * mn : nullptr;
    const int col_l = lane & 31;
    const int row_l = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * C::WTN + j * 32 + col_l;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int rho = (e >> 2) * 8 + row_l + (e & 3);  // row within the 32x32 block
                const int m = m0 + wm * C::WTM + (AIL ? TM * rho + i : i * 32 + rho);
                if ((!CHECK && !CLAMP) || (m < g.M && n < g.N)) {
                    if (Pb) Pb[(size_t)m * g.N + n] = acc[i][j][e];
                    else store_c<DT>(Cb, (size_t)m * g.N + n, acc[i][j][e]);
                }
            }
        }
}

template <int DT, int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool CHECK,
          int SCHED = 0, int MINW = 1>
__global__ __launch_bounds__(64 * WM * WN, MINW) void k_gemm(GemmArgs g)
{
    using S = typename GE<DT>::S;
    constexpr int GROUP_M = 4;

    using L = GemmLds<DT, BM, BN, BK, A_KC, B_KC>;
    __shared__ __attribute__((aligned(16))) S lds_a[2][L::SA];
    __shared__ __attribute__((aligned(16))) S lds_b[2][L::SB];

    // ---- tile selection (XCD-aware remap + grouped ordering)
    const int ntile = g.tiles_m * g.tiles_n;
    long long lin = blockIdx.x;
    if (g.remap) {
        long long total = (long long)ntile * g.batch;
        long long per = total / 8;
        lin = (lin % 8) * per + lin / 8;
    }
    const int bidx = (int)(lin / ntile);
    if (bidx >= g.batch) return;  // whole workgroup: grid larger than the tile count
    const int t = (int)(lin % ntile);
    const int group = t / (GROUP_M * g.tiles_n);
    const int first_m = group * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int tm = first_m + (t % (GROUP_M * g.tiles_n)) % gsz;
    const int tn = (t % (GROUP_M * g.tiles_n)) / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    long long oa, ob;
    batch_offsets(g, bidx, oa, ob);
    // split-K: this workgroup's K chunk [kbase, kbase + Kl)
    const int split = blockIdx.y;
    const int kbase = split * g.k_chunk;
    const int Kl = g.ksplit > 1 ? min(g.k_chunk, g.K - kbase) : g.K;
    const S *A = (const S *)g.a + oa + (long long)kbase * g.a_sk;
    const S *B = (const S *)g.b + ob + (long long)kbase * g.b_sk;

    if constexpr (CHECK) {
        // Whole K steps and packable operands: tiles wholly inside M x N run
        // the unchecked core, edge tiles the same core with clamped rows and
        // a guarded store (all of one launch's workgroups run at once, so an
        // edge tile as slow as a checked one would set the launch's time);
        // only ragged K or unpackable operands pay for per-element checks.
        constexpr bool CLAMPABLE = (A_KC || L::AKM) && (B_KC || L::BKM);
        const bool whole = g.vec_a && g.vec_b && Kl % BK == 0;
        const bool interior = whole && m0 + BM <= g.M && n0 + BN <= g.N;
        const bool clampable = whole && (A_KC || g.M % GE<DT>::PK == 0) && (B_KC || g.N % GE<DT>::PK == 0);
        if (interior)
            gemm_core<DT, BM, BN, BK, WM, WN, A_KC, B_KC, false, SCHED>(g, lds_a, lds_b, A, B, Kl, bidx, split, m0, n0);
        else if (CLAMPABLE && clampable)
            gemm_core<DT, BM, BN, BK, WM, WN, A_KC, B_KC, false, SCHED, CLAMPABLE>(g, lds_a, lds_b, A, B, Kl, bidx,
                                                                                split, m0, n0);
        else
            gemm_core<DT, BM, BN, BK, WM, WN, A_KC, B_KC, true, SCHED>(g, lds_a, lds_b, A, B, Kl, bidx, split, m0, n0);
    } else {
        gemm_core<DT, BM, BN, BK, WM, WN, A_KC, B_KC, false, SCHED>(g, lds_a, lds_b, A, B, Kl, bidx, split, m0, n0);
    }
}


// Split-K epilogue: C = sum of the K-chunk partials, in chunk order, rounded
// once to the output dtype.
// Sum of the split-K partials [ksplit][count] in chunk order, rounded once.
// V adjacent outputs per thread (16-byte loads when V = 4); eight chunks'
// loads are in flight at a time, predicated past the last chunk, and their
// additions stay in order (a chunk past the end is skipped, not added as 0,
// so that a -0.0 sum keeps its sign).
template <int DT, int V>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float *__restrict__ partial, void *__restrict__ c,
                                                       size_t count, int ksplit)
{
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
    if (i >= count) return;
    float acc[V];
    auto load = [&](int k, float (&v)[V]) {
        const float *p = partial + (size_t)k * count + i;
        if constexpr (V == 4) {
            const float4 t = *(const float4 *)p;
            v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
        } else {
#pragma unroll
            for (int e = 0; e < V; e++) v[e] = p[e];
        }
    };
    load(0, acc);
    for (int k = 1; k < ksplit; k += 8) {
        float v[8][V];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (k + u < ksplit) load(k + u, v[u]);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (k + u < ksplit)
#pragma unroll
                for (int e = 0; e < V; e++) acc[e] += v[u][e];
    }
#pragma unroll
    for (int e = 0; e < V; e++) store_c<DT>(c, i + e, acc[e]);
}

// ------------------------------------------- direct-to-LDS 16-bit kernel
// bf16 / fp16 GEMM for whole 256x256 tiles with K a multiple of 64 and
// k-contiguous A.  Operands go from global memory straight into LDS with
// global_load_lds_dwordx4 (no register staging): each such instruction
// fills 1 KB of LDS, 16 bytes per lane at lane-consecutive addresses, and
// the lane -> global address map applies an XOR swizzle so that the
// fragment reads are free of bank conflicts:
//   k-contiguous operand, row r of BK/8 16-byte chunks: physical chunk pc
//     holds logical k chunk pc ^ swz_k(r);
//   row-major B ([k][n], n contiguous), k-row r of 32 chunks: physical
//     chunk pc holds logical n chunk pc ^ ((r & 3) << 2).
// Row-major B fragments are read with ds_read_b64_tr_b16, the gfx950 LDS
// transpose read: in each group of 16 lanes, lane i receives, for j = 0..3,
// element (i % 4) of the 4 elements addressed by lane 4j + i/4.  Lane
// 4j + q therefore addresses B[k + j][n + 4q .. n + 4q + 3], and two such
// reads give a lane the 8 consecutive k of its MFMA B operand.
// Those reads are issued as inline asm and waited for explicitly: the
// compiler would otherwise wait for every in-flight LDS DMA load before
// them.  The two LDS stages are separate arrays, so that the compiler can
// tell the DMA writes into one stage from the fragment reads of the other.
// 8 waves (2 x 4) with 128 x 64 wave tiles; BK = 64 in two stages: the
// loads of step k+1 run while step k is on the matrix cores.
template <int DT, bool B_KC>
__global__ __launch_bounds__(512, 1) void k_gemm_direct(GemmArgs g)
{
    using S = uint16_t;
    constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 4;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    constexpr int CPR = BK / 8;           // 16-byte chunks per k-contiguous row
    constexpr int RPI = 64 / CPR;         // such rows per load instruction
    constexpr int NQ = A_ELEMS / 512 / 8; // load instructions per wave per operand
    constexpr int GROUP_M = 4;
    __shared__ __attribute__((aligned(1024))) S lds0[A_ELEMS + B_ELEMS];
    __shared__ __attribute__((aligned(1024))) S lds1[A_ELEMS + B_ELEMS];

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
    const int wm = wave / WN, wn = wave % WN;

    auto issue = [&](int kt, S *buf) {
        const int k0 = kt * BK;
#pragma unroll
        for (int q4 = 0; q4 < NQ; q4++) {
            const int q = wave * NQ + q4;
            const int row = q * RPI + lane / CPR, pc = lane % CPR;
            const S *src = A + (long long)row * lda + k0 + (pc ^ swz_k(row, CPR)) * 8;
            __builtin_amdgcn_global_load_lds((const void *)src, (PT_LDS_AS void *)(buf + q * 512), 16, 0, 0);
        }
#pragma unroll
        for (int q4 = 0; q4 < NQ; q4++) {
            const int q = wave * NQ + q4;
            const S *src;
            if constexpr (B_KC) {
                const int row = q * RPI + lane / CPR, pc = lane % CPR;
                src = B + (long long)row * ldb + k0 + (pc ^ swz_k(row, CPR)) * 8;
            } else {
                const int row = q * 2 + (lane >> 5), pc = lane & 31;
                src = B + (long long)(k0 + row) * ldb + (pc ^ ((row & 3) << 2)) * 8;
            }
            __builtin_amdgcn_global_load_lds((const void *)src, (PT_LDS_AS void *)(buf + A_ELEMS + q * 512), 16, 0,
                                             0);
        }
    };

    using Frag = typename FragT<DT>::type;
    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    auto read_frags = [&](const S *buf, int slice, Frag (&fa)[TM], Frag (&fb)[TN]) {
        const S *la = buf;
        const S *lb = buf + A_ELEMS;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int row = wm * WTM + i * 32 + (lane & 31);
            const int kc = slice * 2 + (lane >> 5);
            fa[i] = *(const Frag *)(la + row * BK + (kc ^ swz_k(row, CPR)) * 8);
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (B_KC) {
                const int row = wn * WTN + j * 32 + (lane & 31);
                const int kc = slice * 2 + (lane >> 5);
                fb[j] = *(const Frag *)(lb + row * BK + (kc ^ swz_k(row, CPR)) * 8);
            } else {
                const int grp = lane >> 4, s = lane & 15;
                const int n = wn * WTN + j * 32 + (grp & 1) * 16 + 4 * (s & 3);
                union { s16x4_t h[2]; Frag f; } u;
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    const int kk = slice * 16 + (grp >> 1) * 8 + tt * 4 + (s >> 2);
                    const S *p = lb + kk * BN + ((n >> 3) ^ ((kk & 3) << 2)) * 8 + (n & 7);
                    const unsigned addr = (unsigned)(size_t)(PT_LDS_AS const S *)p;
                    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(u.h[tt]) : "v"(addr));
                }
                fb[j] = u.f;
            }
        }
    };
    // completes the asm transpose reads of fb (and, conservatively, every
    // LDS access of the wave) before fb is used
    auto tr_wait = [&](Frag (&f)[TN]) {
        if constexpr (!B_KC) {
            static_assert(TN == 2, "wait operands");
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]));
        }
    };

    const int KT = g.K / BK;
    issue(0, lds0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    Frag fa[2][TM], fb[2][TN];
    auto step = [&](int kt, S *cur, S *nxt) {
        if (kt + 1 < KT) issue(kt + 1, nxt);  // nxt was last read before the previous barrier
        read_frags(cur, 0, fa[0], fb[0]);
        tr_wait(fb[0]);
#pragma unroll
        for (int sl = 0; sl < BK / 16; sl++) {
            if (sl + 1 < BK / 16) read_frags(cur, sl + 1, fa[(sl + 1) & 1], fb[(sl + 1) & 1]);
            mfma_block<DT, TM, TN>(acc, fa[sl & 1], fb[sl & 1]);
            __builtin_amdgcn_iglp_opt(1);
            if (sl + 1 < BK / 16) tr_wait(fb[(sl + 1) & 1]);
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA loads of step kt+1 have landed
        __syncthreads();
    };
    for (int kt = 0; kt < KT; kt += 2) {
        step(kt, lds0, lds1);
        if (kt + 1 < KT) step(kt + 1, lds1, lds0);
    }

    char *Cb = (char *)g.c + (size_t)bidx * (size_t)g.M * (size_t)g.N * sizeof(S);
    const int col_l = lane & 31;
    const int row_l = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * WTN + j * 32 + col_l;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm * WTM + i * 32 + (e >> 2) * 8 + row_l + (e & 3);
                store_c<DT>(Cb, (size_t)m * g.N + n, acc[i][j][e]);
            }
        }
}

// ---------------------------------------------------------------- host side
static int g_sched = 2;

template <int DT, int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool CHECK, int MINW = 1>
static void launch_cfg(const GemmArgs &g, hipStream_t s)
{
    const dim3 grid((unsigned)((long long)g.tiles_m * g.tiles_n * g.batch), (unsigned)(g.ksplit > 1 ? g.ksplit : 1));
    if constexpr (BM == 256 && BN == 128 && A_KC && !B_KC && !CHECK && DT != PT_FLOAT32) {
        // two workgroups per CU: waves sharing a SIMD belong to different
        // workgroups, so their barrier phases do not coincide
        if (g_sched >= 4) {
            if (g_sched == 4)
                k_gemm<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK, 0, 2><<<grid, dim3(64 * WM * WN), 0, s>>>(g);
            else
                k_gemm<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK, 2, 2><<<grid, dim3(64 * WM * WN), 0, s>>>(g);
            return;
        }
    }
    if constexpr (BM == 256 && BN == 256 && A_KC && !B_KC && !CHECK && DT != PT_FLOAT32) {
        if (g_sched == 1) {
            k_gemm<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK, 1><<<grid, dim3(64 * WM * WN), 0, s>>>(g);
            return;
        }
        if (g_sched == 2) {
            k_gemm<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK, 2><<<grid, dim3(64 * WM * WN), 0, s>>>(g);
            return;
        }
        if (g_sched == 3) {
            k_gemm<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK, 3><<<grid, dim3(64 * WM * WN), 0, s>>>(g);
            return;
        }
    }
    k_gemm<DT, BM, BN, BK, WM, WN, A_KC, B_KC, CHECK, 0, MINW><<<grid, dim3(64 * WM * WN), 0, s>>>(g);
}

template <int DT, int BM, int BN, int BK, int WM, int WN, int MINW = 1>
static void launch_layouts(const GemmArgs &g, bool a_kc, bool b_kc, bool check, hipStream_t s)
{
    if (check) {
        if (a_kc && b_kc) launch_cfg<DT, BM, BN, BK, WM, WN, true, true, true, MINW>(g, s);
        else if (a_kc) launch_cfg<DT, BM, BN, BK, WM, WN, true, false, true, MINW>(g, s);
        else if (b_kc) launch_cfg<DT, BM, BN, BK, WM, WN, false, true, true, MINW>(g, s);
        else launch_cfg<DT, BM, BN, BK, WM, WN, false, false, true, MINW>(g, s);
    } else {
        if (a_kc && b_kc) launch_cfg<DT, BM, BN, BK, WM, WN, true, true, false, MINW>(g, s);
        else if (a_kc) launch_cfg<DT, BM, BN, BK, WM, WN, true, false, false, MINW>(g, s);
        else if (b_kc) launch_cfg<DT, BM, BN, BK, WM, WN, false, true, false, MINW>(g, s);
        else launch_cfg<DT, BM, BN, BK, WM, WN, false, false, false, MINW>(g, s);
    }
}

// Tile configurations: workgroup tile BM x BN, K step (1x or 2x the base
// BK of the dtype), wave grid WM x WN.
enum GemmTile {
    TILE_256x128 = 0, TILE_128x128 = 1, TILE_64x64 = 2, TILE_256x256 = 3,
    TILE_256x128_K2 = 4, TILE_256x256_K2 = 5, TILE_256x256_W4 = 6, TILE_256x256_W4_K2 = 7,
    TILE_256x256_DIRECT = 8, TILE_256x128_W8 = 9, TILE_128x128_W8 = 10, TILE_128x128_W8_K2 = 11,
    TILE_128x64_W4M2 = 12, TILE_128x64_W4M2_K2 = 13,
    // LDS-ring kernels (k_gemm_ring, k_gemm_pp, k_gemm_wl): variants 0..23
    // of gemm_ring_variants()
    TILE_RING_FIRST = 14, TILE_RING_LAST = 37,
    // fp32 LDS-ring kernel (k_gemm_f32r, pt_gemm_f32ring.hip): 128x128
    // tiles, K steps of 32, one workgroup per CU
    TILE_F32_RING = 38,
    TILE_COUNT = 39,
    // large bf16 and fp16 products with K a multiple of 64: k_gemm_wl (the
    // 8-wave ring with A in whole 128-byte lines).  Config 4 at steady state,
    // alternating runs on one box: bf16 472-475 us against 488-490 us for the
    // 8-wave ring with BK 32 x 5 stages, fp16 524 us against 532 us.  Other
    // K keep that ring (TILE_RING_HALF).
    TILE_RING_DEFAULT = TILE_RING_FIRST + 23, TILE_RING_DEFAULT_F16 = TILE_RING_DEFAULT,
    TILE_RING_HALF = TILE_RING_FIRST + 16
};
struct TileInfo { int bm, bn, kmul; };
static const TileInfo kTiles[TILE_COUNT] = {
    {256, 128, 1}, {128, 128, 1}, {64, 64, 1}, {256, 256, 1}, {256, 128, 2}, {256, 256, 2},
    {256, 256, 1}, {256, 256, 2}, {256, 256, 2}, {256, 128, 1}, {128, 128, 1}, {128, 128, 2},
    {128, 64, 1}, {128, 64, 2}, {256, 256, 1}, {256, 256, 2}, {256, 256, 1}, {256, 256, 1},
    {256, 256, 1}, {256, 128, 1}, {256, 128, 1}, {256, 256, 2}, {256, 256, 1}, {256, 128, 1},
    {256, 256, 1}, {256, 256, 1}, {256, 256, 1}, {256, 256, 1}, {256, 256, 1}, {256, 256, 1},
    {256, 256, 1}, {256, 256, 1}, {256, 256, 1}, {256, 256, 1}, {256, 256, 1}, {256, 256, 1},
    {256, 256, 1}, {256, 256, 1}, {128, 128, 2}};

static int g_tile_override = -1;

// Workgroups a split-K product aims for (512: two per CU).  PT_SPLITK_WORKGROUPS
// overrides it, a tuning knob read once from the environment.
static long long splitk_workgroups()
{
    static const long long w = [] {
        const char *e = getenv("PT_SPLITK_WORKGROUPS");
        const long long v = e && *e ? atoll(e) : 0;
        return v >= 64 && v <= 8192 ? v : 512;
    }();
    return w;
}

// Ring depth of the fp32 ring kernel: 4 stages (one workgroup per CU) or 2
// (two per CU), for products with and without a K split.
// PT_F32R_STAGES and PT_F32R_SPLIT_STAGES override them (tuning knobs read
// once from the environment).
static int ring_stages(bool split)
{
    auto read = [](const char *name, int dflt) {
        const char *e = getenv(name);
        const int v = e && *e ? atoi(e) : 0;
        return v == 2 || v == 4 ? v : dflt;
    };
    static const int whole = read("PT_F32R_STAGES", 4), parts = read("PT_F32R_SPLIT_STAGES", 4);
    return split ? parts : whole;
}

// The ring kernel's K split aims for one round of workgroups: 256 with 4
// stages (a CU each), 512 with 2.  PT_SPLITK_RING_WORKGROUPS overrides it.
static long long splitk_ring_workgroups()
{
    static const long long w = [] {
        const char *e = getenv("PT_SPLITK_RING_WORKGROUPS");
        const long long v = e && *e ? atoll(e) : 0;
        return v >= 64 && v <= 8192 ? v : (ring_stages(true) == 2 ? 512 : 256);
    }();
    return w;
}

// Tiles chosen by pt_matmul_tune, per (dtype, M, N, K, batch, layout).
static std::mutex g_tuned_mu;
static std::map<std::string, int> g_tuned;

static std::string tune_key(int dtype, int M, int N, int K, long long batch, bool a_k1, bool b_k1)
{
    char key[96];
    snprintf(key, sizeof(key), "%d:%d:%d:%d:%lld:%d:%d", dtype, M, N, K, batch, a_k1 ? 1 : 0, b_k1 ? 1 : 0);
    return key;
}

// K step per LDS stage: 32 for 16-bit operands, 16 for fp32 (same bytes).
template <int DT> struct GemmBK { static constexpr int v = DT == PT_FLOAT32 ? 16 : 32; };

template <int DT>
static void launch_dt(GemmArgs g, int tile, bool a_kc, bool b_kc, bool check, hipStream_t s)
{
    constexpr int BK = GemmBK<DT>::v;
    const TileInfo &ti = kTiles[tile];
    g.tiles_m = (g.M + ti.bm - 1) / ti.bm;
    g.tiles_n = (g.N + ti.bn - 1) / ti.bn;
    switch (tile) {
    case TILE_256x128:
        if constexpr (DT != PT_FLOAT32) {
            if (!check && a_kc && !b_kc) {
                launch_cfg<DT, 256, 128, BK, 2, 2, true, false, false>(g, s);
                break;
            }
        }
        // the 256x128 kernel exists for one layout; the others run 128x128
        // tiles, so the tile grid is recounted for that shape
        g.tiles_m = (g.M + 127) / 128;
        g.tiles_n = (g.N + 127) / 128;
        g.remap = ((long long)g.tiles_m * g.tiles_n * g.batch) % 8 == 0;
        launch_layouts<DT, 128, 128, BK, 2, 2>(g, a_kc, b_kc, check, s);
        break;
    case TILE_128x128: launch_layouts<DT, 128, 128, BK, 2, 2>(g, a_kc, b_kc, check, s); break;
    case TILE_256x256: launch_layouts<DT, 256, 256, BK, 2, 4>(g, a_kc, b_kc, check, s); break;
    case TILE_256x256_K2: launch_layouts<DT, 256, 256, 2 * BK, 2, 4>(g, a_kc, b_kc, check, s); break;
    // 8 waves on a 256x128 tile (128x32 per wave): the fp32 kernel that
    // keeps its accumulators and staging in registers without spilling
    case TILE_256x128_W8: launch_layouts<DT, 256, 128, BK, 2, 4>(g, a_kc, b_kc, check, s); break;
    case TILE_128x128_W8: launch_layouts<DT, 128, 128, BK, 2, 4>(g, a_kc, b_kc, check, s); break;
    // fp32 only (the 16-bit types have their own kernels at these sizes)
    case TILE_128x128_W8_K2:
        if constexpr (DT == PT_FLOAT32) launch_layouts<DT, 128, 128, 2 * BK, 2, 4>(g, a_kc, b_kc, check, s);
        break;
    // 4 waves on 128x64 (64x32 per wave), two workgroups per CU: waves of
    // different workgroups share each SIMD, so one fills the other's
    // barrier and LDS-latency gaps
    case TILE_128x64_W4M2:
        if constexpr (DT == PT_FLOAT32) launch_layouts<DT, 128, 64, BK, 2, 2, 2>(g, a_kc, b_kc, check, s);
        break;
    case TILE_128x64_W4M2_K2:
        if constexpr (DT == PT_FLOAT32) launch_layouts<DT, 128, 64, 2 * BK, 2, 2, 2>(g, a_kc, b_kc, check, s);
        break;
    case TILE_F32_RING:
        // fp32 operands in 16-byte packs with whole K steps run the ring
        // kernel (edge tiles included); others the 8-wave 128x128 kernel
        if constexpr (DT == PT_FLOAT32) {
            if (gemm_f32r_eligible(g, a_kc, b_kc)) {
                launch_gemm_f32r(g, a_kc, b_kc, ring_stages(g.ksplit > 1), s);
                break;
            }
        }
        launch_layouts<DT, 128, 128, BK, 2, 4>(g, a_kc, b_kc, check, s);
        break;
    default: launch_layouts<DT, 64, 64, BK, 2, 2>(g, a_kc, b_kc, check, s); break;
    }
}

__global__ void k_zero_fill(uint8_t *p, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

static int g_precision = 0;

}  // namespace pt

using namespace pt;

extern "C" {

pt_status pt_matmul_set_precision(int precision)
{
    if (precision != 0 && precision != 1)
        return fail(PT_ERR_INVALID, "Unknown matmul precision %d", precision);
    // gfx950 has no reduced-precision fp32 (xf32) MFMA: a TF32 request is
    // refused as on a device without TF32, and strict fp32 stays selected
    if (precision == 1)
        return fail(PT_ERR_UNSUPPORTED, "TF32 matmul precision is not available on gfx950");
    g_precision = precision;
    return PT_OK;
}

const char *pt_matmul_precision_name(void)
{
    return "fp32-strict";
}

// Instruction-scheduling variant of the 256x256 kernels (tuning knob):
// 0 = compiler default, 1/2 = iglp strategies, 3 = MFMA/LDS interleave.
pt_status pt_matmul_set_schedule(int sched)
{
    if (sched < 0 || sched > 5) return fail(PT_ERR_INVALID, "schedule %d", sched);
    g_sched = sched;
    return PT_OK;
}

// Tile override (see kTiles), -1 = automatic.
pt_status pt_matmul_set_tile(int tile)
{
    if (tile < -1 || tile >= TILE_COUNT || tile == TILE_256x128_K2 ||
        tile == TILE_256x256_W4 || tile == TILE_256x256_W4_K2)
        return fail(PT_ERR_INVALID, "tile %d is not built", tile);
    g_tile_override = tile;
    return PT_OK;
}

pt_status pt_matmul(const void *a, const void *b, void *c, int dtype,
                    const int *shape_a, const size_t *strides_a, int nd_a,
                    const int *shape_b, const size_t *strides_b, int nd_b,
                    const int *shape_c, int nd_c, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (dtype != PT_FLOAT32 && dtype != PT_FLOAT16 && dtype != PT_BFLOAT16)
        return fail(PT_ERR_INVALID, "matmul requires matching float32, float16 or bfloat16 operands");
    if (nd_a < 2 || nd_b < 2 || nd_a > PT_MAX_DIMS || nd_b > PT_MAX_DIMS ||
        shape_a[nd_a - 1] != shape_b[nd_b - 2])
        return fail(PT_ERR_INVALID,
                    "matmul requires rank >= 2, matching inner dimensions and broadcast-compatible batches");
    // batch broadcast (tensor_matmul_shape, src/tensor_shape.h:46-59)
    int bnd = (nd_a > nd_b ? nd_a : nd_b) - 2;
    if (nd_c != bnd + 2) return fail(PT_ERR_INVALID, "matmul output rank mismatch");
    if (bnd > GEMM_MAX_BATCH_DIMS) return fail(PT_ERR_INVALID, "matmul supports at most 8 batch dims");
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.M = shape_a[nd_a - 2];
    g.K = shape_a[nd_a - 1];
    g.N = shape_b[nd_b - 1];
    if (shape_c[nd_c - 2] != g.M || shape_c[nd_c - 1] != g.N)
        return fail(PT_ERR_INVALID, "matmul output shape mismatch");
    long long batch = 1;
    int k = 0;
    for (int d = 0; d < bnd; d++) {
        int ia = d - (bnd - (nd_a - 2)), ib = d - (bnd - (nd_b - 2));
        int ea = ia >= 0 ? shape_a[ia] : 1, eb = ib >= 0 ? shape_b[ib] : 1;
        if (ea != eb && ea != 1 && eb != 1)
            return fail(PT_ERR_INVALID,
                        "matmul requires rank >= 2, matching inner dimensions and broadcast-compatible batches");
        int e = ea == 1 ? eb : ea;
        if (e != shape_c[d]) return fail(PT_ERR_INVALID, "matmul output batch shape mismatch");
        if (e == 1) continue;
        g.bshape[k] = e;
        g.bsa[k] = (ia >= 0 && ea != 1) ? (long long)strides_a[ia] : 0;
        g.bsb[k] = (ib >= 0 && eb != 1) ? (long long)strides_b[ib] : 0;
        batch *= e;
        k++;
    }
    g.nbd = k;
    hipStream_t s = stream_of(stream);
    if (batch == 0 || g.M == 0 || g.N == 0) return PT_OK;
    if (g.K == 0) {
        // empty inner product: zeros (host_array_math.phpt:84-85)
        size_t bytes = (size_t)batch * g.M * g.N * dtype_size(dtype);
        k_zero_fill<<<(unsigned)((bytes + 255) / 256), 256, 0, s>>>((uint8_t *)c, bytes);
        PT_LAUNCH_CHECK("matmul zero fill");
        return PT_OK;
    }
    if (batch > 65535LL * 65535LL) return fail(PT_ERR_INVALID, "matmul batch too large");
    g.a = a;
    g.b = b;
    g.c = c;
    g.batch = (int)batch;
    g.a_sm = (long long)strides_a[nd_a - 2];
    g.a_sk = (long long)strides_a[nd_a - 1];
    g.b_sk = (long long)strides_b[nd_b - 2];
    g.b_sn = (long long)strides_b[nd_b - 1];

    // fp32 products with at most 16 columns and k-contiguous A stream A
    // through the small-N kernel (pt_gemm_smalln.hip) unless a tile is forced
    if (dtype == PT_FLOAT32 && g_tile_override < 0 && batch <= 65535 && gemm_smalln_eligible(g)) {
        launch_gemm_smalln(g, s);
        PT_LAUNCH_CHECK("matmul (small-N kernel)");
        counters().mfma_gemm_calls++;
        snprintf(counters().last_matmul, sizeof(counters().last_matmul), "mfma-fp32-smalln");
        return PT_OK;
    }

    const int PKe = dtype == PT_FLOAT32 ? 4 : 8;
    // layout classes: k-contiguous or row/col-contiguous; anything else is
    // read element-wise by the checked kernel
    bool a_kc = g.a_sk == 1 || g.K == 1;
    bool a_rc = g.a_sm == 1 || g.M == 1;
    bool b_kc = g.b_sk == 1 || g.K == 1;
    bool b_rc = g.b_sn == 1 || g.N == 1;
    if (!a_kc && !a_rc) a_kc = true;  // checked path handles arbitrary strides
    if (!b_kc && !b_rc) b_kc = true;
    int tile = g_tile_override;
    bool tuned = false;
    if (tile < 0) {
        std::lock_guard<std::mutex> lock(g_tuned_mu);
        auto it = g_tuned.find(tune_key(dtype, g.M, g.N, g.K, batch, g.a_sk == 1, g.b_sk == 1));
        if (it != g_tuned.end()) {
            tile = it->second;
            tuned = true;
        }
    }
    const char *suffix = tuned ? "-tuned" : "";
    if (tile < 0) {
        long long t256 = ((g.M + 255) / 256) * (long long)((g.N + 255) / 256) * batch;
        // mid-size fp32: 128x128 tiles of 8 waves for either layout of B
        // (dZ2 W2^T of config 5, B k-contiguous: 76-78 us against 82-84 us
        // for 128x64 tiles at two workgroups per CU)
        const int mid32 = TILE_128x128_W8;
        tile = (g.M >= 256 && g.N >= 256 && t256 >= 256)
                   ? (dtype == PT_FLOAT32 ? TILE_256x256
                      : g.K % 64 != 0 ? TILE_RING_HALF
                      : dtype == PT_BFLOAT16 ? TILE_RING_DEFAULT : TILE_RING_DEFAULT_F16)
                   : (g.M >= 128 && g.N >= 128) ? (dtype == PT_FLOAT32 ? mid32 : TILE_128x128)
                                                : TILE_64x64;
    }
    // the fp32-only tiles run the 128x128 kernel for 16-bit operands
    if (dtype != PT_FLOAT32 && (tile == TILE_128x128_W8_K2 || tile == TILE_128x64_W4M2 || tile == TILE_128x64_W4M2_K2 ||
                                tile == TILE_F32_RING))
        tile = TILE_128x128;
    auto aligned = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    if (tile >= TILE_RING_FIRST && tile <= TILE_RING_LAST) {
        // LDS-ring kernels: 16-bit operands, whole tiles (256 rows, 256 or
        // 128 columns), K a multiple of gemm_ring_kmul, k-contiguous A, B k-
        // or n-contiguous, 16-byte aligned rows and batch offsets, and C
        // aligned for the epilogue's 4-byte stores
        const int variant = tile - TILE_RING_FIRST;
        const int kmul = gemm_ring_kmul(variant), bn = gemm_ring_bn(variant);
        const bool b_row = g.b_sn == 1, b_col = g.b_sk == 1;
        const long long ldb = b_row ? g.b_sk : g.b_sn;
        // (pitches below 2^22 elements: the whole-line kernel's per-lane
        // byte offsets within a step are 32-bit)
        bool ok = dtype != PT_FLOAT32 && g.a_sk == 1 && (b_row || b_col) && g.M % 256 == 0 && g.N % bn == 0 &&
                  g.K % kmul == 0 && aligned(a) && aligned(b) && ((uintptr_t)c & 3u) == 0 && g.a_sm % 8 == 0 &&
                  ldb % 8 == 0 && g.a_sm <= (1LL << 22) && ldb <= (1LL << 22);
        for (int d = 0; d < g.nbd; d++)
            if (g.bsa[d] % 8 || g.bsb[d] % 8) ok = false;
        long long tiles = (long long)(g.M / 256) * (g.N / bn) * batch;
        if (ok && tiles <= 0x7fffffffLL) {
            g.tiles_m = g.M / 256;
            g.tiles_n = g.N / bn;
            g.remap = tiles % 8 == 0;
            launch_gemm_ring(g, dtype, b_row, variant, dim3((unsigned)tiles), s);
            PT_LAUNCH_CHECK("matmul");
            counters().mfma_gemm_calls++;
            static const char *kKindName[] = {"mfma-lds-ring", "mfma-lds-pingpong", "mfma-lds-wholeline"};
            snprintf(counters().last_matmul, sizeof(counters().last_matmul), "%s%s",
                     kKindName[gemm_ring_kind(variant)], suffix);
            return PT_OK;
        }
        tile = TILE_256x256_DIRECT;
    }
    if (tile == TILE_256x256_DIRECT) {
        // direct-to-LDS kernel: 16-bit operands, whole 256x256 tiles, K a
        // multiple of 64, k-contiguous A, B k- or n-contiguous, 16-byte
        // aligned rows and batch offsets, C aligned for 4-byte stores
        const bool b_row = g.b_sn == 1, b_col = g.b_sk == 1;
        const long long ldb = b_row ? g.b_sk : g.b_sn;
        bool direct = dtype != PT_FLOAT32 && g.a_sk == 1 && (b_row || b_col) && g.M % 256 == 0 &&
                      g.N % 256 == 0 && g.K % 64 == 0 && aligned(a) && aligned(b) && ((uintptr_t)c & 3u) == 0 &&
                      g.a_sm % 8 == 0 && ldb % 8 == 0;
        for (int d = 0; d < g.nbd; d++)
            if (g.bsa[d] % 8 || g.bsb[d] % 8) direct = false;
        long long tiles = (long long)(g.M / 256) * (g.N / 256) * batch;
        if (direct && tiles <= 0x7fffffffLL) {
            g.tiles_m = g.M / 256;
            g.tiles_n = g.N / 256;
            g.remap = tiles % 8 == 0;
            dim3 grid((unsigned)tiles), block(512);
            if (dtype == PT_BFLOAT16) {
                if (b_row) k_gemm_direct<PT_BFLOAT16, false><<<grid, block, 0, s>>>(g);
                else k_gemm_direct<PT_BFLOAT16, true><<<grid, block, 0, s>>>(g);
            } else {
                if (b_row) k_gemm_direct<PT_FLOAT16, false><<<grid, block, 0, s>>>(g);
                else k_gemm_direct<PT_FLOAT16, true><<<grid, block, 0, s>>>(g);
            }
            PT_LAUNCH_CHECK("matmul");
            counters().mfma_gemm_calls++;
            snprintf(counters().last_matmul, sizeof(counters().last_matmul), "mfma-direct-lds%s", suffix);
            return PT_OK;
        }
        tile = TILE_256x256;
    }
    // checked kernels still load whole 16-byte packs that lie inside the
    // matrix when the operand's contiguous stride is 1 and its pitch and
    // batch offsets keep packs aligned
    {
        bool va = aligned(a) && (a_kc ? (g.a_sk == 1 && g.a_sm % PKe == 0) : (g.a_sm == 1 && g.a_sk % PKe == 0));
        bool vb = aligned(b) && (b_kc ? (g.b_sk == 1 && g.b_sn % PKe == 0) : (g.b_sn == 1 && g.b_sk % PKe == 0));
        for (int d = 0; d < g.nbd; d++) {
            if (g.bsa[d] % PKe) va = false;
            if (g.bsb[d] % PKe) vb = false;
        }
        g.vec_a = va;
        g.vec_b = vb;
    }
    // fp32 products of 128 x 128 tiles or more run the ring kernel wherever
    // it takes the operands (16-byte packs, whole 32-k steps); the others
    // keep the 256x256 or 8-wave 128x128 tiles chosen above.  Config 4 fp32
    // at steady state: 3711-3721 us against 3913 us (256x256); the config-5
    // products: G2 64.1 us against 73.3 us, dW2 69.8 against 78.0 us.
    if (dtype == PT_FLOAT32 && g_tile_override < 0 && !tuned && (tile == TILE_256x256 || tile == TILE_128x128_W8)) {
        GemmArgs whole = g;
        whole.ksplit = 1;
        if (gemm_f32r_eligible(whole, a_kc, b_kc)) tile = TILE_F32_RING;
    }
    int bm = kTiles[tile].bm, bn = kTiles[tile].bn;
    const int BK = (dtype == PT_FLOAT32 ? 16 : 32) * kTiles[tile].kmul;
    bool vec_ok = aligned(a) && aligned(b);
    // vector (unchecked) loads need whole tiles, 16-byte aligned rows and
    // batch offsets that keep that alignment
    bool check = !(g.M % bm == 0 && g.N % bn == 0 && g.K % BK == 0 && vec_ok);
    if (!check) {
        long long lda = a_kc ? g.a_sm : g.a_sk, ldb = b_kc ? g.b_sn : g.b_sk;
        if ((a_kc ? g.a_sk : g.a_sm) != 1 || (b_kc ? g.b_sk : g.b_sn) != 1) check = true;
        if (lda % PKe || ldb % PKe) check = true;
        for (int d = 0; d < g.nbd; d++)
            if (g.bsa[d] % PKe || g.bsb[d] % PKe) check = true;
    }
    long long total_tiles = (long long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * batch;
    g.remap = total_tiles % 8 == 0;
    if (total_tiles > 0x7fffffffLL) return fail(PT_ERR_INVALID, "matmul grid too large");
    // split-K when the tiles cannot give every CU a workgroup and K is
    // long: about 512 workgroups of K chunks (each at least 4 K steps)
    // write fp32 partials, then one ordered sum per output element
    g.ksplit = 1;
    g.k_chunk = g.K;
    g.partial = nullptr;
    if (total_tiles < 256 && g.K >= 8 * BK) {
        // whole rounds: about 2 workgroups per CU, never a partial second round
        long long want = (tile == TILE_F32_RING ? splitk_ring_workgroups() : splitk_workgroups()) / total_tiles;
        long long max_split = g.K / (4 * BK);
        int ks = (int)(want < max_split ? want : max_split);
        if (ks > 64) ks = 64;
        if (ks > 1) {
            int chunk = (g.K + ks - 1) / ks;
            chunk = (chunk + BK - 1) / BK * BK;
            ks = (g.K + chunk - 1) / chunk;
            if (ks > 1) {
                const size_t count = (size_t)batch * g.M * g.N;
                PT_TRY(scratch_alloc((void **)&g.partial, sizeof(float) * count * (size_t)ks, s));
                g.ksplit = ks;
                g.k_chunk = chunk;
            }
        }
    }
    const bool f32ring = dtype == PT_FLOAT32 && tile == TILE_F32_RING && gemm_f32r_eligible(g, a_kc, b_kc);
    switch (dtype) {
    case PT_BFLOAT16: launch_dt<PT_BFLOAT16>(g, tile, a_kc, b_kc, check, s); break;
    case PT_FLOAT16: launch_dt<PT_FLOAT16>(g, tile, a_kc, b_kc, check, s); break;
    default: launch_dt<PT_FLOAT32>(g, tile, a_kc, b_kc, check, s); break;
    }
    if (g.ksplit > 1) {
        hipError_t e1 = hipGetLastError();
        const size_t count = (size_t)batch * g.M * g.N;
        // four outputs per thread when whole 16-byte packs of every chunk line up
        const bool v4 = count % 4 == 0 && ((uintptr_t)g.partial & 15u) == 0;
        const unsigned blocks = (unsigned)(((v4 ? count / 4 : count) + 255) / 256);
#define PT_SPLITK_SUM(DTV)                                                                          \
    do {                                                                                            \
        if (v4) k_splitk_reduce<DTV, 4><<<blocks, 256, 0, s>>>(g.partial, c, count, g.ksplit);     \
        else k_splitk_reduce<DTV, 1><<<blocks, 256, 0, s>>>(g.partial, c, count, g.ksplit);        \
    } while (0)
        switch (dtype) {
        case PT_BFLOAT16: PT_SPLITK_SUM(PT_BFLOAT16); break;
        case PT_FLOAT16: PT_SPLITK_SUM(PT_FLOAT16); break;
        default: PT_SPLITK_SUM(PT_FLOAT32); break;
        }
#undef PT_SPLITK_SUM
        hipError_t e2 = hipGetLastError();
        scratch_free(g.partial, s);
        PT_TRY(check_hip(e1, "matmul (split-K partials)"));
        PT_TRY(check_hip(e2, "matmul (split-K sum)"));
        counters().mfma_gemm_calls++;
        snprintf(counters().last_matmul, sizeof(counters().last_matmul), "%s%s",
                 f32ring ? "mfma-fp32-ring-splitk" : dtype == PT_FLOAT32 ? "mfma-fp32-splitk" : "mfma-low-precision-splitk",
                 suffix);
        return PT_OK;
    }
    PT_LAUNCH_CHECK("matmul");
    counters().mfma_gemm_calls++;
    snprintf(counters().last_matmul, sizeof(counters().last_matmul), "%s%s",
             f32ring ? "mfma-fp32-ring" : dtype == PT_FLOAT32 ? "mfma-fp32" : "mfma-low-precision", suffix);
    return PT_OK;
}

pt_status pt_matmul_tune(const void *a, const void *b, void *c, int dtype,
                         const int *shape_a, const size_t *strides_a, int nd_a,
                         const int *shape_b, const size_t *strides_b, int nd_b,
                         const int *shape_c, int nd_c, int *tiles, float *median_ms,
                         int max_candidates, int *count, int *selected, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (nd_a < 2 || nd_b < 2 || nd_c < 2 || !count || !selected)
        return fail(PT_ERR_INVALID, "matmul tuning needs rank >= 2 operands and result slots");
    const int M = shape_a[nd_a - 2], K = shape_a[nd_a - 1], N = shape_b[nd_b - 1];
    // the reference tunes its cuBLASLt range only (1e7 <= M*N*K,
    // matmul_kernels.cu:336-456)
    if ((double)M * (double)N * (double)K < 1e7)
        return fail(PT_ERR_INVALID, "matmul is too small for autotuning (M*N*K below 1e7)");
    long long batch = 1;
    for (int d = 0; d < nd_c - 2; d++) batch *= shape_c[d];
    const bool a_k1 = strides_a[nd_a - 1] == 1, b_k1 = strides_b[nd_b - 2] == 1;
    static const int kFp32[] = {TILE_256x128, TILE_128x128, TILE_64x64, TILE_256x256, TILE_256x256_K2,
                                TILE_256x128_W8, TILE_128x128_W8, TILE_128x128_W8_K2, TILE_128x64_W4M2,
                                TILE_128x64_W4M2_K2, TILE_F32_RING};
    static const int kHalf[] = {TILE_256x128, TILE_128x128, TILE_64x64, TILE_256x256, TILE_256x256_K2,
                                TILE_256x256_DIRECT, TILE_256x128_W8, TILE_128x128_W8, TILE_RING_DEFAULT,
                                TILE_RING_HALF, TILE_RING_FIRST + 12, TILE_RING_FIRST + 7, TILE_RING_FIRST + 15};
    const int *cands = dtype == PT_FLOAT32 ? kFp32 : kHalf;
    const int ncand = dtype == PT_FLOAT32 ? (int)(sizeof(kFp32) / sizeof(int)) : (int)(sizeof(kHalf) / sizeof(int));
    hipStream_t s = stream_of(stream);
    hipEvent_t e0, e1;
    PT_TRY(check_hip(hipEventCreate(&e0), "tuning event"));
    PT_TRY(check_hip(hipEventCreate(&e1), "tuning event"));
    const int saved = g_tile_override;
    pt_status st = PT_OK;
    int n = 0, best = -1;
    float best_ms = 0.0f;
    for (int ci = 0; ci < ncand && st == PT_OK; ci++) {
        g_tile_override = cands[ci];
        st = pt_matmul(a, b, c, dtype, shape_a, strides_a, nd_a, shape_b, strides_b, nd_b, shape_c, nd_c, stream);
        float times[5];
        for (int r = 0; r < 5 && st == PT_OK; r++) {
            st = check_hip(hipEventRecord(e0, s), "tuning event");
            if (st == PT_OK)
                st = pt_matmul(a, b, c, dtype, shape_a, strides_a, nd_a, shape_b, strides_b, nd_b, shape_c, nd_c,
                               stream);
            if (st == PT_OK) st = check_hip(hipEventRecord(e1, s), "tuning event");
            if (st == PT_OK) st = check_hip(hipEventSynchronize(e1), "tuning wait");
            if (st == PT_OK) st = check_hip(hipEventElapsedTime(&times[r], e0, e1), "tuning time");
        }
        if (st != PT_OK) break;
        std::sort(times, times + 5);
        if (n < max_candidates && tiles && median_ms) {
            tiles[n] = cands[ci];
            median_ms[n] = times[2];
        }
        if (best < 0 || times[2] < best_ms) {
            best = n;
            best_ms = times[2];
        }
        n++;
    }
    g_tile_override = saved;
    (void)hipEventDestroy(e0);  // cleanup: the timing status is what counts
    (void)hipEventDestroy(e1);
    PT_TRY(st);
    *count = n < max_candidates ? n : max_candidates;
    *selected = best;
    {
        std::lock_guard<std::mutex> lock(g_tuned_mu);
        g_tuned[tune_key(dtype, M, N, K, batch, a_k1, b_k1)] = cands[best];
    }
    // the tuned choice runs once more, so `c` holds its product
    return pt_matmul(a, b, c, dtype, shape_a, strides_a, nd_a, shape_b, strides_b, nd_b, shape_c, nd_c, stream);
}

}  // extern "C"
