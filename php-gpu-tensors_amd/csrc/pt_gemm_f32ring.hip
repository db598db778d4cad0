// fp32 LDS-ring GEMM for mid-size products: a few hundred 128 x 128 tiles,
// one workgroup per CU, each running the whole K (or one split-K chunk) of
// its tile.  The config-5 classifier step's products (4096 x 1024 x 1024,
// and the weight gradients 1024 x 1024 x 4096 split over K) are this shape.
// Launched by pt_matmul (pt_gemm.hip) for the fp32 ring tile.
#include "pt_gemm.h"

namespace pt {

// 128 x 128 tiles, 4 waves in a 2 x 2 grid of 64 x 64 wave tiles (2 x 2
// blocks of 32 x 32 on v_mfma_f32_32x32x2_f32, one wave per SIMD), K steps
// of 32 through a ring of 4 LDS stages filled by buffer loads to LDS (16
// KiB per operand and stage, 128 KiB in all).  A load is one instruction:
// the step's base address in a scalar buffer resource, a fixed per-lane
// byte offset in a register and the LDS destination in M0, all computed
// outside the loop or by scalar instructions.  With a vector address add
// per load (global_load_lds) the same kernel took 242 us against 229 us
// on 4096 x 1024 x 4096, and 229 us is what it takes with no loads at all.
// Each operand keeps the layout it has in memory:
//   * k-contiguous (A(m, k) = a[m lda + k], or B(k, n) = b[n ldb + k]): a
//     stage row is one tile row's 32 k, one 128-byte line, with its eight
//     16-byte chunks XOR-swizzled by (row / 2) % 8 (logical chunk c sits at
//     position c ^ swizzle), so that a fragment read of 16 rows x 16 bytes
//     touches every LDS bank once.  A load to LDS writes a lane's 16 bytes
//     at the lane's position, so lane L of a load fetches the chunk that
//     belongs at position L % 8 of its row.  A lane reads 4
//     consecutive k of one row with one ds_read_b128.
//   * m- or n-contiguous (A(m, k) = a[k lda + m], B(k, n) = b[k ldb + n]): a
//     stage row is one k's 128 tile rows, 512 bytes, unpadded.  A lane
//     reads 2 adjacent rows at one k with one ds_read_b64 (each half-wave
//     reads 256 contiguous bytes) for the wave's two blocks: block i's row
//     r is the wave's row 2 r + i.
// The 32x32x2 MFMA takes A(row l % 32, k l / 32) and B(k l / 32, col l % 32)
// from lane l.  Per 8-k slice s a wave runs MFMA e = 0..3 on each of its
// four blocks, and MFMA e's k index l / 32 stands for k = 8 s + 4 (l / 32)
// + e: one 16-byte read of a k-contiguous operand supplies all four e, one
// k-row read of the other layout supplies one.  Both operands follow that
// order, so every MFMA pairs A and B at the same k, and each output's sum
// over K runs in one fixed order.
// Per step a wave issues 8 loads of 1 KiB, the loads of step t + NST - 1,
// into the stage that the previous step's barrier freed, and at its own
// barrier waits only for the loads of step t + 1:
//   * NST = 4 (128 KiB of LDS, one workgroup per CU): loads spread over the
//     first 48 of the step's 64 MFMAs; steps t + 2 and t + 3 stay in flight
//     at the barrier, so a load has more than two steps to land;
//   * NST = 2 (64 KiB, two workgroups per CU): loads issued one per MFMA at
//     the start of the step, all landed at its barrier; the other
//     workgroup's waves keep the SIMD busy while these wait.
// Fragments of slice s + 1 are read while slice s runs on the matrix cores.
// Edge tiles: rows past M (columns past N) load the last whole row or
// 16-byte pack instead and are not stored.  K must be a multiple of 16: a K
// chunk that ends half-way through its last 32-k step reads that step's
// loads within the operand's extent (the buffer resource's range) and zeroes
// both operands' fragments of its last two 8-k slices.
template <bool A_KC, bool B_KC, int NST, bool TAIL>
__global__ __launch_bounds__(256, NST == 2 ? 2 : 1) void k_gemm_f32r(GemmArgs g)
{
    constexpr int BM = 128, BN = 128, BK = 32, NS = BK / 8;
    static_assert(NST == 2 || NST == 4, "ring depth");
    constexpr int SE = BM * BK;       // floats per operand stage (16 KiB)
    constexpr int NQ = SE / 256 / 4;  // 1 KiB loads per operand, wave and step
    constexpr int PER = 2 * NQ;       // loads per wave and step
    constexpr int NRA = A_KC ? 2 : 4, NRB = B_KC ? 2 : 4, NR = NRA + NRB;  // fragment reads per slice
    constexpr int GROUP_M = 4;
    static_assert(NQ == 4 && PER == 8 && NS == 4, "load and slice schedule");
    __shared__ __attribute__((aligned(1024))) float lds_a[NST * SE];
    __shared__ __attribute__((aligned(1024))) float lds_b[NST * SE];

    // ---- tile selection (XCD-aware remap + grouped ordering, as k_gemm)
    const int ntile = g.tiles_m * g.tiles_n;
    long long lin = blockIdx.x;
    if (g.remap) {
        const long long total = (long long)ntile * g.batch, per = total / 8;
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
    const int split = blockIdx.y;
    const int kbase = split * g.k_chunk;
    const int Kl = g.ksplit > 1 ? min(g.k_chunk, g.K - kbase) : g.K;
    const float *A = (const float *)g.a + oa + (long long)kbase * g.a_sk;
    const float *B = (const float *)g.b + ob + (long long)kbase * g.b_sk;

    const int lane = threadIdx.x & 63;
    // the wave index as a uniform value: the loads' LDS destinations (M0)
    // are then scalar arithmetic
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // this wave's loads (load q4 of the wave is the workgroup's load q =
    // 4 wave + q4, LDS bytes [1024 q, 1024 q + 1024) of a stage): a fixed
    // per-lane byte offset from a per-step uniform base, so that a load is
    // one instruction with a scalar base and no vector address arithmetic
    uint32_t offa[NQ], offb[NQ];
#pragma unroll
    for (int q4 = 0; q4 < NQ; q4++) {
        const int q = wave * NQ + q4;
        if constexpr (A_KC) {  // rows 8q .. 8q+7
            const int row = 8 * q + lane / 8;
            const int m = min(m0 + row, g.M - 1) - m0;
            offa[q4] = (uint32_t)(((long long)m * g.a_sm + 4 * ((lane % 8) ^ swz_k(row, 8))) * 4);
        } else {  // k rows 2q, 2q+1
            const int m = min(m0 + 4 * (lane % 32), g.M - 4) - m0;
            offa[q4] = (uint32_t)(((long long)(2 * q + lane / 32) * g.a_sk + m) * 4);
        }
        if constexpr (B_KC) {
            const int row = 8 * q + lane / 8;
            const int n = min(n0 + row, g.N - 1) - n0;
            offb[q4] = (uint32_t)(((long long)n * g.b_sn + 4 * ((lane % 8) ^ swz_k(row, 8))) * 4);
        } else {
            const int n = min(n0 + 4 * (lane % 32), g.N - 4) - n0;
            offb[q4] = (uint32_t)(((long long)(2 * q + lane / 32) * g.b_sk + n) * 4);
        }
    }
    // the tile's first element of each operand, and the step strides
    const char *A0 = (const char *)(A + (A_KC ? (long long)m0 * g.a_sm : (long long)m0));
    const char *B0 = (const char *)(B + (B_KC ? (long long)n0 * g.b_sn : (long long)n0));
    const long long sta = (A_KC ? (long long)BK : (long long)BK * g.a_sk) * 4;
    const long long stb = (B_KC ? (long long)BK : (long long)BK * g.b_sk) * 4;
    // a K chunk may end half-way through its last 32-k step (K a multiple
    // of 16): that step's loads reach 16 k past the chunk, and the loads of
    // each step may read only up to the operand's last element (the buffer
    // unit returns zeros past it)
    const int KT = (Kl + BK - 1) / BK;
    // TAIL (K not a multiple of 32): the step whose upper half lies past
    // the chunk (-1: none), compared as a uniform integer so that the check
    // stays a scalar branch.  Without TAIL the kernel has neither this check
    // nor the range limit, which cost its loop 1.1 % on 4096 x 1024 x 4096.
    const int half_step = TAIL && (Kl % BK) != 0 ? KT - 1 : -1;
    const char *endA = (const char *)((const float *)g.a + oa +
                                      (long long)(g.M - 1) * g.a_sm + (long long)(g.K - 1) * g.a_sk + 1);
    const char *endB = (const char *)((const float *)g.b + ob +
                                      (long long)(g.N - 1) * g.b_sn + (long long)(g.K - 1) * g.b_sk + 1);
    auto range_to = [](const char *base, const char *end) {
        const long long r = end - base;
        return (uint32_t)(r <= 0 ? 0 : (r >= 0xffffffffLL ? 0xffffffffLL : r));
    };
    // only the last step can reach past an operand (earlier steps end
    // within the chunk, and rows and columns are clamped): its range is
    // computed once, and a step picks it with a scalar compare
    const uint32_t last_a = range_to(A0 + (long long)(KT - 1) * sta, endA);
    const uint32_t last_b = range_to(B0 + (long long)(KT - 1) * stb, endB);

    // load IDX of step kt into stage J (loads past the last step re-read it:
    // in bounds, never consumed, and every step waits for the same count)
    auto issue = [&](int kt, auto J, auto IDX) {
        constexpr int j = decltype(J)::value % NST, q = decltype(IDX)::value;
        if constexpr (q < NQ) {
            buffer_load_lds16(A0 + (long long)kt * sta, offa[q],
                              (PT_LDS_AS void *)(lds_a + j * SE + (wave * NQ + q) * 256),
                              TAIL && kt >= KT - 1 ? last_a : 0xffffffffu);
        } else {
            constexpr int q2 = q - NQ;
            buffer_load_lds16(B0 + (long long)kt * stb, offb[q2],
                              (PT_LDS_AS void *)(lds_b + j * SE + (wave * NQ + q2) * 256),
                              TAIL && kt >= KT - 1 ? last_b : 0xffffffffu);
        }
    };

    // fragment read bases (LDS byte addresses).  k-contiguous: one per slice
    // (the swizzled chunk depends on it; block 1 is 32 rows on, an
    // immediate, with the same swizzle); the other layout: one base, the
    // k row an immediate.
    const uint32_t la = (uint32_t)(size_t)(PT_LDS_AS const float *)lds_a;
    const uint32_t lb = (uint32_t)(size_t)(PT_LDS_AS const float *)lds_b;
    uint32_t abase[NS], bbase[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        if constexpr (A_KC) {
            const int ra = wm * 64 + (lane & 31);
            abase[s] = la + (uint32_t)(ra * BK + 4 * ((2 * s + (lane >> 5)) ^ swz_k(ra, 8))) * 4u;
        } else {
            abase[s] = la + (uint32_t)(4 * (lane >> 5) * BM + wm * 64 + 2 * (lane & 31)) * 4u;
        }
        if constexpr (B_KC) {
            const int rb = wn * 64 + (lane & 31);
            bbase[s] = lb + (uint32_t)(rb * BK + 4 * ((2 * s + (lane >> 5)) ^ swz_k(rb, 8))) * 4u;
        } else {
            bbase[s] = lb + (uint32_t)(4 * (lane >> 5) * BN + wn * 64 + 2 * (lane & 31)) * 4u;
        }
    }

    // two fragment sets: a k-contiguous operand as one float4 per block
    // (element e), the other layout as one float2 per e (blocks 0 and 1)
    floatx4 fak[2][2], fbk[2][2];
    f32x2v_t fam[2][4], fbm[2][4];
    auto read_one = [&](auto J, auto S, auto SET, auto R) {
        constexpr int j = decltype(J)::value % NST, s = decltype(S)::value, st = decltype(SET)::value;
        constexpr int r = decltype(R)::value;
        if constexpr (r < NRA) {
            if constexpr (A_KC) lds_read_b128<(j * SE + r * 32 * BK) * 4>(fak[st][r], abase[s]);
            else lds_read_b64<(j * SE + (8 * s + r) * BM) * 4>(fam[st][r], abase[0]);
        } else {
            constexpr int rb = r - NRA;
            if constexpr (B_KC) lds_read_b128<(j * SE + rb * 32 * BK) * 4>(fbk[st][rb], bbase[s]);
            else lds_read_b64<(j * SE + (8 * s + rb) * BN) * 4>(fbm[st][rb], bbase[0]);
        }
    };
    // every LDS read of the wave has returned before set SET is used
    auto frag_wait = [&](auto SET) {
        constexpr int st = decltype(SET)::value;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (A_KC && B_KC)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(fak[st][0]), "+v"(fak[st][1]), "+v"(fbk[st][0]), "+v"(fbk[st][1])::"memory");
        else if constexpr (A_KC)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(fak[st][0]), "+v"(fak[st][1]), "+v"(fbm[st][0]), "+v"(fbm[st][1]),
                           "+v"(fbm[st][2]), "+v"(fbm[st][3])::"memory");
        else if constexpr (B_KC)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(fam[st][0]), "+v"(fam[st][1]), "+v"(fam[st][2]), "+v"(fam[st][3]),
                           "+v"(fbk[st][0]), "+v"(fbk[st][1])::"memory");
        else
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(fam[st][0]), "+v"(fam[st][1]), "+v"(fam[st][2]), "+v"(fam[st][3]),
                           "+v"(fbm[st][0]), "+v"(fbm[st][1]), "+v"(fbm[st][2]), "+v"(fbm[st][3])::"memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    // MFMA Q of a slice: e = Q / 4 over the four blocks
    auto mfma_one = [&](auto SET, auto Q) {
        constexpr int st = decltype(SET)::value, q = decltype(Q)::value;
        constexpr int e = q / 4, i = (q / 2) % 2, jj = q % 2;
        float av, bv;
        if constexpr (A_KC) av = fak[st][i][e];
        else av = fam[st][e][i];
        if constexpr (B_KC) bv = fbk[st][jj][e];
        else bv = fbm[st][e][jj];
        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[i][jj], 0, 0, 0);
    };
    // slice S of step kt (stage J): its MFMAs, the next slice's fragment
    // reads (after slice 3: slice 0 of the next step's stage) and, in
    // slices 0-2, the loads of step kt + 3
    auto slice = [&](int kt, auto J, auto S) {
        constexpr int j = decltype(J)::value, s = decltype(S)::value, st = s & 1;
        if constexpr (TAIL && s >= 2) {
            // k 16..31 of a half step past the chunk's end: both operands'
            // fragments are zeroed, so these MFMAs add exact zeros whatever
            // the loads brought (the next row's values, or zeros)
            if (kt == half_step) {
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    if constexpr (A_KC) fak[st][i] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (B_KC) fbk[st][i] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if constexpr (!A_KC) fam[st][e] = (f32x2v_t){0.0f, 0.0f};
                    if constexpr (!B_KC) fbm[st][e] = (f32x2v_t){0.0f, 0.0f};
                }
            }
        }
        static_for<0, 16>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            mfma_one(IC<st>{}, Q);
            if constexpr (q < NR) {
                if constexpr (s + 1 < NS) read_one(J, IC<s + 1>{}, IC<st ^ 1>{}, Q);
                else read_one(IC<j + 1>{}, IC<0>{}, IC<st ^ 1>{}, Q);
            }
            // loads of step kt + NST - 1: spread over slices 0-2 in the
            // 4-stage ring; in the 2-stage ring, one per MFMA at the start of
            // the step, so that they have most of the step to land
            constexpr int slot = s * 16 + q;
            constexpr int SP = NST > 2 ? 6 : 1, OFF = NST > 2 ? 2 : 0;
            if constexpr (s < NS - 1 && slot % SP == OFF && slot / SP < PER)
                issue(min(kt + NST - 1, KT - 1), IC<j + NST - 1>{}, IC<slot / SP>{});
            __builtin_amdgcn_sched_barrier(0);
        });
        frag_wait(IC<st ^ 1>{});
    };

    // prologue: steps 0 .. 2 in flight, step 0 landed for everyone
    static_for<0, NST - 1>([&](auto P) {
        constexpr int p = decltype(P)::value;
        static_for<0, PER>([&](auto Q) { issue(min(p, KT - 1), P, Q); });
    });
    ring_wait<(NST - 2) * PER>();
    ring_barrier();
    static_for<0, NR>([&](auto R) { read_one(IC<0>{}, IC<0>{}, IC<0>{}, R); });
    frag_wait(IC<0>{});
    for (int kt0 = 0; kt0 < KT; kt0 += NST) {
        static_for<0, NST>([&](auto J) {
            const int kt = kt0 + decltype(J)::value;
            if (kt < KT) {  // uniform branch
                slice(kt, J, IC<0>{});
                slice(kt, J, IC<1>{});
                slice(kt, J, IC<2>{});
                ring_wait<(NST - 2) * PER>();  // this wave's loads of step kt + 1 landed
                ring_barrier();        // ... everyone's; step kt's stage is free
                slice(kt, J, IC<3>{});
            }
        });
    }
    ring_wait<0>();  // no load may still target LDS when the workgroup ends

    // ---- epilogue: lane holds column l % 32 and rows 8 (r / 4) + 4 (l / 32)
    // + r % 4 of each 32 x 32 block
    const size_t mn = (size_t)g.M * (size_t)g.N;
    float *out = g.ksplit > 1 ? g.partial + ((size_t)split * g.batch + bidx) * mn : (float *)g.c + (size_t)bidx * mn;
    const bool pairs = ((uintptr_t)out & 7u) == 0 && (g.N & 1) == 0;  // 8-byte stores of column pairs
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int rho = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int m = m0 + wm * 64 + (A_KC ? 32 * i + rho : 2 * rho + i);
            if (m >= g.M) continue;
            float *orow = out + (size_t)m * g.N;
            if constexpr (B_KC) {
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    const int n = n0 + wn * 64 + 32 * jj + (lane & 31);
                    if (n < g.N) orow[n] = acc[i][jj][r];
                }
            } else {
                const int n = n0 + wn * 64 + 2 * (lane & 31);
                if (pairs && n + 1 < g.N) {
                    const f32x2v_t v = {acc[i][0][r], acc[i][1][r]};
                    *(f32x2v_t *)(orow + n) = v;
                } else {
                    if (n < g.N) orow[n] = acc[i][0][r];
                    if (n + 1 < g.N) orow[n + 1] = acc[i][1][r];
                }
            }
        }
}

bool gemm_f32r_eligible(const GemmArgs &g, bool a_kc, bool b_kc)
{
    // 16-byte packs along each operand's contiguous dimension (vec_a /
    // vec_b: contiguous stride 1, pitch and batch offsets multiples of 4,
    // aligned base), K a multiple of 16 (a last half step of 32 is
    // zero-filled; split chunks are whole steps), for an m- or n-contiguous operand a
    // whole last pack to clamp edge loads to, and pitches that keep a lane's
    // byte offset within a step (at most 127 pitches) in 32 bits
    constexpr long long kMaxPitch = 1LL << 22;
    return g.vec_a && g.vec_b && g.K % 16 == 0 && (g.ksplit <= 1 || g.k_chunk % 32 == 0) &&
           (a_kc ? (g.a_sk == 1 && g.a_sm <= kMaxPitch) : (g.a_sm == 1 && g.a_sk <= kMaxPitch && g.M % 4 == 0 && g.M >= 4)) &&
           (b_kc ? (g.b_sk == 1 && g.b_sn <= kMaxPitch) : (g.b_sn == 1 && g.b_sk <= kMaxPitch && g.N % 4 == 0 && g.N >= 4));
}

void launch_gemm_f32r(const GemmArgs &g, bool a_kc, bool b_kc, int stages, hipStream_t s)
{
    const dim3 grid((unsigned)((long long)g.tiles_m * g.tiles_n * g.batch), (unsigned)(g.ksplit > 1 ? g.ksplit : 1));
    auto go = [&](auto NSTC, auto TAILC) {
        constexpr int NST = decltype(NSTC)::value;
        constexpr bool TAIL = decltype(TAILC)::value != 0;
        if (a_kc) {
            if (b_kc) k_gemm_f32r<true, true, NST, TAIL><<<grid, 256, 0, s>>>(g);
            else k_gemm_f32r<true, false, NST, TAIL><<<grid, 256, 0, s>>>(g);
        } else {
            if (b_kc) k_gemm_f32r<false, true, NST, TAIL><<<grid, 256, 0, s>>>(g);
            else k_gemm_f32r<false, false, NST, TAIL><<<grid, 256, 0, s>>>(g);
        }
    };
    // a K that ends half-way through a 32-k step runs the 4-stage tail form
    if (g.K % 32 != 0) go(IC<4>{}, IC<1>{});
    else if (stages == 2) go(IC<2>{}, IC<0>{});
    else go(IC<4>{}, IC<0>{});
}

}  // namespace pt
