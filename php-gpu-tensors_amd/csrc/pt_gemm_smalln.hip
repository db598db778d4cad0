// fp32 products with at most 16 output columns (C = A B, N <= 16): the
// logits layer of a classifier and its weight gradient.  Such a product
// reads all of A once and does 2 N flops per element of A, so it is bound by
// HBM, not by the matrix cores: a 32x32 MFMA tile would waste most of its
// columns and its few tiles need a K split with a partial buffer.  This
// kernel streams a k-contiguous A once with coalesced 16-byte loads, keeps
// the K x N panel of B in LDS and accumulates on 16x16x4 fp32 MFMAs.
// Launched by pt_matmul (pt_gemm.hip).
#include "pt_gemm.h"

namespace pt {

// ---- A k-contiguous (A(m, k) = a[m * a_sm + k]): a workgroup owns 16 rows
// and its eight waves take interleaved 16-k groups.  Per group a lane loads
// A(m0 + l % 16, k + 4 (l / 16) .. +3) as one 16-byte load (a wave reads 16
// rows x 64 contiguous bytes) and feeds element e to v_mfma_f32_16x16x4_f32
// e, whose k index l / 16 then stands for k + 4 (l / 16) + e; lane l reads
// the matching B(k + 4 (l / 16) + e, l % 16) from LDS.  B sits in LDS in
// chunks of SM_KC k rows of NP = 16 columns (zero past N and past K) with
// a row pitch of 20 floats: the 32 lanes of one LDS cycle read rows four
// apart, which fall 80 words apart, on disjoint banks.  A chunk is one
// pass of the eight waves with all of their loads in flight, so K <= 1024
// costs one memory round trip.  The waves' 16 x 16 partial tiles are summed
// in wave order through LDS.
constexpr int SM_KW = 8;      // waves per workgroup
constexpr int SM_UNROLL = 8;  // 16-k groups in flight per wave
constexpr int SM_KC = SM_KW * SM_UNROLL * 16;  // k rows of B per LDS chunk (80 KiB)
constexpr int SM_PITCH = 20;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <bool VEC>
__global__ __launch_bounds__(64 * SM_KW) void k_gemm_smalln_kc(GemmArgs g)
{
    __shared__ __attribute__((aligned(16))) float bs[SM_KC * SM_PITCH];
    __shared__ float red[SM_KW][16][17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int bidx = blockIdx.y;
    long long oa, ob;
    batch_offsets(g, bidx, oa, ob);
    const float *A = (const float *)g.a + oa;
    const float *B = (const float *)g.b + ob;
    const int m0 = blockIdx.x * 16;
    const int row = min(m0 + (lane & 15), g.M - 1);  // rows past M are read, never stored
    const int kq = 4 * (lane >> 4);                   // this lane's k offset in a group
    const float *arow = A + (long long)row * g.a_sm;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};

    static_assert(SM_KC == SM_KW * SM_UNROLL * 16, "one unrolled pass of the waves covers a chunk");
    for (int k0 = 0; k0 < g.K; k0 += SM_KC) {
        const int kc = min(SM_KC, g.K - k0);
        const int ngroups = (kc + 15) >> 4;
        // this wave's A loads of the chunk, then its share of the B chunk:
        // both in flight before the first wait
        f32x4_t av[SM_UNROLL];
#pragma unroll
        for (int u = 0; u < SM_UNROLL; u++) {
            const int gi = wave + SM_KW * u;
            const int kl = gi * 16 + kq;          // k within the chunk
            if (gi < ngroups && VEC && kl + 4 <= kc) {
                av[u] = *(const f32x4_t *)(arow + k0 + kl);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    av[u][e] = (gi < ngroups && kl + e < kc) ? arow[k0 + kl + e] : 0.0f;
            }
        }
        constexpr int SP = SM_KC * 16 / (64 * SM_KW);
        float stage[SP];
#pragma unroll
        for (int j = 0; j < SP; j++) {
            const int i = threadIdx.x + j * 64 * SM_KW, k = i >> 4, n = i & 15;
            stage[j] = (n < g.N && k < kc) ? B[(long long)(k0 + k) * g.b_sk + (long long)n * g.b_sn] : 0.0f;
        }
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int j = 0; j < SP; j++) {
            const int i = threadIdx.x + j * 64 * SM_KW;
            bs[(i >> 4) * SM_PITCH + (i & 15)] = stage[j];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < SM_UNROLL; u++) {
            const int gi = wave + SM_KW * u;
            if (gi < ngroups) {
                const float *bp = bs + (gi * 16 + kq) * SM_PITCH + (lane & 15);
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][e], bp[e * SM_PITCH], acc, 0, 0, 0);
            }
        }
    }
    // lane l holds C(m0 + 4 (l / 16) + r, l % 16), r = 0..3
#pragma unroll
    for (int r = 0; r < 4; r++) red[wave][4 * (lane >> 4) + r][lane & 15] = acc[r];
    __syncthreads();
    if (threadIdx.x >= 256) return;
    const int mi = threadIdx.x >> 4, n = threadIdx.x & 15, m = m0 + mi;
    float sum = red[0][mi][n];
#pragma unroll
    for (int w = 1; w < SM_KW; w++) sum += red[w][mi][n];
    if (m < g.M && n < g.N) ((float *)g.c)[((size_t)bidx * g.M + m) * g.N + n] = sum;
}

bool gemm_smalln_eligible(const GemmArgs &g)
{
    // m-contiguous A (a transposed operand) keeps the MFMA split-K path: a
    // streaming kernel for it measured no faster (27.9 us against 26.9 us on
    // [1024 x 4096] x [4096 x 10]).  The kernel has no K split, so it also
    // needs one 16-row block per CU at least: a short, long-K product (16 x
    // 65536, 64 x 4096) would stream all of A through a few workgroups,
    // where the split-K path spreads K over about 512.
    return g.N <= 16 && g.a_sk == 1 && (double)g.M * g.K >= (double)(1 << 18) &&
           (long long)((g.M + 15) / 16) * g.batch >= 256;
}

void launch_gemm_smalln(const GemmArgs &g, hipStream_t s)
{
    // 16-byte loads need 16-byte aligned rows and batch offsets
    bool vec = ((uintptr_t)g.a & 15u) == 0 && g.a_sm % 4 == 0;
    for (int d = 0; d < g.nbd; d++)
        if (g.bsa[d] % 4) vec = false;
    const dim3 grid((unsigned)((g.M + 15) / 16), (unsigned)g.batch);
    if (vec) k_gemm_smalln_kc<true><<<grid, 64 * SM_KW, 0, s>>>(g);
    else k_gemm_smalln_kc<false><<<grid, 64 * SM_KW, 0, s>>>(g);
}

}  // namespace pt
