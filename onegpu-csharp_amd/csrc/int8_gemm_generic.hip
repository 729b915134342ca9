// The generic MFMA int8 product: any alignment of any operand (bytes are gathered one by one where a row is not
// aligned), any M, N, K, both layouts of B. Same arithmetic as the fast tiled kernel (int8_gemm.hip): operands in the
// signed domain, v_mfma_i32_16x16x64_i8, zero points applied from row and column byte sums at the store. 128 x 128
// tiles, 4 waves of 64 x 64. Used when an operand's rows are not aligned for the fast kernel's vector loads.
#include "og_internal.hpp"

namespace og {

typedef int32_t v4i __attribute__((ext_vector_type(4)));


constexpr int GBK = 64;  // k per step: one v_mfma_i32_16x16x64_i8

// Position of 16-byte chunk q of LDS row r: chunks are XOR-swizzled by bits 1-2 of the row so that the 16 rows a
// fragment read touches (rows r..r+15, one chunk each) spread over all banks for both 32- and 64-bank LDS.
__device__ __forceinline__ int gswz(int r, int q) { return (q ^ ((r >> 1) ^ (r >> 2))) & 3; }

// 16 bytes of one k-contiguous row starting at k, bytes at k >= K (or the whole row when !row_ok) as zero, others
// moved to the signed domain by `flip` (0 or 0x80808080).
__device__ __forceinline__ uint4 gload_row16(const uint8_t *row, int32_t k, int32_t K, bool row_ok, bool vec_ok,
                                            uint32_t flip)
{
    uint4 v = make_uint4(0, 0, 0, 0);
    if (!row_ok) return v;
    if (vec_ok && k + 16 <= K) {
        v = *reinterpret_cast<const uint4 *>(row + k);
        v.x ^= flip; v.y ^= flip; v.z ^= flip; v.w ^= flip;
        return v;
    }
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; e++) {
        if (k + e < K) w[e >> 2] |= ((uint32_t)row[k + e] ^ (flip & 0xFFu)) << ((e & 3) * 8);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Four consecutive columns n..n+3 of one row of a K x N operand (byte j = column n + j), zero outside the product.
__device__ __forceinline__ uint32_t gload_cols4(const uint8_t *row, int32_t n, int32_t N, bool row_ok, bool vec_ok,
                                               uint32_t flip)
{
    if (!row_ok) return 0u;
    if (vec_ok && n + 4 <= N) return *reinterpret_cast<const uint32_t *>(row + n) ^ flip;
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (n + e < N) w |= ((uint32_t)row[n + e] ^ (flip & 0xFFu)) << (e * 8);
    }
    return w;
}

// BM x BN tile per workgroup of WM x WN waves; each wave owns (BM / WM) x (BN / WN) outputs as 16 x 16 fragments.
template <int BM, int BN, int WM, int WN, bool TRANS_B>
struct GenCfg {
    static constexpr int THREADS = 64 * WM * WN;
    static constexpr int FM = BM / WM / 16;
    static constexpr int FN = BN / WN / 16;
    static constexpr int A_CHUNKS = BM * 4 / THREADS;                          // 16-byte chunks of A per thread
    static constexpr int B_CHUNKS = BN * 4 / THREADS;                          // (transposed B) chunks per thread
    static constexpr int B_COLGROUPS = BN / 4;                                 // (K x N B) 4-column groups
    static constexpr int B_KGROUPS = THREADS / B_COLGROUPS;                    // k groups across threads
    static constexpr int B_ROWS = GBK / B_KGROUPS;                              // k rows per thread (multiple of 4)
    static_assert(A_CHUNKS >= 1 && (BM * 4) % THREADS == 0, "A staging");
    static_assert(TRANS_B ? (B_CHUNKS >= 1 && (BN * 4) % THREADS == 0) : (B_ROWS % 8 == 0 && B_ROWS <= 16), "B staging");
};

template <int BM, int BN, int WM, int WN, bool TRANS_B, bool SUM_A, bool SUM_B>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_generic(GemmArgs g, int32_t tiles_n, int32_t tiles_m)
{
    using C = GenCfg<BM, BN, WM, WN, TRANS_B>;
    __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * GBK];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * GBK];
    __shared__ int32_t RowSum[SUM_A ? BM : 1];
    __shared__ int32_t ColSum[SUM_B ? BN : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int i16 = lane & 15, g4 = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;

    // Tile order: consecutive workgroups go to different XCDs (round robin), so remap the id so that each XCD gets a
    // contiguous run of tiles, then walk that run in groups of 8 row-tiles so that concurrent tiles share A and B rows.
    const int64_t tiles = (int64_t)tiles_n * tiles_m;
    const int64_t nblocks = tiles * g.batch;
    int64_t bid = blockIdx.x;
    if ((nblocks & 7) == 0) bid = (bid & 7) * (nblocks >> 3) + (bid >> 3);
    const int32_t batch = (int32_t)(bid / tiles);
    const int64_t t = bid % tiles;
    int32_t tm, tn;
    {
        const int32_t GROUP = 8;
        int64_t per_group = (int64_t)GROUP * tiles_n;
        int64_t grp = t / per_group;
        int32_t first_m = (int32_t)(grp * GROUP);
        int32_t gsize = min(tiles_m - first_m, GROUP);
        int64_t in = t % per_group;
        tm = first_m + (int32_t)(in % gsize);
        tn = (int32_t)(in / gsize);
    }
    const int32_t m0 = tm * BM, n0 = tn * BN;

    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    const uint32_t flip_a = a_signed ? 0u : 0x80808080u, flip_b = b_signed ? 0u : 0x80808080u;
    const uint8_t *A = g.A + batch * g.strideA;
    const uint8_t *B = g.B + batch * g.strideB;
    const bool vec_a = ((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 15) == 0;
    const bool vec_b = TRANS_B ? (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 15) == 0)
                               : (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 3) == 0);

    if (SUM_A) for (int i = tid; i < BM; i += C::THREADS) RowSum[i] = 0;
    if (SUM_B) for (int i = tid; i < BN; i += C::THREADS) ColSum[i] = 0;

    // Staging registers and byte-sum partials. A thread stages the same rows / columns at every k step.
    uint4 ra[C::A_CHUNKS];
    int32_t sa[C::A_CHUNKS];
    constexpr int RB = TRANS_B ? C::B_CHUNKS : C::B_ROWS;
    uint32_t rbw[TRANS_B ? 1 : C::B_ROWS];
    uint4 rbv[TRANS_B ? C::B_CHUNKS : 1];
    int32_t sb[TRANS_B ? C::B_CHUNKS : 4];
#pragma unroll
    for (int i = 0; i < C::A_CHUNKS; i++) sa[i] = 0;
#pragma unroll
    for (int i = 0; i < (TRANS_B ? C::B_CHUNKS : 4); i++) sb[i] = 0;
    (void)RB;

    auto load_tile = [&](int32_t k0) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            int c = tid + C::THREADS * i, r = c >> 2, q = c & 3;
            int32_t gm = m0 + r;
            ra[i] = gload_row16(A + (int64_t)gm * g.lda, k0 + 16 * q, g.K, gm < g.M, vec_a, flip_a);
        }
        if (TRANS_B) {
#pragma unroll
            for (int i = 0; i < C::B_CHUNKS; i++) {
                int c = tid + C::THREADS * i, r = c >> 2, q = c & 3;
                int32_t gn = n0 + r;
                rbv[i] = gload_row16(B + (int64_t)gn * g.ldb, k0 + 16 * q, g.K, gn < g.N, vec_b, flip_b);
            }
        } else {
            int cg = tid % C::B_COLGROUPS, kg = tid / C::B_COLGROUPS;
            int32_t gn = n0 + 4 * cg;
#pragma unroll
            for (int r = 0; r < C::B_ROWS; r++) {
                int32_t gk = k0 + kg * C::B_ROWS + r;
                rbw[r] = gload_cols4(B + (int64_t)gk * g.ldb, gn, g.N, gk < g.K, vec_b, flip_b);
            }
        }
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            int c = tid + C::THREADS * i, r = c >> 2, q = c & 3;
            *reinterpret_cast<uint4 *>(&As[buf][r * GBK + 16 * gswz(r, q)]) = ra[i];
            if (SUM_A) sa[i] = dot4(ra[i].w, 0x01010101u, dot4(ra[i].z, 0x01010101u,
                                    dot4(ra[i].y, 0x01010101u, dot4(ra[i].x, 0x01010101u, sa[i]))));
        }
        if (TRANS_B) {
#pragma unroll
            for (int i = 0; i < C::B_CHUNKS; i++) {
                int c = tid + C::THREADS * i, r = c >> 2, q = c & 3;
                *reinterpret_cast<uint4 *>(&Bs[buf][r * GBK + 16 * gswz(r, q)]) = rbv[i];
                if (SUM_B) sb[i] = dot4(rbv[i].w, 0x01010101u, dot4(rbv[i].z, 0x01010101u,
                                        dot4(rbv[i].y, 0x01010101u, dot4(rbv[i].x, 0x01010101u, sb[i]))));
            }
        } else {
            int cg = tid % C::B_COLGROUPS, kg = tid / C::B_COLGROUPS;
            // B_ROWS rows x 4 columns -> per column B_ROWS bytes of consecutive k.
            uint32_t col[4][C::B_ROWS / 4];
#pragma unroll
            for (int b4 = 0; b4 < C::B_ROWS / 4; b4++)
                transpose4x4(rbw[4 * b4], rbw[4 * b4 + 1], rbw[4 * b4 + 2], rbw[4 * b4 + 3], col[0][b4], col[1][b4],
                             col[2][b4], col[3][b4]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                int n = 4 * cg + j;
                int kb = kg * C::B_ROWS;  // first k byte of this thread's run
                if constexpr (C::B_ROWS == 16) {
                    *reinterpret_cast<uint4 *>(&Bs[buf][n * GBK + 16 * gswz(n, kb >> 4)]) =
                        make_uint4(col[j][0], col[j][1], col[j][2], col[j][3]);
                } else {  // 8 rows: one half of a 16-byte chunk
                    *reinterpret_cast<uint2 *>(&Bs[buf][n * GBK + 16 * gswz(n, kb >> 4) + (kb & 8)]) =
                        make_uint2(col[j][0], col[j][1]);
                }
                if (SUM_B) {
#pragma unroll
                    for (int b4 = 0; b4 < C::B_ROWS / 4; b4++) sb[j] = dot4(col[j][b4], 0x01010101u, sb[j]);
                }
            }
        }
    };

    v4i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; i++)
#pragma unroll
        for (int j = 0; j < C::FN; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    const int32_t nk = (g.K + GBK - 1) / GBK;
    if (nk > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    for (int32_t kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_tile((kt + 1) * GBK);
        v4i af[C::FM], bf[C::FN];
#pragma unroll
        for (int i = 0; i < C::FM; i++) {
            int r = wm * (BM / WM) + 16 * i + i16;
            af[i] = *reinterpret_cast<const v4i *>(&As[cur][r * GBK + 16 * gswz(r, g4)]);
        }
#pragma unroll
        for (int j = 0; j < C::FN; j++) {
            int n = wn * (BN / WN) + 16 * j + i16;
            bf[j] = *reinterpret_cast<const v4i *>(&Bs[cur][n * GBK + 16 * gswz(n, g4)]);
        }
#pragma unroll
        for (int i = 0; i < C::FM; i++)
#pragma unroll
            for (int j = 0; j < C::FN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) store_tile(cur ^ 1);
        __syncthreads();
    }

    // Byte sums of this tile's rows and columns, gathered from every thread's staging partials.
    if (SUM_A) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            int c = tid + C::THREADS * i;
            atomicAdd(&RowSum[c >> 2], sa[i]);
        }
    }
    if (SUM_B) {
        if (TRANS_B) {
#pragma unroll
            for (int i = 0; i < C::B_CHUNKS; i++) {
                int c = tid + C::THREADS * i;
                atomicAdd(&ColSum[c >> 2], sb[i]);
            }
        } else {
            int cg = tid % C::B_COLGROUPS;
#pragma unroll
            for (int j = 0; j < 4; j++) atomicAdd(&ColSum[4 * cg + j], sb[j]);
        }
    }
    if (SUM_A || SUM_B) __syncthreads();

    // Store: MFMA 16 x 16 output layout, lane l holds rows 4 * (l / 16) + r, column l % 16.
    const bool za_row = g.flags & OG_GEMM_ZA_PER_ROW, zb_col = g.flags & OG_GEMM_ZB_PER_COL;
    const uint32_t K = (uint32_t)g.K;
#pragma unroll
    for (int j = 0; j < C::FN; j++) {
        int nl = wn * (BN / WN) + 16 * j + i16;
        int32_t n = n0 + nl;
        if (n >= g.N) continue;
        uint32_t wz = (uint32_t)signed_zero(g.ZB, n, zb_col, b_signed);
        uint32_t st = SUM_B ? (uint32_t)ColSum[nl] : 0u;
#pragma unroll
        for (int i = 0; i < C::FM; i++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int ml = wm * (BM / WM) + 16 * i + 4 * g4 + r;
                int32_t m = m0 + ml;
                if (m >= g.M) continue;
                uint32_t zz = (uint32_t)signed_zero(g.ZA, m, za_row, a_signed);
                uint32_t ss = SUM_A ? (uint32_t)RowSum[ml] : 0u;
                uint32_t v = (uint32_t)acc[i][j][r] - wz * ss - zz * st + K * zz * wz;
                store_value(g, batch * g.strideC + (int64_t)m * g.N + n, n, v);
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, bool TRANS_B>
static hipError_t launch_generic_cfg(const GemmArgs &g, hipStream_t s)
{
    int32_t tn = (g.N + BN - 1) / BN, tm = (g.M + BM - 1) / BM;
    int64_t blocks = (int64_t)tn * tm * g.batch;
    if (blocks <= 0) return hipSuccess;
    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    // A byte sum is needed only when the other operand's shifted zero point can be non-zero.
    const bool sum_a = (g.flags & OG_GEMM_ZB) || !b_signed;
    const bool sum_b = (g.flags & OG_GEMM_ZA) || !a_signed;
    dim3 grid((uint32_t)blocks), block(64 * WM * WN);
    if (sum_a && sum_b)
        hipLaunchKernelGGL((k_gemm_generic<BM, BN, WM, WN, TRANS_B, true, true>), grid, block, 0, s, g, tn, tm);
    else if (sum_a)
        hipLaunchKernelGGL((k_gemm_generic<BM, BN, WM, WN, TRANS_B, true, false>), grid, block, 0, s, g, tn, tm);
    else if (sum_b)
        hipLaunchKernelGGL((k_gemm_generic<BM, BN, WM, WN, TRANS_B, false, true>), grid, block, 0, s, g, tn, tm);
    else
        hipLaunchKernelGGL((k_gemm_generic<BM, BN, WM, WN, TRANS_B, false, false>), grid, block, 0, s, g, tn, tm);
    return hipGetLastError();
}

hipError_t launch_gemm_generic(const GemmArgs &g, hipStream_t s, const char **kernel)
{
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    *kernel = "mfma-i8-generic128x128x64";
    return trans_b ? launch_generic_cfg<128, 128, 2, 2, true>(g, s) : launch_generic_cfg<128, 128, 2, 2, false>(g, s);
}

}  // namespace og
