// int8 products C = (A - za)(B - zb) with int32 wrap-around, for gfx950 (CDNA4).
//
//  - gemm_tiled: the MFMA kernel. Operands are staged through LDS in the signed domain (an unsigned byte u becomes
//    s = u ^ 0x80 = u - 128 and its zero point z becomes z' = z - 128), multiplied with v_mfma_i32_16x16x64_i8, and the
//    zero points are applied once per output from byte sums gathered while staging:
//        sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w'      (exact modulo 2^32)
//    the same rearrangement the reference's packed-dot kernel uses (Int8GemmDot.hlsl:1-11, 134-140). B stored K x N
//    (n contiguous) is transposed 4 x 4 bytes at a time in registers (v_perm_b32) so that every MFMA lane reads 16
//    consecutive k of one column. LDS rows are 64 bytes of k; the four 16-byte chunks of a row are XOR-swizzled so that
//    the 16-byte fragment reads of a wave hit distinct banks.
//  - gemm_portable: plain integer multiply-adds on 64 x 64 tiles; any alignment, any layout. It is the variant
//    Int8GemmOptions.AllowPackedDot = false selects (the reference's "portable" kernel, Int8GemmKernel.hlsl).
#include "og_internal.hpp"

namespace og {

typedef int32_t v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ portable kernel

constexpr int PT = 64;   // tile edge
constexpr int PK = 16;   // k per step

__global__ __launch_bounds__(256) void k_gemm_portable(GemmArgs g, int32_t tiles_n, int32_t tiles_m)
{
    __shared__ int32_t As[PK][PT + 1];
    __shared__ int32_t Bs[PK][PT + 1];
    const int tid = threadIdx.x;
    const int64_t tiles = (int64_t)tiles_n * tiles_m;
    const int64_t bid = blockIdx.x;
    const int32_t batch = (int32_t)(bid / tiles);
    const int64_t t = bid % tiles;
    const int32_t m0 = (int32_t)(t / tiles_n) * PT, n0 = (int32_t)(t % tiles_n) * PT;
    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    const bool za_row = g.flags & OG_GEMM_ZA_PER_ROW, zb_col = g.flags & OG_GEMM_ZB_PER_COL;
    const uint8_t *A = g.A + batch * g.strideA;
    const uint8_t *B = g.B + batch * g.strideB;
    const int tx = tid & 15, ty = tid >> 4;
    uint32_t acc[4][4] = {};

    for (int32_t k0 = 0; k0 < g.K; k0 += PK) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int idx = tid + 256 * e;
            int r = idx / PK, kk = idx % PK;
            int32_t gm = m0 + r, gk = k0 + kk;
            int32_t v = 0;
            if (gm < g.M && gk < g.K) {
                uint8_t b = A[(int64_t)gm * g.lda + gk];
                int32_t z = g.ZA ? (a_signed ? sext8(g.ZA[za_row ? gm : 0]) : (int32_t)g.ZA[za_row ? gm : 0]) : 0;
                v = (a_signed ? sext8(b) : (int32_t)b) - z;
            }
            As[kk][r] = v;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int idx = tid + 256 * e;
            int c, kk;
            if (trans_b) { c = idx / PK; kk = idx % PK; } else { c = idx % PT; kk = idx / PT; }
            int32_t gn = n0 + c, gk = k0 + kk;
            int32_t v = 0;
            if (gn < g.N && gk < g.K) {
                uint8_t b = trans_b ? B[(int64_t)gn * g.ldb + gk] : B[(int64_t)gk * g.ldb + gn];
                int32_t z = g.ZB ? (b_signed ? sext8(g.ZB[zb_col ? gn : 0]) : (int32_t)g.ZB[zb_col ? gn : 0]) : 0;
                v = (b_signed ? sext8(b) : (int32_t)b) - z;
            }
            Bs[kk][c] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < PK; kk++) {
            int32_t a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) { a[i] = As[kk][ty + 16 * i]; b[i] = Bs[kk][tx + 16 * i]; }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] += (uint32_t)(a[i] * b[j]);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; i++) {
        int32_t m = m0 + ty + 16 * i;
        if (m >= g.M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int32_t n = n0 + tx + 16 * j;
            if (n < g.N) store_value(g, batch * g.strideC + (int64_t)m * g.N + n, n, acc[i][j]);
        }
    }
}

hipError_t launch_gemm_portable(const GemmArgs &g, hipStream_t s, const char **kernel)
{
    int32_t tn = (g.N + PT - 1) / PT, tm = (g.M + PT - 1) / PT;
    int64_t blocks = (int64_t)tn * tm * g.batch;
    *kernel = "portable-tile64x64x16";
    if (blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_gemm_portable, dim3((uint32_t)blocks), dim3(256), 0, s, g, tn, tm);
    return hipGetLastError();
}

// ------------------------------------------------------------------ MFMA kernel (aligned operands)

// Position of 16-byte chunk q of LDS row r, for rows of C chunks: q ^ (bits of r). With 64 banks of 4 bytes this makes
// three access patterns conflict-free: a fragment read (16 consecutive rows, one chunk each), an A-staging write
// (consecutive chunks of consecutive rows) and a B-staging write (rows 4c + (s ^ ((c >> 2) & 3)) of 16 lanes c).
template <int C>
__device__ __forceinline__ int chunk_pos(int r, int q)
{
    return q ^ (((r * C) >> 4) & (C - 1));
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// A raw buffer resource over [base, base + bytes): loads past the end return zeros.
__device__ __forceinline__ rsrc_t make_rsrc(const uint8_t *base, int64_t bytes)
{
    uint32_t n = bytes <= 0 ? 0u : (bytes >= 0xFFFFFFFFll ? 0xFFFFFFFFu : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short)0, (int)n, 0x00020000);
}

__device__ __forceinline__ uint4 ld128(rsrc_t r, uint32_t off)
{
    v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

__device__ __forceinline__ uint32_t ld32(rsrc_t r, uint32_t off) { return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }

// Keeps the first `valid` bytes (0..16) of a 16-byte chunk.
__device__ __forceinline__ uint4 keep_bytes(uint4 v, int32_t valid)
{
    auto m = [](int32_t n) -> uint32_t { return n >= 4 ? 0xFFFFFFFFu : (n <= 0 ? 0u : ((1u << (8 * n)) - 1u)); };
    return make_uint4(v.x & m(valid), v.y & m(valid - 4), v.z & m(valid - 8), v.w & m(valid - 12));
}

__device__ __forceinline__ uint4 xor4(uint4 v, uint32_t f) { return make_uint4(v.x ^ f, v.y ^ f, v.z ^ f, v.w ^ f); }

// 4 x 4 byte transpose with the columns taken in a per-lane order: c[s] = column sigma(s) of the rows r0..r3, where the
// first-stage selectors sel_lo / sel_hi name the byte pairs (sigma(0), sigma(1)) and (sigma(2), sigma(3)).
__device__ __forceinline__ void transpose4x4_sel(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t sel_lo,
                                                 uint32_t sel_hi, uint32_t &c0, uint32_t &c1, uint32_t &c2, uint32_t &c3)
{
    uint32_t lo01 = perm(r1, r0, sel_lo), hi01 = perm(r1, r0, sel_hi);
    uint32_t lo23 = perm(r3, r2, sel_lo), hi23 = perm(r3, r2, sel_hi);
    c0 = perm(lo23, lo01, 0x05040100u);
    c1 = perm(lo23, lo01, 0x07060302u);
    c2 = perm(hi23, hi01, 0x05040100u);
    c3 = perm(hi23, hi01, 0x07060302u);
}

// BM x BN x BK tile per workgroup of WM x WN waves; each wave owns (BM / WM) x (BN / WN) outputs as 16 x 16 fragments.
// Every thread stages 16 rows x 4 columns of a K x N operand per stage (so BK = 16 * THREADS / (BN / 4)).
template <int BM, int BN, int BK, int WM, int WN, bool TRANS_B>
struct TileCfg {
    static constexpr int THREADS = 64 * WM * WN;
    static constexpr int C = BK / 16;                         // 16-byte chunks per LDS row
    static constexpr int FM = BM / WM / 16;
    static constexpr int FN = BN / WN / 16;
    static constexpr int KSUB = BK / 64;                      // MFMA k-steps per stage
    static constexpr int A_CHUNKS = BM * C / THREADS;         // 16-byte chunks of A per thread per stage
    static constexpr int B_CHUNKS = BN * C / THREADS;         // (B stored N x K) chunks per thread
    static constexpr int B_COLGROUPS = BN / 4;                // (B stored K x N) 4-column groups
    static constexpr int B_KGROUPS = THREADS / B_COLGROUPS;   // 16-row groups
    static_assert(BM * C % THREADS == 0 && A_CHUNKS >= 1, "A staging");
    static_assert(TRANS_B ? (BN * C % THREADS == 0 && B_CHUNKS >= 1) : (B_KGROUPS * 16 == BK), "B staging");
    static_assert(BK % 64 == 0 && C <= 8, "k per stage");
};

// Requires every row of A (and of B stored N x K) to start on 16 bytes, rows of B stored K x N on 4 bytes, and each
// batch's operands to span less than 2^31 bytes; M, N and K are free (rows and columns past the product read as zero
// through the buffer resources' range checks, k past K is masked in the last stage).
template <int BM, int BN, int BK, int WM, int WN, bool TRANS_B, bool SUM_A, bool SUM_B>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_tiled(GemmArgs g, int32_t tiles_n, int32_t tiles_m)
{
    using T = TileCfg<BM, BN, BK, WM, WN, TRANS_B>;
    constexpr int C = T::C;
    __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * BK];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * BK];
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
    const int32_t lda = g.lda, ldb = g.ldb, K = g.K;

    // This tile's slices of A and B, as byte ranges that end with the product's last valid byte.
    const uint8_t *a_base = g.A + batch * g.strideA + (int64_t)m0 * lda;
    const int64_t a_valid = (int64_t)(min(g.M - m0, BM) - 1) * lda + K;
    const uint8_t *b_base;
    int64_t b_valid;
    if constexpr (TRANS_B) {
        b_base = g.B + batch * g.strideB + (int64_t)n0 * ldb;
        b_valid = (int64_t)(min(g.N - n0, BN) - 1) * ldb + K;
    } else {
        b_base = g.B + batch * g.strideB + n0;
        b_valid = (int64_t)(K - 1) * ldb + ((min(g.N - n0, BN) + 3) & ~3);   // whole dwords (b_dwords_ok)
    }

    if (SUM_A) for (int i = tid; i < BM; i += T::THREADS) RowSum[i] = 0;
    if (SUM_B) for (int i = tid; i < BN; i += T::THREADS) ColSum[i] = 0;

    // A K x N operand: this thread stages rows 16 kg .. 16 kg + 15 of columns 4 cg .. 4 cg + 3 at every stage, and
    // writes column 4 cg + (s ^ xo) at its s-th LDS write (the order that keeps those writes conflict-free).
    const int cg = tid % T::B_COLGROUPS, kg = tid / T::B_COLGROUPS;
    const uint32_t xo = (uint32_t)(cg >> 2) & 3u;
    const uint32_t sg0 = xo, sg1 = 1u ^ xo, sg2 = 2u ^ xo, sg3 = 3u ^ xo;
    const uint32_t sel_lo = sg0 | ((4u + sg0) << 8) | (sg1 << 16) | ((4u + sg1) << 24);
    const uint32_t sel_hi = sg2 | ((4u + sg2) << 8) | (sg3 << 16) | ((4u + sg3) << 24);
    const uint32_t b_row0 = (uint32_t)(16 * kg) * (uint32_t)ldb + 4u * (uint32_t)cg;

    uint4 ra[T::A_CHUNKS];
    int32_t sa[T::A_CHUNKS];
    uint32_t rbw[TRANS_B ? 1 : 16];
    uint4 rbv[TRANS_B ? T::B_CHUNKS : 1];
    int32_t sb[TRANS_B ? T::B_CHUNKS : 4];
#pragma unroll
    for (int i = 0; i < T::A_CHUNKS; i++) sa[i] = 0;
#pragma unroll
    for (int i = 0; i < (TRANS_B ? T::B_CHUNKS : 4); i++) sb[i] = 0;

    auto load_tile = [&](int32_t k0) {
        const rsrc_t ar = make_rsrc(a_base + k0, a_valid - k0);
#pragma unroll
        for (int i = 0; i < T::A_CHUNKS; i++) {
            const int c = tid + T::THREADS * i, r = c / C, q = c % C;
            ra[i] = ld128(ar, (uint32_t)r * (uint32_t)lda + 16u * q);
        }
        if constexpr (TRANS_B) {
            const rsrc_t br = make_rsrc(b_base + k0, b_valid - k0);
#pragma unroll
            for (int i = 0; i < T::B_CHUNKS; i++) {
                const int c = tid + T::THREADS * i, r = c / C, q = c % C;
                rbv[i] = ld128(br, (uint32_t)r * (uint32_t)ldb + 16u * q);
            }
        } else {
            const rsrc_t br = make_rsrc(b_base + (int64_t)k0 * ldb, b_valid - (int64_t)k0 * ldb);
#pragma unroll
            for (int r = 0; r < 16; r++) rbw[r] = ld32(br, b_row0 + (uint32_t)r * (uint32_t)ldb);
        }
    };

    // Moves the staged bytes to the signed domain and, in a stage that runs past K, zeroes the bytes beyond it.
    auto fix_tile = [&](int32_t k0, bool tail) {
#pragma unroll
        for (int i = 0; i < T::A_CHUNKS; i++) ra[i] = xor4(ra[i], flip_a);
        if constexpr (TRANS_B) {
#pragma unroll
            for (int i = 0; i < T::B_CHUNKS; i++) rbv[i] = xor4(rbv[i], flip_b);
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) rbw[r] ^= flip_b;
        }
        if (tail) {
#pragma unroll
            for (int i = 0; i < T::A_CHUNKS; i++) ra[i] = keep_bytes(ra[i], K - (k0 + 16 * ((tid + T::THREADS * i) % C)));
            if constexpr (TRANS_B) {
#pragma unroll
                for (int i = 0; i < T::B_CHUNKS; i++) rbv[i] = keep_bytes(rbv[i], K - (k0 + 16 * ((tid + T::THREADS * i) % C)));
            } else {
#pragma unroll
                for (int r = 0; r < 16; r++) rbw[r] = (k0 + 16 * kg + r < K) ? rbw[r] : 0u;
            }
        }
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < T::A_CHUNKS; i++) {
            const int c = tid + T::THREADS * i, r = c / C, q = c % C;
            *reinterpret_cast<uint4 *>(&As[buf][r * BK + 16 * chunk_pos<C>(r, q)]) = ra[i];
            if (SUM_A) sa[i] = dot4(ra[i].w, 0x01010101u, dot4(ra[i].z, 0x01010101u,
                                    dot4(ra[i].y, 0x01010101u, dot4(ra[i].x, 0x01010101u, sa[i]))));
        }
        if constexpr (TRANS_B) {
#pragma unroll
            for (int i = 0; i < T::B_CHUNKS; i++) {
                const int c = tid + T::THREADS * i, r = c / C, q = c % C;
                *reinterpret_cast<uint4 *>(&Bs[buf][r * BK + 16 * chunk_pos<C>(r, q)]) = rbv[i];
                if (SUM_B) sb[i] = dot4(rbv[i].w, 0x01010101u, dot4(rbv[i].z, 0x01010101u,
                                        dot4(rbv[i].y, 0x01010101u, dot4(rbv[i].x, 0x01010101u, sb[i]))));
            }
        } else {
            uint32_t col[4][4];   // col[s][b4]: bytes 4 b4 .. 4 b4 + 3 (k) of column 4 cg + (s ^ xo)
#pragma unroll
            for (int b4 = 0; b4 < 4; b4++)
                transpose4x4_sel(rbw[4 * b4], rbw[4 * b4 + 1], rbw[4 * b4 + 2], rbw[4 * b4 + 3], sel_lo, sel_hi,
                                 col[0][b4], col[1][b4], col[2][b4], col[3][b4]);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int n = 4 * cg + (int)((uint32_t)s ^ xo);
                *reinterpret_cast<uint4 *>(&Bs[buf][n * BK + 16 * chunk_pos<C>(n, kg)]) =
                    make_uint4(col[s][0], col[s][1], col[s][2], col[s][3]);
                if (SUM_B) {
#pragma unroll
                    for (int b4 = 0; b4 < 4; b4++) sb[s] = dot4(col[s][b4], 0x01010101u, sb[s]);
                }
            }
        }
    };

    v4i acc[T::FM][T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; i++)
#pragma unroll
        for (int j = 0; j < T::FN; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    // One stage's MFMAs on LDS buffer `buf`. The B fragments stay in registers for the stage, the A fragment is read
    // one ahead, and `between` (the next stage's staging: signed-domain fix-up, transpose, LDS writes, next loads) is
    // placed halfway through so its VALU and LDS work runs while the MFMA pipe is busy.
    auto compute = [&](int buf, auto &&between) {
#pragma unroll
        for (int ks = 0; ks < T::KSUB; ks++) {
            v4i bf[T::FN];
#pragma unroll
            for (int j = 0; j < T::FN; j++) {
                const int n = wn * (BN / WN) + 16 * j + i16;
                bf[j] = *reinterpret_cast<const v4i *>(&Bs[buf][n * BK + 16 * chunk_pos<C>(n, 4 * ks + g4)]);
            }
            auto read_a = [&](int i) {
                const int r = wm * (BM / WM) + 16 * i + i16;
                return *reinterpret_cast<const v4i *>(&As[buf][r * BK + 16 * chunk_pos<C>(r, 4 * ks + g4)]);
            };
            v4i a_cur = read_a(0);
#pragma unroll
            for (int i = 0; i < T::FM; i++) {
                const v4i a_next = (i + 1 < T::FM) ? read_a(i + 1) : a_cur;
#pragma unroll
                for (int j = 0; j < T::FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_cur, bf[j], acc[i][j], 0, 0, 0);
                if (ks == T::KSUB - 1 && i == T::FM / 2 - 1) between();
                a_cur = a_next;
            }
        }
    };

    // Stages 0 .. nfull - 1 lie wholly inside K; a last partial stage (K % BK != 0) is masked when it is staged.
    const int32_t nk = (K + BK - 1) / BK, nfull = K / BK;
    if (nk > 0) {
        load_tile(0);
        fix_tile(0, nfull == 0);
        store_tile(0);
        if (nk > 1) load_tile(BK);
    }
    __syncthreads();
    // Steady state: stage kt + 1 (already loaded) is full, stage kt + 2 exists.
    for (int32_t kt = 0; kt + 2 < nk; kt++) {
        compute(kt & 1, [&] {
            fix_tile((kt + 1) * BK, false);
            store_tile((kt + 1) & 1);
            load_tile((kt + 2) * BK);
        });
        __syncthreads();
    }
    if (nk >= 2) {
        const int32_t kt = nk - 2;
        compute(kt & 1, [&] {
            fix_tile((kt + 1) * BK, kt + 1 >= nfull);
            store_tile((kt + 1) & 1);
        });
        __syncthreads();
    }
    if (nk >= 1) compute((nk - 1) & 1, [] {});

    // Byte sums of this tile's rows and columns, gathered from every thread's staging partials.
    if (SUM_A) {
#pragma unroll
        for (int i = 0; i < T::A_CHUNKS; i++) atomicAdd(&RowSum[(tid + T::THREADS * i) / C], sa[i]);
    }
    if (SUM_B) {
        if constexpr (TRANS_B) {
#pragma unroll
            for (int i = 0; i < T::B_CHUNKS; i++) atomicAdd(&ColSum[(tid + T::THREADS * i) / C], sb[i]);
        } else {
#pragma unroll
            for (int s = 0; s < 4; s++) atomicAdd(&ColSum[4 * cg + (int)((uint32_t)s ^ xo)], sb[s]);
        }
    }
    if (SUM_A || SUM_B) __syncthreads();

    // Store: MFMA 16 x 16 output layout, lane l holds rows 4 * (l / 16) + r, column l % 16.
    const bool za_row = g.flags & OG_GEMM_ZA_PER_ROW, zb_col = g.flags & OG_GEMM_ZB_PER_COL;
    const uint32_t Ku = (uint32_t)K;
    // One copy of the loop per output kind, int32 / float32 or requantized bytes (written out twice: wrapping it in a
    // lambda makes this kernel spill).
#define OG_TILED_STORE_LOOP(STORE)                                                                                     \
    for (int j = 0; j < T::FN; j++) {                                                                                  \
        const int nl = wn * (BN / WN) + 16 * j + i16;                                                                  \
        const int32_t n = n0 + nl;                                                                                     \
        if (n >= g.N) continue;                                                                                        \
        const uint32_t wz = (uint32_t)signed_zero(g.ZB, n, zb_col, b_signed);                                          \
        const uint32_t st = SUM_B ? (uint32_t)ColSum[nl] : 0u;                                                         \
        const uint32_t cib = (g.epi & OG_EPI_INT_BIAS) ? (uint32_t)g.bias[n] : 0u;                                     \
        const float csc = (g.epi & (OG_EPI_FLOAT | EPI_REQUANT)) ? column_scale(g, n) : 0.0f;                          \
        const float cfb = (g.epi & OG_EPI_FLOAT_BIAS) ? g.fbias[n] : 0.0f;                                             \
        _Pragma("unroll") for (int i = 0; i < T::FM; i++) {                                                            \
            _Pragma("unroll") for (int r = 0; r < 4; r++) {                                                            \
                const int ml = wm * (BM / WM) + 16 * i + 4 * g4 + r;                                                   \
                const int32_t m = m0 + ml;                                                                             \
                if (m >= g.M) continue;                                                                                \
                const uint32_t zz = (uint32_t)signed_zero(g.ZA, m, za_row, a_signed);                                  \
                const uint32_t ss = SUM_A ? (uint32_t)RowSum[ml] : 0u;                                                 \
                const uint32_t v = (uint32_t)acc[i][j][r] - wz * ss - zz * st + Ku * zz * wz;                          \
                STORE(g, batch * g.strideC + (int64_t)m * g.N + n, v + cib, csc, cfb);                                 \
            }                                                                                                          \
        }                                                                                                              \
    }
    if (g.epi & EPI_REQUANT) {
#pragma unroll
        OG_TILED_STORE_LOOP(store_requantized_col)
    } else {
#pragma unroll
        OG_TILED_STORE_LOOP(store_sum_col)
    }
#undef OG_TILED_STORE_LOOP
}

template <int BM, int BN, int BK, int WM, int WN, bool TRANS_B>
static hipError_t launch_tiled_cfg(const GemmArgs &g, hipStream_t s)
{
    int32_t tn = (g.N + BN - 1) / BN, tm = (g.M + BM - 1) / BM;
    int64_t blocks = (int64_t)tn * tm * g.batch;
    if (blocks <= 0) return hipSuccess;
    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    // A byte sum is needed only when the other operand's shifted zero point can be non-zero.
    const bool sum_a = (g.flags & OG_GEMM_ZB) || !b_signed;
    const bool sum_b = (g.flags & OG_GEMM_ZA) || !a_signed;
    dim3 grid((uint32_t)blocks), block(64 * WM * WN);
#define OG_TILED(SA, SB) hipLaunchKernelGGL((k_gemm_tiled<BM, BN, BK, WM, WN, TRANS_B, SA, SB>), grid, block, 0, s, g, tn, tm)
    if (sum_a && sum_b) OG_TILED(true, true);
    else if (sum_a) OG_TILED(true, false);
    else if (sum_b) OG_TILED(false, true);
    else OG_TILED(false, false);
#undef OG_TILED
    return hipGetLastError();
}

// The aligned kernel's conditions (see k_gemm_tiled).
bool tiled_fast_ok(const GemmArgs &g)
{
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    const int64_t lim = 0x7FFFFFFFll;
    if (((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 15) != 0) return false;
    if (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & (trans_b ? 15 : 3)) != 0) return false;
    if ((int64_t)g.M * g.lda > lim) return false;
    if ((int64_t)(trans_b ? g.N : g.K) * g.ldb > lim) return false;
    return b_dwords_ok(g);
}

// The large tile when it still gives (nearly) every CU a tile of its own; the small one otherwise.
bool tiled_uses_large(int32_t M, int32_t N, int32_t batch)
{
    int64_t big = (int64_t)((M + 255) / 256) * ((N + 255) / 256) * batch;
    return big >= 200;
}

hipError_t launch_gemm_tiled(const GemmArgs &g, hipStream_t s, const char **kernel)
{
    if (!tiled_fast_ok(g)) return launch_gemm_generic(g, s, kernel);
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    const bool large = (g.flags & OG_GEMM_LARGE_TILE) || tiled_uses_large(g.M, g.N, g.batch);
    if (direct_ok(g)) return launch_gemm_direct(g, s, kernel, large);
    if (large) {
        *kernel = "mfma-i8-tile256x256x64";
        return trans_b ? launch_tiled_cfg<256, 256, 64, 2, 2, true>(g, s) : launch_tiled_cfg<256, 256, 64, 2, 2, false>(g, s);
    }
    *kernel = "mfma-i8-tile128x128x128";
    return trans_b ? launch_tiled_cfg<128, 128, 128, 2, 2, true>(g, s) : launch_tiled_cfg<128, 128, 128, 2, 2, false>(g, s);
}

}  // namespace og
