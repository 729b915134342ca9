// Few-rows int8 products (M <= 16, B stored K x N), one workgroup per tile of B: the decode-step shape, bound by
// reading B once from HBM.
//
//  - B is cut into tiles of 256 rows x 256 columns. Each workgroup loads one tile into LDS by DMA
//    (buffer_load ... lds), 16 loads a thread all in flight at once, after its <= 16 rows of A (one load a thread),
//    and computes the tile's 64-row sub-stages as they land. Many short workgroups, two resident per CU, keep more
//    bytes in flight than a persistent loop and let the hardware balance the CUs.
//  - B is read back with the gfx950 transpose read ds_read_b64_tr_b8 and each wave runs v_mfma_i32_16x16x64_i8 on its
//    64 columns. The MFMA's A operand has 16 rows; when M < 16, row M is all ones, so the same MFMA also produces the
//    column sums of B that A's zero point needs (M = 16 runs a second MFMA against ones).
//  - Each tile writes its part (the sums s t of its k-range, the column sums of B and the row sums of A over it) with
//    plain stores and exits; nothing waits for them. A second, small kernel adds a slab's parts in a fixed order,
//    applies the zero points and the epilogue once with the whole K, and stores C. The kernel boundary orders the
//    two; no counters, atomics or fences are involved, and integer sums are exact in any order anyway.
//        sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w'   (mod 2^32; Int8GemmDot.hlsl:1-11)
#include <algorithm>
#include <type_traits>

#include "og_internal.hpp"

namespace og {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u4w __attribute__((ext_vector_type(4)));

constexpr int GT_COLS = 256, GT_THREADS = 256;
constexpr int GT_KT = 256;                 // rows of B per tile (a multiple of 64, at most 256)
constexpr int GT_AROW = 256;               // bytes of an A row in LDS (16 chunks, GT_KT / 16 of them used)
constexpr int GT_SUB = 64;                 // rows per sub-stage (one MFMA deep)
constexpr int GT_NSUB = GT_KT / GT_SUB;
constexpr int GT_LPS = GT_SUB * GT_COLS / 16 / GT_THREADS;   // DMA loads per thread per sub-stage
constexpr int GT_ROWS_PER_SUM = 4;         // rows of C per thread of the summing kernel

__device__ __forceinline__ u4w tile_rsrc(const uint8_t *base, int32_t bytes)
{
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return (u4w){(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, (uint32_t)max(bytes, 0), 0x00020000u};
}

// LDS DMA: lane l's 16 bytes at rsrc + voff land at LDS address lds + 16 l. From inline assembly, so that the compiler
// adds no waits of its own; the sub-stages wait for exactly their loads (vmcnt counts them in issue order). Nothing
// else in the kernel uses M0.
__device__ __forceinline__ void tile_dma16(u4w rsrc, uint32_t lds, uint32_t voff)
{
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(lds), "v"(voff), "s"(rsrc) : "memory");
}

template <int N>
__device__ __forceinline__ void tile_wait_vm_barrier()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Position of 16-byte chunk c of tile row k in LDS (rows of 256 bytes): XOR-swizzled so that the 8 rows one
// transpose read touches fall in different banks.
__device__ __forceinline__ int tile_pos(int k, int c) { return c ^ ((k & 7) | (((k >> 4) & 1) << 3)); }

__device__ __forceinline__ uint32_t tile_sad16(v4i v, uint32_t acc)
{
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.x, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.y, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.z, 0u, acc);
    return __builtin_amdgcn_sad_u8((uint32_t)v.w, 0u, acc);
}

template <typename F, int... I>
__device__ __forceinline__ void tile_static_for(F &&f, std::integer_sequence<int, I...>)
{
    (f(std::integral_constant<int, I>{}), ...);
}

}  // namespace

// A part in the MFMA's own layout: row groups of 4 (rows 0 .. M - 1 of sums, row M the column sums of B), each 256
// columns of 4 ints (one 16-byte store a lane), then 16 row sums of A.
__host__ __device__ inline int32_t gemv_tile_groups(int32_t M) { return (M + 4) / 4; }
__host__ __device__ inline int64_t gemv_tile_part(int32_t M) { return (int64_t)gemv_tile_groups(M) * GT_COLS * 4 + 16; }

// SUM_A / SUM_B: the row sums of A / column sums of B are needed; FLIP_A / FLIP_B: the operand is unsigned.
// Workgroup x takes slab x % slabs of row band x / slabs (band = batch * nkc + kc): the workgroups running together read
// whole rows of B. Tile (q = batch * slabs + slab, kc) writes part q * nkc + kc.
template <bool SUM_A, bool SUM_B, bool FLIP_A, bool FLIP_B>
__global__ __launch_bounds__(GT_THREADS) void k_gemv_tiles(GemmArgs g, int32_t slabs, int32_t nkc, int32_t *parts)
{
    static_assert(GT_KT % GT_SUB == 0 && GT_KT <= GT_AROW, "tile rows");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[GT_KT * GT_COLS + 16 * GT_AROW];
    uint8_t *const asmem = smem + GT_KT * GT_COLS;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g4 = lane >> 4;
    const int64_t band = blockIdx.x / slabs;
    const int32_t slab = (int32_t)(blockIdx.x % slabs), b = (int32_t)(band / nkc), kc = (int32_t)(band % nkc);
    const int64_t q = (int64_t)b * slabs + slab;
    const int32_t M = g.M, N = g.N, K = g.K, ldb = g.ldb;
    const int32_t n0 = slab * GT_COLS, k0 = kc * GT_KT, rows = min(GT_KT, K - k0);

    // All loads are DMA issued here, in the order they are waited for: A's k-range of this tile (16 rows x 256
    // bytes; rows past M read as zero, bytes past K are masked when used), then B's sub-stages (rows past K and bytes
    // past the operand read as zero).
    {
        const uint32_t lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)smem;
        // A in LDS: 16 rows of 256 bytes, chunk c of row r at position c ^ r (the 16 rows a fragment read touches
        // spread over the banks); thread t fills slot t, row t / 16 at position t % 16. With tiles under 256 rows the
        // chunks past the tile are loaded too (the next k-range, or zeros past the operand) and never read.
        const int r = tid >> 4, c = (tid & 15) ^ r;
        const u4w ra = tile_rsrc(g.A + b * g.strideA + k0, (M - 1) * g.lda + min(GT_KT, K - k0));
        tile_dma16(ra, lds + GT_KT * GT_COLS + (uint32_t)wave * 1024u, (uint32_t)r * (uint32_t)g.lda + 16u * (uint32_t)c);
        const u4w rb = tile_rsrc(g.B + b * g.strideB + (int64_t)k0 * ldb + n0, (rows - 1) * ldb + min(GT_COLS, N - n0));
#pragma unroll
        for (int i = 0; i < GT_NSUB * GT_LPS; i++) {
            const int s = (i * 4 + wave) * 64 + lane, k = s >> 4, p = s & 15;
            tile_dma16(rb, lds + (uint32_t)wave * 1024u + (uint32_t)i * 4096u,
                       (uint32_t)k * (uint32_t)ldb + 16u * (uint32_t)tile_pos(k, p));
        }
    }

    const bool ones_row = SUM_B && M < 16, ones_mfma = SUM_B && M == 16;
    v4i acc[4], accs[4];
#pragma unroll
    for (int j = 0; j < 4; j++) { acc[j] = (v4i){0, 0, 0, 0}; accs[j] = (v4i){0, 0, 0, 0}; }
    uint32_t rsum = 0;
    tile_static_for([&](auto ks_tag) {
        constexpr int ks = decltype(ks_tag)::value;
        tile_wait_vm_barrier<GT_LPS * (GT_NSUB - 1 - ks)>();   // sub-stage ks landed (this wave's loads, then all)
        const bool kv = k0 + GT_SUB * ks + 16 * g4 < K;
        const bool av = kv && i16 < M;
        v4i a = *reinterpret_cast<const v4i *>(asmem + i16 * GT_AROW + 16 * ((4 * ks + g4) ^ i16));
        if constexpr (!FLIP_A) a = av ? a : (v4i){0, 0, 0, 0};
        if constexpr (SUM_A) rsum = av ? tile_sad16(FLIP_A ? a : (a ^ (int32_t)0x80808080), rsum) : rsum;
        if constexpr (FLIP_A) a = av ? (a ^ (int32_t)0x80808080) : (v4i){0, 0, 0, 0};
        const int32_t one = kv ? 0x01010101 : 0;
        if (ones_row && i16 == M) a = (v4i){one, one, one, one};
        const v4i ones = (v4i){one, one, one, one};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = wave * 4 + j;   // 16-byte chunk of the block's columns
            v2i h[2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int k = GT_SUB * ks + 16 * g4 + 8 * hh + (i16 >> 1);
                h[hh] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (__attribute__((address_space(3))) v2i *)(smem + k * GT_COLS + 16 * tile_pos(k, c) + 8 * (i16 & 1)));
            }
            v4i bf = (v4i){h[0].x, h[0].y, h[1].x, h[1].y};
            if constexpr (FLIP_B) bf ^= (int32_t)0x80808080;
            acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bf, acc[j], 0, 0, 0);
            if (ones_mfma) accs[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ones, bf, accs[j], 0, 0, 0);
        }
    }, std::make_integer_sequence<int, GT_NSUB>{});

    // The part. MFMA 16 x 16 layout: lane l holds rows 4 (l / 16) + r, column l % 16 of each block, i.e. row group
    // l / 16 of its column; rows past M + 1 are not needed and row groups past them not written. With M = 16 the
    // column sums come from the second MFMA (all its rows equal), as row group 4.
    const int32_t groups = gemv_tile_groups(M);
    int32_t *const part = parts + (q * nkc + kc) * gemv_tile_part(M);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int col = wave * 64 + 16 * j + i16;
        if (g4 < groups) *reinterpret_cast<v4i *>(part + (g4 * GT_COLS + col) * 4) = acc[j];
        if (ones_mfma && g4 == 0) *reinterpret_cast<v4i *>(part + (4 * GT_COLS + col) * 4) = accs[j];
    }
    if (SUM_A && wave == 0) {
        // Biased byte sums of the four k-groups (lanes l, l + 16, l + 32, l + 48); the signed sum is 128 less per byte.
        uint32_t v = rsum + (uint32_t)__shfl_xor((int32_t)rsum, 16);
        v += (uint32_t)__shfl_xor((int32_t)v, 32);
        if (g4 == 0) part[groups * GT_COLS * 4 + i16] = (int32_t)(v - 128u * (uint32_t)rows);
    }
}

// The parts of a slab added up, for a row group (4 rows) and 64 of its columns: workgroup x takes quarter x % 4 of the
// columns, row group (x / 4) % row_groups of slab x / (4 row_groups). Thread t sums, for column t % 64, the parts
// p = t / 64 (mod 4), all its loads in flight at once (one round for up to 16 parts); the four partial sums meet in
// LDS and the first 64 threads apply the zero points with the whole K, then the epilogue.
template <bool SUM_A, bool SUM_B, bool FLIP_A, bool FLIP_B>
__global__ __launch_bounds__(GT_THREADS) void k_gemv_tiles_sum(GemmArgs g, int32_t slabs, int32_t nkc,
                                                                const int32_t *parts)
{
    __shared__ v4i red_v[4][64], red_r[4][64];
    __shared__ uint32_t red_c[4][64];
    const int tid = threadIdx.x, cl = tid & 63, u = tid >> 6;
    const int32_t row_groups = (g.M + GT_ROWS_PER_SUM - 1) / GT_ROWS_PER_SUM;
    const int64_t x = blockIdx.x;
    const int32_t cq = (int32_t)(x & 3);
    const int64_t rest = x >> 2, q = rest / row_groups;
    const int32_t m0 = (int32_t)(rest % row_groups) * GT_ROWS_PER_SUM;
    const int32_t b = (int32_t)(q / slabs), slab = (int32_t)(q % slabs);
    const int32_t M = g.M, N = g.N, K = g.K;
    const int32_t col = 64 * cq + cl, n = slab * GT_COLS + col;
    const int64_t stride = gemv_tile_part(M);
    const int32_t *pp = parts + q * nkc * stride;
    const int32_t gi = m0 / 4, groups = gemv_tile_groups(M);
    const bool cs_here = M / 4 == gi;   // the column sums (row M) share this row group

    v4i v = {0, 0, 0, 0}, rs = {0, 0, 0, 0};
    uint32_t cs = 0;
    for (int32_t p0 = u; p0 < nkc; p0 += 16) {
        v4i xv[4], r[4];
        uint32_t c[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            // Parts past the last read the last one (inside the workspace) and are masked off.
            const int32_t *part = pp + min(p0 + 4 * e, nkc - 1) * stride;
            xv[e] = *reinterpret_cast<const v4i *>(part + (gi * GT_COLS + col) * 4);
            r[e] = SUM_A ? *reinterpret_cast<const v4i *>(part + groups * GT_COLS * 4 + 4 * gi) : (v4i){0, 0, 0, 0};
            c[e] = (SUM_B && !cs_here) ? (uint32_t)part[((M / 4) * GT_COLS + col) * 4 + (M & 3)] : 0u;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int32_t keep = p0 + 4 * e < nkc ? -1 : 0;
            v += xv[e] & keep;
            rs += r[e] & keep;
            cs += (cs_here ? (uint32_t)xv[e][M & 3] : c[e]) & (uint32_t)keep;
        }
    }
    red_v[u][cl] = v;
    red_r[u][cl] = rs;
    red_c[u][cl] = cs;
    __syncthreads();
    if (u != 0 || n >= N) return;
#pragma unroll
    for (int w = 1; w < 4; w++) {
        v += red_v[w][cl];
        rs += red_r[w][cl];
        cs += red_c[w][cl];
    }
    uint32_t wz = 0;
    if (SUM_A) {
        const uint32_t w = g.ZB ? g.ZB[(g.flags & OG_GEMM_ZB_PER_COL) ? n : 0] : 0u;
        wz = FLIP_B ? w - 128u : (uint32_t)sext8(w);
    }
    const bool per = g.flags & OG_GEMM_ZA_PER_ROW;
#pragma unroll
    for (int r = 0; r < GT_ROWS_PER_SUM; r++) {
        const int32_t m = m0 + r;
        if (m >= M) break;
        uint32_t zz = 0;
        if (SUM_B) {
            const uint32_t z = g.ZA ? g.ZA[per ? m : 0] : 0u;
            zz = FLIP_A ? z - 128u : (uint32_t)sext8(z);
        }
        const uint32_t res = (uint32_t)v[r] - wz * (uint32_t)rs[r] - zz * (cs - (uint32_t)K * wz);
        store_value(g, b * g.strideC + (int64_t)m * N + n, n, res);
    }
}

// The tiled few-rows kernel's conditions: B stored K x N; 16-byte aligned rows of both operands, K and N multiples
// of 16 (no 16-byte load straddles a row end); a tile's byte range under 2^31; grids within range.
bool gemv_tiles_ok(const GemmArgs &g)
{
    if (g.flags & OG_GEMM_TRANSPOSE_B) return false;
    if (g.M < 1 || g.M > 16 || g.K < 1 || g.N < 1) return false;
    if ((g.N & 15) != 0 || (g.K & 15) != 0) return false;
    if (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 15) != 0) return false;
    if (((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 15) != 0) return false;
    if ((int64_t)GT_KT * g.ldb + GT_COLS > 0x7FFFFFFFll || (int64_t)16 * g.lda + GT_KT > 0x7FFFFFFFll) return false;
    const int64_t q = (int64_t)g.batch * ((g.N + GT_COLS - 1) / GT_COLS);
    return q * ((g.K + GT_KT - 1) / GT_KT) <= 0x7FFFFFFFll && q * 16 <= 0x7FFFFFFFll;
}

uint64_t gemv_tiles_workspace_bytes(const GemmArgs &g)
{
    const int64_t q = (int64_t)g.batch * ((g.N + GT_COLS - 1) / GT_COLS);
    return (uint64_t)(q * ((g.K + GT_KT - 1) / GT_KT) * gemv_tile_part(g.M) * 4);
}

// step 0: the tiles (parts into ws.partials); step 1: the sums of the parts.
hipError_t launch_gemv_tiles(const GemmArgs &g, const Workspace &ws, hipStream_t s, const char **kernel, int step)
{
    const int32_t slabs = (g.N + GT_COLS - 1) / GT_COLS, nkc = (g.K + GT_KT - 1) / GT_KT;
    const int64_t q = (int64_t)g.batch * slabs;
    const bool fa = !(g.flags & OG_GEMM_A_INT8), fb = !(g.flags & OG_GEMM_B_INT8);
    const bool sa = (g.flags & OG_GEMM_ZB) || fb, sb = (g.flags & OG_GEMM_ZA) || fa;
    const dim3 block(GT_THREADS);
    const dim3 grid(step == 0 ? (uint32_t)(q * nkc) : (uint32_t)(q * ((g.M + GT_ROWS_PER_SUM - 1) / GT_ROWS_PER_SUM) * 4));
    *kernel = step == 0 ? "mfma-i8-rows16-tiles" : "rows16-tiles-sum";
#define OG_GT(SA, SB, FA, FB)                                                                                       \
    do {                                                                                                           \
        if (step == 0) hipLaunchKernelGGL((k_gemv_tiles<SA, SB, FA, FB>), grid, block, 0, s, g, slabs, nkc, ws.partials); \
        else hipLaunchKernelGGL((k_gemv_tiles_sum<SA, SB, FA, FB>), grid, block, 0, s, g, slabs, nkc, ws.partials);   \
    } while (0)
    if (fa && fb) OG_GT(true, true, true, true);
    else if (fa) { if (sa) OG_GT(true, true, true, false); else OG_GT(false, true, true, false); }
    else if (fb) { if (sb) OG_GT(true, true, false, true); else OG_GT(true, false, false, true); }
    else if (sa && sb) OG_GT(true, true, false, false);
    else if (sa) OG_GT(true, false, false, false);
    else if (sb) OG_GT(false, true, false, false);
    else OG_GT(false, false, false, false);
#undef OG_GT
    return hipGetLastError();
}

}  // namespace og
