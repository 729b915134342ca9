// Few-rows int8 products (M <= 16, B stored K x N): the decode-step shape, bound by streaming B once from HBM.
//
// Each wave owns 64 columns. Lane (c = lane % 16, g = lane / 16) loads a 16-row x 4-column block of B per 64-row step
// (one 4-byte load per row, 16 lanes cover 64 contiguous bytes of a row), transposes it 4 x 4 bytes at a time with
// v_perm_b32 into four 16-byte k-runs, and feeds them to four v_mfma_i32_16x16x64_i8 whose A operand is the (at most 16)
// activation rows. MFMA j therefore produces columns 4c + j. The activations are shifted to the signed domain as in the
// tiled kernel; each k-slice corrects its own partial sums for the zero points with the slice's row and column byte sums
//     sum_slice (s - z')(t - w') = sum s t - w' sum s - z' sum t + k_s z' w'
// so slices just add up (mod 2^32) in the second pass, which then applies the epilogue. With one slice the first pass
// stores the finished values itself.
#include "og_internal.hpp"

namespace og {

typedef int32_t v4i __attribute__((ext_vector_type(4)));

constexpr int SK_COLS = 256;   // columns per workgroup (4 waves x 64)

__device__ __forceinline__ uint4 load_row16_s(const uint8_t *row, int32_t k, int32_t K, bool row_ok, bool vec_ok,
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

__device__ __forceinline__ uint32_t load_cols4_s(const uint8_t *row, int32_t n, int32_t N, bool row_ok, bool vec_ok,
                                                 uint32_t flip)
{
    if (!row_ok) return 0u;
    if (vec_ok && n + 4 <= N) return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(row + n)) ^ flip;
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (n + e < N) w |= ((uint32_t)row[n + e] ^ (flip & 0xFFu)) << (e * 8);
    }
    return w;
}

// grid.x = col_blocks * slices * batch. partials: [batch][slice][M][np] int32 (np = N rounded up to 4).
template <bool SUM_A, bool SUM_B, bool DIRECT>
__global__ __launch_bounds__(256) void k_gemm_skinny(GemmArgs g, int32_t ks, int32_t slices, int32_t col_blocks,
                                                     int32_t np, int32_t *partials)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, g4 = lane >> 4;
    int64_t bid = blockIdx.x;
    const int32_t cb = (int32_t)(bid % col_blocks);
    bid /= col_blocks;
    const int32_t s = (int32_t)(bid % slices);
    const int32_t batch = (int32_t)(bid / slices);

    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    const uint32_t flip_a = a_signed ? 0u : 0x80808080u, flip_b = b_signed ? 0u : 0x80808080u;
    const uint8_t *A = g.A + batch * g.strideA;
    const uint8_t *B = g.B + batch * g.strideB;
    const bool vec_a = ((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 15) == 0;
    const bool vec_b = ((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 3) == 0;
    const int32_t n = cb * SK_COLS + wave * 64 + 4 * c;   // first of this lane's four columns
    const int32_t k_begin = s * ks, k_end = min(g.K, k_begin + ks);

    v4i acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = (v4i){0, 0, 0, 0};
    int32_t sum_t[4] = {0, 0, 0, 0};
    int32_t sum_s = 0;
    const bool row_ok = c < g.M;   // the A operand's row is lane % 16
    const uint8_t *arow = A + (int64_t)c * g.lda;

    for (int32_t k0 = k_begin; k0 < k_end; k0 += 64) {
        uint4 av = load_row16_s(arow, k0 + 16 * g4, k_end, row_ok, vec_a, flip_a);
        uint32_t rb[16];
        if (vec_b && n + 4 <= g.N && k0 + 16 * g4 + 16 <= k_end) {
            // All 16 rows and 4 columns in range: 16 word loads in flight together.
            const uint8_t *bp = B + (int64_t)(k0 + 16 * g4) * g.ldb + n;
#pragma unroll
            for (int r = 0; r < 16; r++)
                rb[r] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(bp + (int64_t)r * g.ldb));
#pragma unroll
            for (int r = 0; r < 16; r++) rb[r] ^= flip_b;
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int32_t gk = k0 + 16 * g4 + r;
                rb[r] = load_cols4_s(B + (int64_t)gk * g.ldb, n, g.N, gk < k_end, vec_b, flip_b);
            }
        }
        uint32_t col[4][4];
#pragma unroll
        for (int b4 = 0; b4 < 4; b4++)
            transpose4x4(rb[4 * b4], rb[4 * b4 + 1], rb[4 * b4 + 2], rb[4 * b4 + 3], col[0][b4], col[1][b4], col[2][b4],
                         col[3][b4]);
        v4i a = (v4i){(int32_t)av.x, (int32_t)av.y, (int32_t)av.z, (int32_t)av.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v4i b = (v4i){(int32_t)col[j][0], (int32_t)col[j][1], (int32_t)col[j][2], (int32_t)col[j][3]};
            acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[j], 0, 0, 0);
            if (SUM_B) {
#pragma unroll
                for (int b4 = 0; b4 < 4; b4++) sum_t[j] = dot4(col[j][b4], 0x01010101u, sum_t[j]);
            }
        }
        if (SUM_A) sum_s = dot4(av.w, 0x01010101u, dot4(av.z, 0x01010101u, dot4(av.y, 0x01010101u, dot4(av.x, 0x01010101u, sum_s))));
    }

    // Slice byte sums: the four k-groups of a column (row) sit in lanes l, l + 16, l + 32, l + 48.
    if (SUM_B) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sum_t[j] += __shfl_xor(sum_t[j], 16);
            sum_t[j] += __shfl_xor(sum_t[j], 32);
        }
    }
    if (SUM_A) {
        sum_s += __shfl_xor(sum_s, 16);
        sum_s += __shfl_xor(sum_s, 32);
    }

    const bool za_row = g.flags & OG_GEMM_ZA_PER_ROW, zb_col = g.flags & OG_GEMM_ZB_PER_COL;
    const uint32_t ks_real = (uint32_t)max(0, k_end - k_begin);
    uint32_t wz[4];
#pragma unroll
    for (int j = 0; j < 4; j++) wz[j] = (n + j < g.N) ? (uint32_t)signed_zero(g.ZB, n + j, zb_col, b_signed) : 0u;

    // Output layout of the 16 x 16 MFMA: lane (c, g4) holds rows 4 * g4 + r of columns n + j (MFMA j).
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int32_t m = 4 * g4 + r;
        const uint32_t ss = SUM_A ? (uint32_t)__shfl(sum_s, m) : 0u;   // lane m (< 16) holds row m's sum
        if (m >= g.M || n >= g.N) continue;
        const uint32_t zz = (uint32_t)signed_zero(g.ZA, m, za_row, a_signed);
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[j] = (uint32_t)acc[j][r] - wz[j] * ss - zz * (SUM_B ? (uint32_t)sum_t[j] : 0u) + ks_real * zz * wz[j];
        if (DIRECT) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (n + j < g.N) store_value(g, batch * g.strideC + (int64_t)m * g.N + n + j, n + j, v[j]);
        } else {
            int32_t *p = partials + (((int64_t)batch * slices + s) * g.M + m) * np + n;
            *reinterpret_cast<int4 *>(p) = make_int4((int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3]);
        }
    }
}

// Adds the slices' corrected partial sums and applies the epilogue: one thread per output.
__global__ __launch_bounds__(256) void k_gemm_skinny_reduce(GemmArgs g, int32_t slices, int32_t np,
                                                            const int32_t *partials)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_batch = (int64_t)g.M * g.N;
    if (i >= per_batch * g.batch) return;
    const int32_t batch = (int32_t)(i / per_batch);
    const int64_t r = i % per_batch;
    const int32_t m = (int32_t)(r / g.N), n = (int32_t)(r % g.N);
    const int32_t *p = partials + ((int64_t)batch * slices * g.M + m) * np + n;
    const int64_t slice_stride = (int64_t)g.M * np;
    // Eight slices' loads in flight at a time (a trip of one load waits out a memory round trip per slice).
    uint32_t v = 0;
    int32_t s = 0;
    for (; s + 8 <= slices; s += 8) {
        uint32_t x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = (uint32_t)p[(s + u) * slice_stride];
#pragma unroll
        for (int u = 0; u < 8; u++) v += x[u];
    }
    for (; s < slices; s++) v += (uint32_t)p[s * slice_stride];
    store_value(g, batch * g.strideC + (int64_t)m * g.N + n, n, v);
}

int skinny_slices(int32_t M, int32_t N, int32_t K, int32_t batch)
{
    int32_t col_blocks = (N + SK_COLS - 1) / SK_COLS;
    int64_t base = (int64_t)col_blocks * batch;
    int32_t steps = (K + 63) / 64;
    if (steps <= 1) return 1;
    // Enough workgroups to keep every CU streaming, but each slice's partials (M x N int32, written and read back) stay a
    // small fraction of the slice's bytes of B: k rows per slice >= 32 * M.
    int64_t want = (1024 + base - 1) / base;
    int32_t min_steps = max(1, (32 * M + 63) / 64);
    int64_t slices = want < steps / min_steps ? want : steps / min_steps;
    if (slices < 1) slices = 1;
    int32_t ks_steps = (int32_t)((steps + slices - 1) / slices);
    return (steps + ks_steps - 1) / ks_steps;
}

static int32_t skinny_ks(int32_t K, int32_t slices)
{
    int32_t steps = (K + 63) / 64;
    return ((steps + slices - 1) / slices) * 64;
}

uint64_t skinny_workspace_bytes(int32_t M, int32_t N, int32_t K, int32_t batch)
{
    int32_t slices = skinny_slices(M, N, K, batch);
    if (slices <= 1) return 0;
    int64_t np = ((int64_t)N + 3) / 4 * 4;
    return (uint64_t)batch * slices * M * np * 4;
}

hipError_t launch_gemm_skinny(const GemmArgs &g, const Workspace &ws, hipStream_t s, const char **kernel, int step)
{
    const int32_t slices = skinny_slices(g.M, g.N, g.K, g.batch);
    const int32_t ks = skinny_ks(g.K, slices);
    const int32_t col_blocks = (g.N + SK_COLS - 1) / SK_COLS;
    const int32_t np = (g.N + 3) / 4 * 4;
    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    const bool sum_a = (g.flags & OG_GEMM_ZB) || !b_signed;
    const bool sum_b = (g.flags & OG_GEMM_ZA) || !a_signed;
    if (step == 1) {
        *kernel = "skinny-reduce";
        int64_t total = (int64_t)g.M * g.N * g.batch;
        if (slices <= 1 || total <= 0) return hipSuccess;
        hipLaunchKernelGGL(k_gemm_skinny_reduce, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, g, slices, np,
                           (const int32_t *)ws.partials);
        return hipGetLastError();
    }
    const bool direct = slices <= 1;
    *kernel = direct ? "mfma-i8-rows16-direct" : "mfma-i8-rows16-splitk";
    dim3 grid((uint32_t)((int64_t)col_blocks * slices * g.batch)), block(256);
    int32_t *p = ws.partials;
#define OG_SKINNY(SA, SB, D) hipLaunchKernelGGL((k_gemm_skinny<SA, SB, D>), grid, block, 0, s, g, ks, slices, col_blocks, np, p)
    if (direct) {
        if (sum_a && sum_b) OG_SKINNY(true, true, true);
        else if (sum_a) OG_SKINNY(true, false, true);
        else if (sum_b) OG_SKINNY(false, true, true);
        else OG_SKINNY(false, false, true);
    } else {
        if (sum_a && sum_b) OG_SKINNY(true, true, false);
        else if (sum_a) OG_SKINNY(true, false, false);
        else if (sum_b) OG_SKINNY(false, true, false);
        else OG_SKINNY(false, false, false);
    }
#undef OG_SKINNY
    return hipGetLastError();
}

}  // namespace og
