// The 256 x 256 direct kernel for B stored K x N, and the dispatch of both tile sizes and layouts (the kernel itself
// and its launch templates are in int8_gemm_direct.hpp; the other instances are in int8_gemm_direct_nk.hip and
// int8_gemm_direct128.hip).
#include "int8_gemm_direct.hpp"

#include <algorithm>

namespace og {

// The direct kernel's conditions: K a multiple of the stage depth (64), 16-byte aligned rows for both operands,
// each batch's operands under 2^31 bytes.
bool direct_ok(const GemmArgs &g)
{
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    const int64_t lim = 0x7FFFFFFFll;
    if (g.K % DBK != 0) return false;
    if (((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 15) != 0) return false;
    if (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 15) != 0) return false;
    if ((int64_t)g.M * g.lda > lim) return false;
    if ((int64_t)(trans_b ? g.N : g.K) * g.ldb > lim) return false;
    return b_dwords_ok(g);
}

uint32_t direct_range_groups(const GemmArgs &g, bool large)
{
    if (large) return 0;   // the 256 tile has no range epilogue
    return (uint32_t)std::min<int64_t>(((g.N + 127) / 128) * ((g.M + 127) / 128) * g.batch, int64_t(1) << 30);
}

hipError_t launch_gemm_direct(const GemmArgs &g, hipStream_t s, const char **kernel, bool large)
{
    const int32_t bt = large ? 256 : 128;
    const int32_t tn = (g.N + bt - 1) / bt, tm = (g.M + bt - 1) / bt;
    const int64_t blocks = (int64_t)tn * tm * g.batch;
    *kernel = large ? "mfma-i8-direct256x256x64" : "mfma-i8-direct128x128x64";
    if (blocks <= 0) return hipSuccess;
    const dim3 grid((uint32_t)blocks);
    if (!large) launch_direct128(g, s, grid, tn, tm, 1, g.K);
    else if (g.flags & OG_GEMM_TRANSPOSE_B) launch_direct_nk256(g, s, grid, tn, tm);
    else launch_direct_t<256, false, 8>(g, s, grid, tn, tm, 1, g.K);
    return hipGetLastError();
}

int direct_split(const GemmArgs &g)
{
    // Grids that fill under half the chip with 128 x 128 tiles, cut along K into slices of at least 4 stages, with
    // no more workgroups than CUs (a second round would undo the gain). The split pays when the stages it takes off
    // each workgroup's serial walk outweigh what the split adds: every slice's int32 result written and read back, and
    // a launch. Conservative costs from MI355X measurements: 0.25 us per 64-deep stage of one 128 tile (C2's 12 stages
    // take 13.2 us and Whisper's 36 stages 22 us, of which about 9 us are a workgroup's fixed cost), 3 us a launch,
    // 4 TB/s for the partial sums.
    if (g.K <= 0 || g.M <= 0 || g.N <= 0 || (g.flags & OG_GEMM_LARGE_TILE)) return 1;
    const int64_t tiles = (int64_t)((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch;
    const int64_t stages = g.K / DBK;
    if (tiles * 2 > kSplitTargetTiles || stages < 8) return 1;
    int64_t ks = std::min<int64_t>(kSplitTargetTiles / tiles, stages / 4);
    // The partial sums (int32, every slice's whole result) stay within the workspace's budget and int32 indexing.
    const int64_t per_slice = (int64_t)g.M * g.N * g.batch * 4;
    ks = std::min<int64_t>(ks, kSplitMaxBytes / std::max<int64_t>(per_slice, 1));
    if (ks < 2) return 1;
    // As many slices as slices of that length need, so that none is empty.
    const int64_t per = (stages + ks - 1) / ks;
    ks = (stages + per - 1) / per;
    const double saved_us = 0.25 * (double)(stages - per);
    const double cost_us = 3.0 + (double)(2 * ks + 1) * (double)per_slice / 4e6;
    return ks >= 2 && saved_us > 1.2 * cost_us ? (int)ks : 1;
}

uint64_t direct_split_workspace_bytes(const GemmArgs &g, int ks)
{
    return (uint64_t)ks * (uint64_t)g.M * (uint64_t)g.N * (uint64_t)g.batch * 4u;
}

namespace {

// Slice kc's partial for (b, m, n) is parts[((b * ks + kc) * M + m) * N + n]; their sum gets the bias and the epilogue.
// V4: four neighbouring columns a thread (N a multiple of 4), one 16-byte load per slice.
template <bool V4>
__global__ __launch_bounds__(256) void k_splitk_sum(GemmArgs g, int32_t ks, const int32_t *parts)
{
    __shared__ float red[2 * 256 / 64];
    // A ranged float product: the NaN-ignoring range of the values this thread stores.
    const bool ranged = g.ranges != nullptr;
    float rmn = __int_as_float(0x7F800000), rmx = __int_as_float(0xFF800000);
    auto put = [&](int64_t ci, int32_t col, uint32_t sum) {
        if (ranged) {
            const float f = sum_to_float(g, col, sum);
            static_cast<float *>(g.C)[ci] = f;
            rmn = fminf(rmn, f);
            rmx = fmaxf(rmx, f);
        } else {
            store_value(g, ci, col, sum);
        }
    };
    const int64_t mn = (int64_t)g.M * g.N, per = V4 ? mn / 4 : mn, total = per * g.batch;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        const int64_t b = t / per, r = (t - b * per) * (V4 ? 4 : 1);
        const int32_t n = (int32_t)(r % g.N);
        const int32_t *p = parts + b * ks * mn + r;
        if constexpr (V4) {
            // Four slices' loads in flight at a time (a trip of one load waits out a memory round trip per slice).
            uint4 sum = make_uint4(0u, 0u, 0u, 0u);
            int32_t kc = 0;
            for (; kc + 4 <= ks; kc += 4) {
                uint4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = *reinterpret_cast<const uint4 *>(p + (kc + u) * mn);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    sum.x += v[u].x;
                    sum.y += v[u].y;
                    sum.z += v[u].z;
                    sum.w += v[u].w;
                }
            }
            for (; kc < ks; kc++) {
                const uint4 v = *reinterpret_cast<const uint4 *>(p + kc * mn);
                sum.x += v.x;
                sum.y += v.y;
                sum.z += v.z;
                sum.w += v.w;
            }
            const int64_t c = b * g.strideC + r;
            put(c, n, sum.x);
            put(c + 1, n + 1, sum.y);
            put(c + 2, n + 2, sum.z);
            put(c + 3, n + 3, sum.w);
        } else {
            uint32_t sum = 0;
            int32_t kc = 0;
            for (; kc + 4 <= ks; kc += 4) {
                uint32_t v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = (uint32_t)p[(kc + u) * mn];
                sum += v[0] + v[1] + v[2] + v[3];
            }
            for (; kc < ks; kc++) sum += (uint32_t)p[kc * mn];
            put(b * g.strideC + r, n, sum);
        }
    }
    if (ranged) store_workgroup_range<256>(rmn, rmx, red, g.ranges, blockIdx.x);
}

}  // namespace

// The summing pass's grid: one workgroup a 256 four-column groups (or columns), at most 2^20 workgroups.
static int64_t splitk_sum_groups(const GemmArgs &g)
{
    const bool v4 = g.N % 4 == 0;   // the partials start 256-byte aligned, so each row of 4-column groups is aligned
    const int64_t total = (int64_t)g.M * g.N * g.batch / (v4 ? 4 : 1);
    return std::min<int64_t>((total + 255) / 256, int64_t(1) << 20);
}

uint32_t direct_split_range_groups(const GemmArgs &g) { return (uint32_t)splitk_sum_groups(g); }

hipError_t launch_gemm_direct_split(const GemmArgs &g, const Workspace &ws, hipStream_t s, const char **kernel, int ks,
                                    int step)
{
    const int32_t tn = (g.N + 127) / 128, tm = (g.M + 127) / 128;
    if (step == 0) {
        *kernel = "mfma-i8-direct128x128x64-splitk";
        // Each slice: the whole k range's product machinery on its slice, int32 sums into the partials.
        GemmArgs gs = g;
        gs.C = ws.partials;
        gs.strideC = (int64_t)g.M * g.N;
        gs.batch = g.batch * ks;
        gs.epi = 0;
        gs.ranges = nullptr;   // the summing pass records the ranges
        const int64_t stages = g.K / DBK;
        const int32_t kslice = (int32_t)((stages + ks - 1) / ks) * DBK;
        const int64_t blocks = (int64_t)tn * tm * gs.batch;
        launch_direct128(gs, s, dim3((uint32_t)blocks), tn, tm, ks, kslice);
        return hipGetLastError();
    }
    *kernel = "splitk-sum";
    const bool v4 = g.N % 4 == 0;
    const int64_t wgs = splitk_sum_groups(g);
    if (v4) hipLaunchKernelGGL(k_splitk_sum<true>, dim3((uint32_t)wgs), dim3(256), 0, s, g, (int32_t)ks, ws.partials);
    else hipLaunchKernelGGL(k_splitk_sum<false>, dim3((uint32_t)wgs), dim3(256), 0, s, g, (int32_t)ks, ws.partials);
    return hipGetLastError();
}

}  // namespace og
