// The 256 x 256 direct kernel for B stored K x N, and the dispatch of both tile sizes and layouts (the kernel itself
// and its launch templates are in int8_gemm_direct.hpp; the other instances are in int8_gemm_direct_nk.hip and
// int8_gemm_direct128.hip).
#include "int8_gemm_direct.hpp"

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

hipError_t launch_gemm_direct(const GemmArgs &g, hipStream_t s, const char **kernel, bool large)
{
    const int32_t bt = large ? 256 : 128;
    const int32_t tn = (g.N + bt - 1) / bt, tm = (g.M + bt - 1) / bt;
    const int64_t blocks = (int64_t)tn * tm * g.batch;
    *kernel = large ? "mfma-i8-direct256x256x64" : "mfma-i8-direct128x128x64";
    if (blocks <= 0) return hipSuccess;
    const dim3 grid((uint32_t)blocks);
    if (!large) launch_direct128(g, s, grid, tn, tm);
    else if (g.flags & OG_GEMM_TRANSPOSE_B) launch_direct_nk256(g, s, grid, tn, tm);
    else launch_direct_t<256, false>(g, s, grid, tn, tm);
    return hipGetLastError();
}

}  // namespace og
