// The large-product kernel for B stored K x N, and the dispatch of both layouts (the kernel itself and its launch
// templates are in int8_gemm_direct.hpp; B stored N x K is instantiated in int8_gemm_direct_nk.hip).
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
    return true;
}

hipError_t launch_gemm_direct(const GemmArgs &g, hipStream_t s, const char **kernel)
{
    const int32_t tn = (g.N + DBN - 1) / DBN, tm = (g.M + DBM - 1) / DBM;
    const int64_t blocks = (int64_t)tn * tm * g.batch;
    *kernel = "mfma-i8-direct256x256x64";
    if (blocks <= 0) return hipSuccess;
    const dim3 grid((uint32_t)blocks);
    if (g.flags & OG_GEMM_TRANSPOSE_B) launch_direct_nk(g, s, grid, tn, tm);
    else launch_direct_t<false>(g, s, grid, tn, tm);
    return hipGetLastError();
}

}  // namespace og
