// The 128 x 128 direct kernel, both layouts of B (the kernel is in int8_gemm_direct.hpp; instantiated here so that the
// tile sizes compile in parallel).
#include "int8_gemm_direct.hpp"

namespace og {

void launch_direct128(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm, int32_t ks, int32_t kslice)
{
    if (g.flags & OG_GEMM_TRANSPOSE_B) launch_direct_t<128, true, 8>(g, s, grid, tn, tm, ks, kslice);
    else launch_direct_t<128, false, 8>(g, s, grid, tn, tm, ks, kslice);
}

}  // namespace og
