// The 256 x 256 direct kernel for B stored N x K (the same kernel as int8_gemm_direct.hip, instantiated here so that
// the layouts compile in parallel).
#include "int8_gemm_direct.hpp"

namespace og {

void launch_direct_nk256(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm)
{
    launch_direct_t<256, true, 8>(g, s, grid, tn, tm, 1, g.K);
}

}  // namespace og
