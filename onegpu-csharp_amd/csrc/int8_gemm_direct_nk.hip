// The large-product kernel for B stored N x K (the same kernel as int8_gemm_direct.hip, instantiated here so that the
// two layouts compile in parallel).
#include "int8_gemm_direct.hpp"

namespace og {

void launch_direct_nk(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm)
{
    launch_direct_t<true>(g, s, grid, tn, tm);
}

}  // namespace og
