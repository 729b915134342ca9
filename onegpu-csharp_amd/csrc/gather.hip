// ONNX Gather along one axis (GatherKernels.EncodeGather, GatherKernels.cs:66-118; Gather.hlsl:25-43 and
// GatherDriver.hlsli:6-92), the int8 embedding lookup in front of the first int8 product, for any payload width.
//
// The data tensor is [outer, axisLen, inner] elements and the output [outer, count, inner]: output row (o, i) is a copy
// of data row (o, index[i]), inner * width contiguous bytes either way. So the kernel copies byte rows and never looks
// at element types: 16 bytes a thread, one vector load and store when both tensors and the row length are 16-byte
// aligned (an embedding table of 384 or 768 int8 values), byte by byte otherwise. Bytes of the output outside the
// gathered range are never written, so packed 8-bit and 16-bit neighbours keep their values without the reference's
// read-modify-write of whole words.
//
// An index outside [-axisLen, axisLen) (or an int64 index that does not fit an int32) reads nothing: its output row is
// zero and the position of the index goes into the status word through an atomic minimum, so the smallest offending
// position wins whatever the scheduling (IndexCommon.hlsli:1-5, 12-43). Only the thread of a row's first chunk records.
#include "og_internal.hpp"

#include <algorithm>

namespace og {

namespace {

constexpr int kGatherThreads = 256;

// Index i as the reference reads it (IndexCommon.hlsli:12-24): int64 indices must fit an int32.
__device__ __forceinline__ bool read_index(const void *idx, int64_t i, bool wide, int32_t &v)
{
    if (wide) {
        const uint32_t *w = static_cast<const uint32_t *>(idx) + 2 * i;
        const uint32_t lo = w[0], hi = w[1];
        v = (int32_t)lo;
        return hi == ((int32_t)lo < 0 ? 0xFFFFFFFFu : 0u);
    }
    v = static_cast<const int32_t *>(idx)[i];
    return true;
}

// A possibly negative index mapped into [0, len) (IndexCommon.hlsli:27-43).
__device__ __forceinline__ bool normalize_index(int32_t v, uint32_t len, uint32_t &r)
{
    if (v >= 0) {
        r = (uint32_t)v;
        return r < len;
    }
    const uint32_t a = 0u - (uint32_t)v;
    r = len - a;
    return a <= len;
}

template <bool ALIGNED16>
__global__ __launch_bounds__(kGatherThreads) void k_gather_rows(GatherArgs a)
{
    const int64_t cpr = (a.row_bytes + 15) / 16;   // 16-byte chunks a row
    const int64_t total = a.rows * cpr;
    for (int64_t t = (int64_t)blockIdx.x * kGatherThreads + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * kGatherThreads) {
        const int64_t row = t / cpr, c = t - row * cpr;
        const int64_t o = row / a.count, i = row - o * a.count;
        int32_t v;
        uint32_t r = 0;
        const bool ok = read_index(a.idx, i, a.wide, v) && normalize_index(v, a.axis_len, r);
        if (!ok && c == 0 && a.status) atomicMin(a.status, (uint32_t)i);
        uint8_t *dst = a.out + row * a.row_bytes + 16 * c;
        const uint8_t *src = a.data + (o * (int64_t)a.axis_len + r) * a.row_bytes + 16 * c;
        if constexpr (ALIGNED16) {
            uint4 x = make_uint4(0u, 0u, 0u, 0u);
            if (ok) x = *reinterpret_cast<const uint4 *>(src);
            *reinterpret_cast<uint4 *>(dst) = x;
        } else {
            const int n = (int)min((int64_t)16, a.row_bytes - 16 * c);
            for (int k = 0; k < n; k++) dst[k] = ok ? src[k] : (uint8_t)0;
        }
    }
}

}  // namespace

hipError_t launch_gather(const GatherArgs &a, hipStream_t s, const char **kernel)
{
    const bool aligned = ((uintptr_t)a.data % 16 == 0) && ((uintptr_t)a.out % 16 == 0) && (a.row_bytes % 16 == 0);
    *kernel = aligned ? "gather-rows16" : "gather-bytes";
    const int64_t total = a.rows * ((a.row_bytes + 15) / 16);
    if (total == 0) return hipSuccess;
    // One chunk a thread while the grid stays within 2^20 workgroups; beyond that the threads loop.
    const int64_t wgs = std::min<int64_t>((total + kGatherThreads - 1) / kGatherThreads, int64_t(1) << 20);
    if (aligned) hipLaunchKernelGGL(k_gather_rows<true>, dim3((uint32_t)wgs), dim3(kGatherThreads), 0, s, a);
    else hipLaunchKernelGGL(k_gather_rows<false>, dim3((uint32_t)wgs), dim3(kGatherThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace og
