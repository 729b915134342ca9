// The element-wise and reduction kernels around the int8 product, for gfx950:
//  - DynamicQuantizeLinear: a min/max pass writing one range per workgroup, then a quantize pass in which every
//    workgroup combines those ranges into the scale and zero point and quantizes one block of x with 16-byte loads,
//    writing 16 output bytes per thread (no host round trip, no counters or fences: the kernel boundary orders the
//    passes).
//  - DequantizeLinear / QuantizeLinear and the QLinearMatMul requantization (the int8 epilogue's mode 2).
// Division is IEEE float32 division (correctly rounded: built with -fhip-fp32-correctly-rounded-divide-sqrt and
// denormals kept), rounding is rintf (half to even), and no multiply is contracted into an add (-ffp-contract=off),
// which reproduces the reference's CPU definitions bit for bit.
#include <algorithm>

#include "og_internal.hpp"

namespace og {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool is_nan_bits(float x) { return (__float_as_uint(x) & 0x7FFFFFFFu) > 0x7F800000u; }

// ------------------------------------------------------------------ DynamicQuantizeLinear

constexpr int DQ_THREADS = 256;    // pass 2 (and the element-wise kernels' block of 4096 elements)
constexpr int DQ1_THREADS = 1024;  // pass 1: 16 waves a workgroup, at most kDqMaxGroups workgroups, one per CU

__device__ __forceinline__ void minmax_acc(float v, float &mn, float &mx)
{
    // NaN-ignoring, as the reference compares (v < min, v > max).
    mn = (v < mn) ? v : mn;
    mx = (v > mx) ? v : mx;
}

template <int NT>
__device__ __forceinline__ void block_minmax(float &mn, float &mx, float *smin, float *smax)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        float a = __shfl_xor(mn, o), b = __shfl_xor(mx, o);
        mn = (a < mn) ? a : mn;
        mx = (b > mx) ? b : mx;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { smin[wave] = mn; smax[wave] = mx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < NT / 64; w++) {
            mn = (smin[w] < mn) ? smin[w] : mn;
            mx = (smax[w] > mx) ? smax[w] : mx;
        }
    }
}

// scale = (hi - lo) / 255, zp = clamp(rne(0 - lo / scale), 0, 255), scale 0 -> (1, 0)
// (DynamicQuantize.hlsl:218-232; Int8Tests.cs:600-613).
__device__ void dq_params(float mn, float mx, float &scale, uint32_t &zp)
{
    float lo = fminf(0.0f, mn), hi = fmaxf(0.0f, mx);   // mn/mx are never NaN: a NaN never wins a compare
    scale = (hi - lo) / 255.0f;
    zp = 0u;
    if (scale != 0.0f && isfinite(scale)) {
        float z = rintf(0.0f - lo / scale);
        zp = z < 0.0f ? 0u : (z > 255.0f ? 255u : (uint32_t)z);
    }
    if (scale == 0.0f) {
        scale = 1.0f;
        zp = 0u;
    }
}

// Pass 1: each workgroup's range (NaN-ignoring min and max) over its grid-stride share of x.
__global__ __launch_bounds__(DQ1_THREADS) void k_dq_minmax(const float *x, uint32_t count, float *ranges)
{
    __shared__ float smin[DQ1_THREADS / 64], smax[DQ1_THREADS / 64];
    float mn = __int_as_float(0x7F800000), mx = __int_as_float(0xFF800000);
    const uint32_t tid = blockIdx.x * DQ1_THREADS + threadIdx.x, nthreads = gridDim.x * DQ1_THREADS;
    if (((uintptr_t)x & 15) == 0) {
        const uint32_t n4 = count / 4;
        const f4 *x4 = reinterpret_cast<const f4 *>(x);
        // Four 16-byte loads in flight a thread (each instruction still reads contiguous memory across the wave): a
        // loop of one load a trip waits out a whole memory round trip per trip.
        uint32_t i = tid;
        for (; i + 3 * nthreads < n4; i += 4 * nthreads) {
            f4 v[4];
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = __builtin_nontemporal_load(&x4[i + q * nthreads]);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                minmax_acc(v[q].x, mn, mx); minmax_acc(v[q].y, mn, mx); minmax_acc(v[q].z, mn, mx); minmax_acc(v[q].w, mn, mx);
            }
        }
        for (; i < n4; i += nthreads) {
            f4 v = __builtin_nontemporal_load(&x4[i]);
            minmax_acc(v.x, mn, mx); minmax_acc(v.y, mn, mx); minmax_acc(v.z, mn, mx); minmax_acc(v.w, mn, mx);
        }
        for (uint32_t i = n4 * 4 + tid; i < count; i += nthreads) minmax_acc(x[i], mn, mx);
    } else {
        for (uint32_t i = tid; i < count; i += nthreads) minmax_acc(x[i], mn, mx);
    }
    block_minmax<DQ1_THREADS>(mn, mx, smin, smax);
    if (threadIdx.x == 0) {
        ranges[2 * blockIdx.x] = mn;
        ranges[2 * blockIdx.x + 1] = mx;
    }
}

__device__ __forceinline__ uint32_t dq_one(float x, float scale, float zp)
{
    float v = rintf(x / scale) + zp;
    return is_nan_bits(v) ? 0u : (uint32_t)fminf(fmaxf(v, 0.0f), 255.0f);
}

// Pass 2's scale and zero point, in every workgroup: pass 1's ranges combined (the kernel boundary orders them; min and
// max are order-free, so every workgroup derives the same values). Each thread loads P of the (min, max) pairs before
// the caller's block of x, unconditionally (the buffer always holds P * DQ_THREADS pairs, so no load waits on a
// branch), and ignores the pairs from `groups` on; workgroup 0 also writes the scale and zero point out (the zero point
// one byte, its neighbours untouched). P = 1 over the quantizer's own 256 ranges; up to 4 over a ranged product's.
typedef float f2 __attribute__((ext_vector_type(2)));
static_assert(kDqMaxGroups == DQ_THREADS && kRangesMax == 4 * DQ_THREADS, "the ranges split evenly over the threads");

template <int P>
__device__ __forceinline__ void dq_load_ranges(const float *ranges, f2 (&r)[P])
{
#pragma unroll
    for (int q = 0; q < P; q++) r[q] = reinterpret_cast<const f2 *>(ranges)[threadIdx.x + q * DQ_THREADS];
}

template <int P>
__device__ __forceinline__ void dq_combine(const f2 (&r)[P], uint32_t groups, float *smin, float *smax,
                                           float *sparam, float *scale_out, uint8_t *zero_out, float &scale, float &zpf)
{
    float mn = __int_as_float(0x7F800000), mx = __int_as_float(0xFF800000);
#pragma unroll
    for (int q = 0; q < P; q++) {
        if (threadIdx.x + q * DQ_THREADS < groups) {
            mn = (r[q].x < mn) ? r[q].x : mn;
            mx = (r[q].y > mx) ? r[q].y : mx;
        }
    }
    block_minmax<DQ_THREADS>(mn, mx, smin, smax);
    if (threadIdx.x == 0) {
        float sc;
        uint32_t zp;
        dq_params(mn, mx, sc, zp);
        sparam[0] = sc;
        sparam[1] = (float)zp;
        if (blockIdx.x == 0) {
            *scale_out = sc;
            *zero_out = (uint8_t)zp;
        }
    }
    __syncthreads();
    scale = sparam[0];
    zpf = sparam[1];
}

// Pass 2: workgroup b quantizes elements 4096 b .. 4096 b + 4095. It requests the ranges, then its block of x, and
// combines the ranges while x is still on its way from HBM. In a whole block with x and y 16-byte aligned, lane l of
// wave w takes elements 1024 w + 256 c + 4 l .. + 3 (c = 0..3) with one 16-byte load and one 4-byte store each, so
// every instruction covers one contiguous span across the wave; otherwise lane t takes elements t, t + 256, ...
template <int P>
__global__ __launch_bounds__(DQ_THREADS) void k_dq_quantize(const float *x, uint8_t *y, uint32_t count,
                                                            const float *ranges, uint32_t groups, float *scale_out,
                                                            uint8_t *zero_out)
{
    __shared__ float smin[DQ_THREADS / 64], smax[DQ_THREADS / 64], sparam[2];
    f2 r[P];
    dq_load_ranges<P>(ranges, r);
    const uint64_t blk = (uint64_t)blockIdx.x * 4096;
    float scale, zp;
    if ((((uintptr_t)x | (uintptr_t)y) & 15) == 0 && blk + 4096 <= count) {
        const uint32_t lane_off = (threadIdx.x >> 6) * 1024u + (threadIdx.x & 63u) * 4u;
        f4 v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(x + blk + lane_off + 256 * c));
        dq_combine(r, groups, smin, smax, sparam, scale_out, zero_out, scale, zp);
#pragma unroll
        for (int c = 0; c < 4; c++)
            *reinterpret_cast<uint32_t *>(y + blk + lane_off + 256 * c) =
                dq_one(v[c].x, scale, zp) | (dq_one(v[c].y, scale, zp) << 8) | (dq_one(v[c].z, scale, zp) << 16) |
                (dq_one(v[c].w, scale, zp) << 24);
    } else {
        dq_combine(r, groups, smin, smax, sparam, scale_out, zero_out, scale, zp);
        for (uint64_t i = blk + threadIdx.x; i < blk + 4096 && i < count; i += DQ_THREADS) y[i] = (uint8_t)dq_one(x[i], scale, zp);
    }
}

static uint32_t dq_groups(uint32_t count)
{
    // About 64 KB of x per workgroup, at most kDqMaxGroups.
    uint32_t g = (count + 16383) / 16384;
    return g < 1 ? 1 : (g > (uint32_t)kDqMaxGroups ? (uint32_t)kDqMaxGroups : g);
}

hipError_t launch_dynamic_quantize(const DqArgs &d, const Workspace &ws, hipStream_t s, const char **kernel, int step)
{
    const uint32_t groups = dq_groups(d.count);
    if (step == 0) {
        *kernel = "dq-minmax";
        hipLaunchKernelGGL(k_dq_minmax, dim3(groups), dim3(DQ1_THREADS), 0, s, d.x, d.count, ws.dq_ranges);
    } else {
        *kernel = "dq-quantize";
        // One block of 4096 elements a workgroup (at most 2^20 workgroups for a 32-bit count).
        const uint32_t wgs = d.count == 0 ? 1u : (uint32_t)(((uint64_t)d.count + 4095) / 4096);
        hipLaunchKernelGGL(k_dq_quantize<1>, dim3(wgs), dim3(DQ_THREADS), 0, s, d.x, d.y, d.count,
                           (const float *)ws.dq_ranges, groups, d.scale, d.zero);
    }
    return hipGetLastError();
}

hipError_t launch_dynamic_quantize_ranged(const DqArgs &d, const float *ranges, uint32_t groups, hipStream_t s,
                                          const char **kernel)
{
    *kernel = "dq-quantize";
    const uint32_t wgs = d.count == 0 ? 1u : (uint32_t)(((uint64_t)d.count + 4095) / 4096);
#define OG_DQR(P) hipLaunchKernelGGL(k_dq_quantize<P>, dim3(wgs), dim3(DQ_THREADS), 0, s, d.x, d.y, d.count, ranges, \
                                     groups, d.scale, d.zero)
    if (groups <= (uint32_t)DQ_THREADS) OG_DQR(1);
    else if (groups <= 2u * DQ_THREADS) OG_DQR(2);
    else OG_DQR(4);
#undef OG_DQR
    return hipGetLastError();
}

hipError_t launch_range_pass(const float *x, uint32_t count, float *ranges, hipStream_t s, const char **kernel,
                             uint32_t *groups)
{
    *kernel = "dq-minmax";
    *groups = dq_groups(count);
    hipLaunchKernelGGL(k_dq_minmax, dim3(*groups), dim3(DQ1_THREADS), 0, s, x, count, ranges);
    return hipGetLastError();
}

// ------------------------------------------------------------------ DequantizeLinear / QuantizeLinear
//
// Both are element-wise streams; a workgroup of 256 threads takes 4096 consecutive elements. When every tensor the
// pass streams starts 16-byte aligned, lane l of wave w moves elements 1024 w + 256 c + 4 l .. + 3 for c = 0..3 with
// one vector access each (4, 8 or 16 bytes): every instruction then reads or writes one contiguous span across the
// wave, which is what streams at HBM rate (16 contiguous elements a lane, a 64-byte stride across the wave, runs at
// half of it). Otherwise, and in the tensor's last partial block, lane t takes elements t, t + 256, ... one at a time.
// The scale (and zero point) of element j is the one at axis index (j / inner) % axis_len: found once a run of 4.

constexpr int kEwThreads = 256, kEwBlock = 4096;

typedef int32_t i4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

// binary32 -> binary16 bits: the hardware conversion (round to nearest even, binary16 subnormals kept, overflow to
// infinity), with every NaN made the quiet NaN 0x7E00 of its sign, as the reference's integer conversion writes it.
__device__ __forceinline__ uint16_t f2h(float f)
{
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
    return is_nan_bits(f) ? (uint16_t)(((__float_as_uint(f) >> 16) & 0x8000u) | 0x7E00u) : h;
}

template <int KIND>
__device__ __forceinline__ int32_t load_q(const void *p, uint32_t i)
{
    if (KIND == OG_KIND_U8) return (int32_t) static_cast<const uint8_t *>(p)[i];
    if (KIND == OG_KIND_I8) return (int32_t) static_cast<const int8_t *>(p)[i];
    return static_cast<const int32_t *>(p)[i];
}

// The axis index of a run of consecutive elements, starting at element j and moved one element by step().
template <bool PER_AXIS>
struct AxisWalk {
    uint32_t a = 0, r = 0;
    __device__ __forceinline__ AxisWalk(const DequantArgs &d, uint32_t j)
    {
        if (PER_AXIS) {
            if (d.inner == 1) {
                a = j % d.axis_len;
            } else {
                const uint32_t q = j / d.inner;
                r = j - q * d.inner;
                a = q % d.axis_len;
            }
        }
    }
    __device__ __forceinline__ void step(const DequantArgs &d)
    {
        if (PER_AXIS && ++r == d.inner) {
            r = 0;
            if (++a == d.axis_len) a = 0;
        }
    }
};

// The first element of lane run c (0..3) of this thread in an aligned block.
__device__ __forceinline__ uint32_t ew_run(uint32_t block, int c)
{
    return block * kEwBlock + (threadIdx.x >> 6) * 1024u + (uint32_t)c * 256u + (threadIdx.x & 63u) * 4u;
}

// The scale and zero point at axis index a.
template <int KIND>
struct DequantParam {
    int32_t zp;
    float scale;
    __device__ __forceinline__ DequantParam(const DequantArgs &d, uint32_t a)
        : zp(d.has_zero ? load_q<KIND>(d.zero, a) : 0), scale(d.scale[a]) {}
};

// y = fl((x - zp) * scale), the difference wrapping in 32 bits (DequantizeKernels.cs:64-150).
template <int KIND>
__device__ __forceinline__ float dequant_one(int32_t x, const DequantParam<KIND> &p)
{
    return __fmul_rn((float)(int32_t)((uint32_t)x - (uint32_t)p.zp), p.scale);
}

template <bool F16>
__device__ __forceinline__ void store_y(void *out, uint32_t j, float y)
{
    if (F16) static_cast<uint16_t *>(out)[j] = f2h(y);
    else static_cast<float *>(out)[j] = y;
}

// The scales and zero points of a run of four elements whose axis indices are a .. a + 3 (per column: inner 1, an
// axis length that is a multiple of 4, the scales 16-byte and the zero points 4-element aligned): one vector load each.
template <int KIND>
__device__ __forceinline__ void column_params(const DequantArgs &d, uint32_t a, DequantParam<KIND> p[4])
{
    const f4 s = *reinterpret_cast<const f4 *>(d.scale + a);
    int32_t z[4] = {0, 0, 0, 0};
    if (d.has_zero) {
        if constexpr (KIND == OG_KIND_I32) {
            const i4v v = *reinterpret_cast<const i4v *>(static_cast<const int32_t *>(d.zero) + a);
            z[0] = v.x; z[1] = v.y; z[2] = v.z; z[3] = v.w;
        } else {
            const uint32_t v = *reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(d.zero) + a);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t b = (v >> (8 * e)) & 0xFFu;
                z[e] = KIND == OG_KIND_I8 ? (int32_t)(int8_t)b : (int32_t)b;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        p[e].zp = z[e];
        p[e].scale = s[e];
    }
}

// PER: 0 one scale for the tensor, 1 per axis, 2 per column in runs of four (column_params' conditions).
template <int KIND, bool F16, int PER, bool VEC>
__device__ __forceinline__ void dequant_block(const DequantArgs &d, uint32_t blk)
{
    constexpr bool PER_AXIS = PER != 0;
    if (VEC && ((uint64_t)blk + 1) * kEwBlock <= d.count) {
        int32_t q[4][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {   // all loads first, so that the four are in flight together
            const uint32_t j = ew_run(blk, c);
            if constexpr (KIND == OG_KIND_I32) {
                const i4v v = __builtin_nontemporal_load(reinterpret_cast<const i4v *>(static_cast<const int32_t *>(d.x) + j));
                q[c][0] = v.x; q[c][1] = v.y; q[c][2] = v.z; q[c][3] = v.w;
            } else {
                const uint32_t v = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(d.x) + j));
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t b = (v >> (8 * e)) & 0xFFu;
                    q[c][e] = KIND == OG_KIND_I8 ? (int32_t)(int8_t)b : (int32_t)b;
                }
            }
        }
        const DequantParam<KIND> p0(d, 0);   // the one scale and zero point of a per-tensor pass
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t j = ew_run(blk, c);
            float y[4];
            if constexpr (PER == 2) {
                DequantParam<KIND> p[4] = {p0, p0, p0, p0};
                column_params<KIND>(d, j % d.axis_len, p);
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = dequant_one<KIND>(q[c][e], p[e]);
            } else {
                AxisWalk<PER_AXIS> w(d, j);
#pragma unroll
                for (int e = 0; e < 4; e++, w.step(d)) y[e] = dequant_one<KIND>(q[c][e], PER_AXIS ? DequantParam<KIND>(d, w.a) : p0);
            }
            if constexpr (F16) {
                const u2v h = {(uint32_t)f2h(y[0]) | ((uint32_t)f2h(y[1]) << 16), (uint32_t)f2h(y[2]) | ((uint32_t)f2h(y[3]) << 16)};
                *reinterpret_cast<u2v *>(static_cast<uint16_t *>(d.out) + j) = h;
            } else {
                *reinterpret_cast<f4 *>(static_cast<float *>(d.out) + j) = f4{y[0], y[1], y[2], y[3]};
            }
        }
    } else {
#pragma unroll 4
        for (int e = 0; e < kEwBlock / kEwThreads; e++) {
            const uint64_t j = (uint64_t)blk * kEwBlock + (uint64_t)e * kEwThreads + threadIdx.x;
            if (j < d.count) {
                const AxisWalk<PER_AXIS> w(d, (uint32_t)j);
                store_y<F16>(d.out, (uint32_t)j, dequant_one<KIND>(load_q<KIND>(d.x, (uint32_t)j), DequantParam<KIND>(d, w.a)));
            }
        }
    }
}

template <int KIND, bool F16, int PER, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_dequantize(DequantArgs d)
{
    dequant_block<KIND, F16, PER, VEC>(d, blockIdx.x);
}

// Up to kDqBatch dequantize passes of one shape in one launch: pass blockIdx.y over its blocks blockIdx.x.
struct DequantBatch {
    DequantArgs d[kDqBatch];
};

template <int KIND, bool F16, int PER, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_dequantize_batch(DequantBatch b)
{
    dequant_block<KIND, F16, PER, VEC>(b.d[blockIdx.y], blockIdx.x);
}

static bool ew_aligned(const void *a, const void *b) { return (((uintptr_t)a | (uintptr_t)b) & 15) == 0; }

static dim3 ew_grid(uint32_t count) { return dim3((uint32_t)(((uint64_t)count + kEwBlock - 1) / kEwBlock)); }

// The variant a pass takes: PER 2 (per column in runs of four) when the scale and zero point are aligned for it.
template <int KIND>
static int dequant_per(const DequantArgs &d)
{
    const uintptr_t zero_align = KIND == OG_KIND_I32 ? 15 : 3;
    const bool columns = d.per_axis && d.inner == 1 && d.axis_len % 4 == 0 && ((uintptr_t)d.scale & 15) == 0 &&
                         (!d.has_zero || ((uintptr_t)d.zero & zero_align) == 0);
    return columns ? 2 : d.per_axis ? 1 : 0;
}

// n passes (n = 1: d[0] alone, k_dequantize; else k_dequantize_batch over the first n), all taking variant (per, vec).
template <int KIND, bool F16>
static void launch_dequantize_as(const DequantArgs *d, int n, int per, bool vec, hipStream_t s)
{
    const dim3 block(kEwThreads);
#define OG_DQ(P, V)                                                                                                   \
    do {                                                                                                              \
        if (n == 1) {                                                                                                 \
            hipLaunchKernelGGL((k_dequantize<KIND, F16, P, V>), ew_grid(d[0].count), block, 0, s, d[0]);              \
        } else {                                                                                                      \
            DequantBatch b{};                                                                                         \
            for (int i = 0; i < n; i++) b.d[i] = d[i];                                                                \
            hipLaunchKernelGGL((k_dequantize_batch<KIND, F16, P, V>), dim3(ew_grid(d[0].count).x, (uint32_t)n), block, \
                               0, s, b);                                                                              \
        }                                                                                                             \
    } while (0)
    if (per == 2) OG_DQ(2, true);
    else if (per == 1) { if (vec) OG_DQ(1, true); else OG_DQ(1, false); }
    else { if (vec) OG_DQ(0, true); else OG_DQ(0, false); }
#undef OG_DQ
}

hipError_t launch_dequantize(const DequantArgs &d, int kind, bool f16_out, hipStream_t s, const char **kernel)
{
    return launch_dequantize_batch(&d, 1, kind, f16_out, s, kernel);
}

hipError_t launch_dequantize_batch(const DequantArgs *d, int n, int kind, bool f16_out, hipStream_t s,
                                   const char **kernel)
{
    // Every pass of a batch has the count, axis and zero-point form of the first (the caller checks); the batch takes
    // the variant every pass can take.
    bool vec = true;
    int per = 2;
    for (int i = 0; i < n; i++) {
        vec = vec && ew_aligned(d[i].x, d[i].out);
        const int p = kind == OG_KIND_I32 ? dequant_per<OG_KIND_I32>(d[i]) : dequant_per<OG_KIND_U8>(d[i]);
        per = std::min(per, p);
    }
    if (per == 2 && !vec) per = 1;
    *kernel = n > 1 ? (f16_out ? (vec ? "dequantize4-f16-batch" : "dequantize-f16-batch") : (vec ? "dequantize4-f32-batch" : "dequantize-f32-batch"))
                    : (f16_out ? (vec ? "dequantize4-f16" : "dequantize-f16") : (vec ? "dequantize4-f32" : "dequantize-f32"));
    if (n <= 0 || d[0].count == 0) return hipSuccess;
    for (int i0 = 0; i0 < n; i0 += kDqBatch) {
        const int m = std::min(n - i0, kDqBatch);
        switch (kind * 2 + (f16_out ? 1 : 0)) {
        case 0: launch_dequantize_as<OG_KIND_U8, false>(d + i0, m, per, vec, s); break;
        case 1: launch_dequantize_as<OG_KIND_U8, true>(d + i0, m, per, vec, s); break;
        case 2: launch_dequantize_as<OG_KIND_I8, false>(d + i0, m, per, vec, s); break;
        case 3: launch_dequantize_as<OG_KIND_I8, true>(d + i0, m, per, vec, s); break;
        case 4: launch_dequantize_as<OG_KIND_I32, false>(d + i0, m, per, vec, s); break;
        default: launch_dequantize_as<OG_KIND_I32, true>(d + i0, m, per, vec, s); break;
        }
    }
    return hipGetLastError();
}

// The scale and zero point (as a float) at axis index a.
template <bool SIGNED>
struct QuantParam {
    float zp, scale;
    __device__ __forceinline__ QuantParam(const DequantArgs &d, uint32_t a)
        : zp(!d.has_zero ? 0.0f
                         : (float)(SIGNED ? (int32_t) static_cast<const int8_t *>(d.zero)[a]
                                          : (int32_t) static_cast<const uint8_t *>(d.zero)[a])),
          scale(d.scale[a]) {}
};

// y = saturate(rne(x / scale) + zp), NaN to the lowest value (DequantizeKernels.cs:204-272).
template <bool SIGNED>
__device__ __forceinline__ uint32_t quant_one(float x, const QuantParam<SIGNED> &p)
{
    const float lo = SIGNED ? -128.0f : 0.0f, hi = SIGNED ? 127.0f : 255.0f;
    float v = __fadd_rn(rintf(x / p.scale), p.zp);
    if (is_nan_bits(v)) v = lo;
    return (uint32_t)(int32_t)fminf(fmaxf(v, lo), hi) & 0xFFu;
}

template <bool F16>
__device__ __forceinline__ float load_x(const void *p, uint32_t j)
{
    return F16 ? (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t *>(p)[j]) : static_cast<const float *>(p)[j];
}

template <bool SIGNED, bool F16, bool PER_AXIS, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_quantize(DequantArgs d)
{
    uint8_t *out = static_cast<uint8_t *>(d.out);
    if (VEC && ((uint64_t)blockIdx.x + 1) * kEwBlock <= d.count) {
        float x[4][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t j = ew_run(blockIdx.x, c);
            if constexpr (F16) {
                const u2v v = __builtin_nontemporal_load(reinterpret_cast<const u2v *>(static_cast<const uint16_t *>(d.x) + j));
#pragma unroll
                for (int e = 0; e < 4; e++)
                    x[c][e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[e >> 1] >> (16 * (e & 1))));
            } else {
                const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(static_cast<const float *>(d.x) + j));
                x[c][0] = v.x; x[c][1] = v.y; x[c][2] = v.z; x[c][3] = v.w;
            }
        }
        const QuantParam<SIGNED> p0(d, 0);   // the one scale and zero point of a per-tensor pass
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t j = ew_run(blockIdx.x, c);
            AxisWalk<PER_AXIS> w(d, j);
            uint32_t y = 0;
#pragma unroll
            for (int e = 0; e < 4; e++, w.step(d)) y |= quant_one<SIGNED>(x[c][e], PER_AXIS ? QuantParam<SIGNED>(d, w.a) : p0) << (8 * e);
            *reinterpret_cast<uint32_t *>(out + j) = y;
        }
    } else {
#pragma unroll 4
        for (int e = 0; e < kEwBlock / kEwThreads; e++) {
            const uint64_t j = (uint64_t)blockIdx.x * kEwBlock + (uint64_t)e * kEwThreads + threadIdx.x;
            if (j < d.count) {
                const AxisWalk<PER_AXIS> w(d, (uint32_t)j);
                out[j] = (uint8_t)quant_one<SIGNED>(load_x<F16>(d.x, (uint32_t)j), QuantParam<SIGNED>(d, w.a));
            }
        }
    }
}

template <bool SIGNED, bool F16>
static void launch_quantize_as(const DequantArgs &d, bool vec, hipStream_t s)
{
    const dim3 grid = ew_grid(d.count), block(kEwThreads);
    if (d.per_axis) {
        if (vec) hipLaunchKernelGGL((k_quantize<SIGNED, F16, true, true>), grid, block, 0, s, d);
        else hipLaunchKernelGGL((k_quantize<SIGNED, F16, true, false>), grid, block, 0, s, d);
    } else {
        if (vec) hipLaunchKernelGGL((k_quantize<SIGNED, F16, false, true>), grid, block, 0, s, d);
        else hipLaunchKernelGGL((k_quantize<SIGNED, F16, false, false>), grid, block, 0, s, d);
    }
}

hipError_t launch_quantize(const DequantArgs &d, bool is_signed, bool f16_in, hipStream_t s, const char **kernel)
{
    const bool vec = ew_aligned(d.x, d.out);
    static const char *names[2][2][2] = {{{"quantize-f32-u8", "quantize-f16-u8"}, {"quantize-f32-i8", "quantize-f16-i8"}},
                                         {{"quantize4-f32-u8", "quantize4-f16-u8"}, {"quantize4-f32-i8", "quantize4-f16-i8"}}};
    *kernel = names[vec][is_signed][f16_in];
    if (d.count == 0) return hipSuccess;
    if (is_signed) {
        if (f16_in) launch_quantize_as<true, true>(d, vec, s);
        else launch_quantize_as<true, false>(d, vec, s);
    } else {
        if (f16_in) launch_quantize_as<false, true>(d, vec, s);
        else launch_quantize_as<false, false>(d, vec, s);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ Int8Gemm's second pass (Int8Epilogue.hlsl)

__global__ __launch_bounds__(256) void k_int8_epilogue(EpilogueArgs e)
{
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    if (t >= e.count) return;
    const uint32_t col = t % e.n;
    if (e.mode == 3) {
        float *o = static_cast<float *>(e.out);
        o[t] = __fadd_rn(o[t], e.fbias[col]);
        return;
    }
    uint32_t acc = (uint32_t)e.acc[t];
    if (e.flags & 1u) acc += (uint32_t)e.bias[col];
    if (e.mode == 0) {
        static_cast<int32_t *>(e.out)[t] = (int32_t)acc;
        return;
    }
    const float s = e.scale[(e.flags & 2u) ? col : 0u];
    if (e.mode == 1) {
        static_cast<float *>(e.out)[t] = __fmul_rn((float)(int32_t)acc, s);
        return;
    }
    // Mode 2 (Int8Epilogue.hlsl:54-68): NaN to the lowest value; rne; clamp to [lo - zp, hi - zp]; + zp.
    static_cast<uint8_t *>(e.out)[t] = (uint8_t)requantize_byte(acc, s, e.zero_point, (e.flags & 8u) != 0u);
}

hipError_t launch_int8_epilogue(const EpilogueArgs &e, hipStream_t s, const char **kernel)
{
    *kernel = "int8-epilogue";
    if (e.count == 0) return hipSuccess;
    hipLaunchKernelGGL(k_int8_epilogue, dim3((e.count + 255) / 256), dim3(256), 0, s, e);
    return hipGetLastError();
}

// ------------------------------------------------------------------ utilities

__global__ __launch_bounds__(256) void k_fill_bytes(uint8_t *dst, uint8_t value, uint64_t bytes)
{
    const uint64_t i = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (i + 16 <= bytes && ((uintptr_t)(dst + i) & 15) == 0) {
        uint32_t w = value * 0x01010101u;
        *reinterpret_cast<uint4 *>(dst + i) = make_uint4(w, w, w, w);
        return;
    }
    for (uint64_t k = i; k < i + 16 && k < bytes; k++) dst[k] = value;
}

hipError_t launch_fill_bytes(void *dst, uint8_t value, uint64_t bytes, hipStream_t s)
{
    if (bytes == 0) return hipSuccess;
    uint64_t threads = (bytes + 15) / 16;
    hipLaunchKernelGGL(k_fill_bytes, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, s,
                       static_cast<uint8_t *>(dst), value, bytes);
    return hipGetLastError();
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// The same streams as the CPU oracle's ora_synth_* (bit-identical for the integer kinds).
__global__ __launch_bounds__(256) void k_synth(int kind, uint64_t key, void *out, uint64_t count, double lo, double hi)
{
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    const uint64_t x = splitmix64(key + i);
    if (kind == 2) {
        const uint64_t y = splitmix64(x ^ 0xD1B54A32D192ED03ull);
        const double u1 = (double)((x >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(y >> 11) * 0x1.0p-53;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        static_cast<float *>(out)[i] = (float)(lo + hi * z);
        return;
    }
    const int64_t l = (int64_t)lo, h = (int64_t)hi;
    const uint64_t range = (uint64_t)(h - l + 1);
    const int64_t v = l + (int64_t)(((x >> 32) * range) >> 32);
    if (kind == 0) static_cast<uint8_t *>(out)[i] = (uint8_t)v;
    else static_cast<int32_t *>(out)[i] = (int32_t)v;
}

hipError_t launch_synth(int kind, uint64_t seed, uint32_t tensor, void *out, uint64_t count, double lo, double hi,
                        hipStream_t s)
{
    if (count == 0) return hipSuccess;
    uint64_t key;
    {
        uint64_t x = (seed << 32) ^ (uint64_t)tensor;
        x += 0x9E3779B97F4A7C15ull;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        key = x ^ (x >> 31);
    }
    const uint64_t chunk = 256ull * 65535ull * 256ull;   // elements per launch
    for (uint64_t off = 0; off < count; off += chunk) {
        uint64_t n = count - off < chunk ? count - off : chunk;
        size_t esize = kind == 0 ? 1 : 4;
        hipLaunchKernelGGL(k_synth, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, kind, key + off,
                           static_cast<uint8_t *>(out) + off * esize, n, lo, hi);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

__global__ __launch_bounds__(256) void k_col_absmax_scale(const float *w, uint32_t rows, uint32_t cols, float divisor,
                                                          float *scale)
{
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    float m = 0.0f;
    for (uint32_t r = 0; r < rows; r++) m = fmaxf(m, fabsf(w[(uint64_t)r * cols + c]));
    scale[c] = m / divisor;
}

hipError_t launch_col_absmax_scale(const float *w, uint32_t rows, uint32_t cols, float divisor, float *scale,
                                   hipStream_t s)
{
    if (cols == 0) return hipSuccess;
    hipLaunchKernelGGL(k_col_absmax_scale, dim3((cols + 255) / 256), dim3(256), 0, s, w, rows, cols, divisor, scale);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_scale_product(const float *a, const float *b, uint32_t n, float *out)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = __fmul_rn(a[0], b[i]);
}

hipError_t launch_scale_product(const float *a, const float *b, uint32_t n, float *out, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_scale_product, dim3((n + 255) / 256), dim3(256), 0, s, a, b, n, out);
    return hipGetLastError();
}

}  // namespace og
