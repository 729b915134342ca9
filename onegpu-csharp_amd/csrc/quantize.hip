// The element-wise and reduction kernels around the int8 product, for gfx950:
//  - DynamicQuantizeLinear: a min/max pass writing one range per workgroup, then a quantize pass in which every
//    workgroup combines those ranges into the scale and zero point and streams x again with 16-byte loads, writing 16
//    output bytes per thread (no host round trip, no counters or fences: the kernel boundary orders the passes).
//  - DequantizeLinear / QuantizeLinear and the QLinearMatMul requantization (the int8 epilogue's mode 2).
// Division is IEEE float32 division (correctly rounded: built with -fhip-fp32-correctly-rounded-divide-sqrt and
// denormals kept), rounding is rintf (half to even), and no multiply is contracted into an add (-ffp-contract=off),
// which reproduces the reference's CPU definitions bit for bit.
#include "og_internal.hpp"

namespace og {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool is_nan_bits(float x) { return (__float_as_uint(x) & 0x7FFFFFFFu) > 0x7F800000u; }

// ------------------------------------------------------------------ DynamicQuantizeLinear

constexpr int DQ_THREADS = 256;

__device__ __forceinline__ void minmax_acc(float v, float &mn, float &mx)
{
    // NaN-ignoring, as the reference compares (v < min, v > max).
    mn = (v < mn) ? v : mn;
    mx = (v > mx) ? v : mx;
}

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
        for (int w = 1; w < DQ_THREADS / 64; w++) {
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
__global__ __launch_bounds__(DQ_THREADS) void k_dq_minmax(const float *x, uint32_t count, float *ranges)
{
    __shared__ float smin[DQ_THREADS / 64], smax[DQ_THREADS / 64];
    float mn = __int_as_float(0x7F800000), mx = __int_as_float(0xFF800000);
    const uint32_t tid = blockIdx.x * DQ_THREADS + threadIdx.x, nthreads = gridDim.x * DQ_THREADS;
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
    block_minmax(mn, mx, smin, smax);
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

// Pass 2: every workgroup combines pass 1's ranges (the kernel boundary orders them; min and max are order-free, so
// every workgroup derives the same scale and zero point) and quantizes its grid-stride share of x, 16 elements a
// thread with 16-byte loads and one 16-byte store when x and y are 16-byte aligned. Workgroup 0 writes the scale and
// the zero point (one byte, its neighbours untouched).
__global__ __launch_bounds__(DQ_THREADS) void k_dq_quantize(const float *x, uint8_t *y, uint32_t count,
                                                            const float *ranges, uint32_t groups, float *scale_out,
                                                            uint8_t *zero_out)
{
    __shared__ float smin[DQ_THREADS / 64], smax[DQ_THREADS / 64], sparam[2];
    float mn = __int_as_float(0x7F800000), mx = __int_as_float(0xFF800000);
    for (uint32_t g = threadIdx.x; g < groups; g += DQ_THREADS) {
        const float a = ranges[2 * g], b = ranges[2 * g + 1];
        mn = (a < mn) ? a : mn;
        mx = (b > mx) ? b : mx;
    }
    block_minmax(mn, mx, smin, smax);
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
    const float scale = sparam[0], zp = sparam[1];
    const bool vec = (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
    const uint64_t stride = (uint64_t)gridDim.x * DQ_THREADS * 16;
    for (uint64_t i0 = ((uint64_t)blockIdx.x * DQ_THREADS + threadIdx.x) * 16; i0 < count; i0 += stride) {
        if (vec && i0 + 16 <= count) {
            const f4 *x4 = reinterpret_cast<const f4 *>(x + i0);
            uint32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                f4 v = __builtin_nontemporal_load(&x4[q]);
                w[q] = dq_one(v.x, scale, zp) | (dq_one(v.y, scale, zp) << 8) | (dq_one(v.z, scale, zp) << 16) |
                       (dq_one(v.w, scale, zp) << 24);
            }
            *reinterpret_cast<uint4 *>(y + i0) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (uint64_t i = i0; i < i0 + 16 && i < count; i++) y[i] = (uint8_t)dq_one(x[i], scale, zp);
        }
    }
}

static uint32_t dq_groups(uint32_t count)
{
    // About 16 KB of x per workgroup, at most kDqMaxGroups.
    uint32_t g = (count + 4095) / 4096;
    return g < 1 ? 1 : (g > (uint32_t)kDqMaxGroups ? (uint32_t)kDqMaxGroups : g);
}

hipError_t launch_dynamic_quantize(const DqArgs &d, const Workspace &ws, hipStream_t s, const char **kernel, int step)
{
    const uint32_t groups = dq_groups(d.count);
    if (step == 0) {
        *kernel = "dq-minmax";
        hipLaunchKernelGGL(k_dq_minmax, dim3(groups), dim3(DQ_THREADS), 0, s, d.x, d.count, ws.dq_ranges);
    } else {
        *kernel = "dq-quantize";
        // 16 elements a thread, at most 2048 workgroups (each re-reads the ranges).
        const uint64_t threads = ((uint64_t)d.count + 15) / 16;
        uint64_t wgs = (threads + DQ_THREADS - 1) / DQ_THREADS;
        wgs = wgs > 2048 ? 2048 : wgs;
        hipLaunchKernelGGL(k_dq_quantize, dim3((uint32_t)wgs), dim3(DQ_THREADS), 0, s, d.x, d.y, d.count,
                           (const float *)ws.dq_ranges, groups, d.scale, d.zero);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ DequantizeLinear / QuantizeLinear

// binary32 -> binary16, round to nearest even, overflow to infinity, NaN to a quiet NaN of the same sign
// (the integer conversion of Common.hlsl:52-92, so the bits do not depend on the hardware converter).
__device__ __forceinline__ uint16_t f2h(float f)
{
    uint32_t x = __float_as_uint(f);
    uint32_t s = (x >> 16) & 0x8000u, a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(s | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t)(s | 0x7C00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t)s;
        uint32_t e = a >> 23, mant = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t m = mant >> sh, rem = mant & ((1u << sh) - 1u), halfway = 1u << (sh - 1u);
        if (rem > halfway || (rem == halfway && (m & 1u) != 0u)) m += 1u;
        return (uint16_t)(s | m);
    }
    uint32_t r = a - 0x38000000u;
    r += 0xFFFu + ((r >> 13) & 1u);
    return (uint16_t)(s | (r >> 13));
}

template <int KIND>
__device__ __forceinline__ int32_t load_q(const void *p, uint32_t i)
{
    if (KIND == OG_KIND_U8) return (int32_t)static_cast<const uint8_t *>(p)[i];
    if (KIND == OG_KIND_I8) return (int32_t) static_cast<const int8_t *>(p)[i];
    return static_cast<const int32_t *>(p)[i];
}

template <int KIND, bool F16>
__global__ __launch_bounds__(256) void k_dequantize(DequantArgs d)
{
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= d.count) return;
    const uint32_t a = d.per_axis ? (j / d.inner) % d.axis_len : 0u;
    const int32_t zp = d.has_zero ? load_q<KIND>(d.zero, a) : 0;
    const int32_t q = (int32_t)((uint32_t)load_q<KIND>(d.x, j) - (uint32_t)zp);   // wraps in 32 bits
    const float y = __fmul_rn((float)q, d.scale[a]);
    if (F16) static_cast<uint16_t *>(d.out)[j] = f2h(y);
    else static_cast<float *>(d.out)[j] = y;
}

hipError_t launch_dequantize(const DequantArgs &d, int kind, bool f16_out, hipStream_t s, const char **kernel)
{
    *kernel = f16_out ? "dequantize-f16" : "dequantize-f32";
    if (d.count == 0) return hipSuccess;
    dim3 grid((d.count + 255) / 256), block(256);
#define OG_DQ(K, H) hipLaunchKernelGGL((k_dequantize<K, H>), grid, block, 0, s, d)
    switch (kind * 2 + (f16_out ? 1 : 0)) {
    case 0: OG_DQ(OG_KIND_U8, false); break;
    case 1: OG_DQ(OG_KIND_U8, true); break;
    case 2: OG_DQ(OG_KIND_I8, false); break;
    case 3: OG_DQ(OG_KIND_I8, true); break;
    case 4: OG_DQ(OG_KIND_I32, false); break;
    default: OG_DQ(OG_KIND_I32, true); break;
    }
#undef OG_DQ
    return hipGetLastError();
}

template <bool SIGNED, bool F16>
__global__ __launch_bounds__(256) void k_quantize(DequantArgs d)
{
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= d.count) return;
    const uint32_t a = d.per_axis ? (j / d.inner) % d.axis_len : 0u;
    int32_t zp = 0;
    if (d.has_zero) zp = SIGNED ? (int32_t) static_cast<const int8_t *>(d.zero)[a] : (int32_t) static_cast<const uint8_t *>(d.zero)[a];
    const float x = F16 ? (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t *>(d.x)[j])
                        : static_cast<const float *>(d.x)[j];
    const float lo = SIGNED ? -128.0f : 0.0f, hi = SIGNED ? 127.0f : 255.0f;
    float v = __fadd_rn(rintf(x / d.scale[a]), (float)zp);
    if (is_nan_bits(v)) v = lo;
    const int32_t q = (int32_t)fminf(fmaxf(v, lo), hi);
    static_cast<uint8_t *>(d.out)[j] = (uint8_t)q;
}

hipError_t launch_quantize(const DequantArgs &d, bool is_signed, bool f16_in, hipStream_t s, const char **kernel)
{
    *kernel = is_signed ? (f16_in ? "quantize-f16-i8" : "quantize-f32-i8") : (f16_in ? "quantize-f16-u8" : "quantize-f32-u8");
    if (d.count == 0) return hipSuccess;
    dim3 grid((d.count + 255) / 256), block(256);
    if (is_signed) {
        if (f16_in) hipLaunchKernelGGL((k_quantize<true, true>), grid, block, 0, s, d);
        else hipLaunchKernelGGL((k_quantize<true, false>), grid, block, 0, s, d);
    } else {
        if (f16_in) hipLaunchKernelGGL((k_quantize<false, true>), grid, block, 0, s, d);
        else hipLaunchKernelGGL((k_quantize<false, false>), grid, block, 0, s, d);
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
