// ONNX ConvInteger (ConvIntegerKernels.Encode, ConvIntegerKernels.cs:97-253): the two kernels of its own besides the
// int8 product.
//
// Pack (ConvIntegerPack.hlsl): the windows of every image and group unfold into a byte matrix of K = CinG * KH * KW
// rows and OH * OW columns (Chellapilla, Puri and Simard, 2006), row (c * KH + kh) * KW + kw, column oh * OW + ow
// holding x[n, g * CinG + c, oh * SH - PH + kh * DH, ow * SW - PW + kw * DW], or x's zero point where that position lies
// in the padding (so a padded tap adds nothing once the product subtracts the zero point). Rows are padded to a multiple
// of 16 bytes (ldb) so that the MFMA product can feed them to LDS with 16-byte DMA; the padding columns hold the zero
// point too and the product never reads them. One thread writes 16 bytes of one row.
//
// Padded depth: when K is at least 64 and not a multiple of 64, the launcher pads it to one (kp) so that the products
// take the LDS-DMA kernel. Rows k .. kp - 1 of every column matrix hold x's zero point, so each padded tap adds
// (w - wz) (xz - xz) = 0, and the same launch copies the weights into rows of kp bytes, zero past k; the 16-byte
// chunks of both go through one grid-stride loop (the column chunks first).
//
// Depthwise (one input channel a group): no matrix at all. One thread per output element sums its KH * KW taps,
// (x - xz) * (w - wz[m]) in 32-bit wrap-around, skipping taps in the padding (they are the real value zero).
#include "og_internal.hpp"

#include <algorithm>

namespace og {

namespace {

constexpr int kConvThreads = 256;

__device__ __forceinline__ int32_t byte_val(uint8_t b, bool is_signed) { return is_signed ? (int32_t)(int8_t)b : (int32_t)b; }

template <bool ALIGNED16>
__global__ __launch_bounds__(kConvThreads) void k_conv_pack(ConvPackArgs a)
{
    const int64_t chunks_per_row = a.ldb / 16;
    const int64_t rows = (int64_t)a.images * a.groups * a.kp;
    const int64_t total = rows * chunks_per_row, wchunks = a.kp / 16, wtotal = (int64_t)a.wrows * wchunks;
    const int32_t taps = a.kh * a.kw;
    const uint32_t pad = a.xz ? (uint32_t)*a.xz : 0u;
    const int32_t ncols = a.oh * a.ow;
    for (int64_t t = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; t < total + wtotal;
         t += (int64_t)gridDim.x * kConvThreads) {
        if (t >= total) {
            // Weight chunk: row m, bytes 16 c .. + 15 of the padded copy.
            const int64_t tw = t - total, m = tw / wchunks;
            const int32_t c0 = 16 * (int32_t)(tw - m * wchunks);
            uint32_t word[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint32_t wv = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int32_t kk = c0 + 4 * q + e;
                    wv |= (kk < a.k ? (uint32_t)a.wt[m * a.k + kk] : 0u) << (8 * e);
                }
                word[q] = wv;
            }
            *reinterpret_cast<uint4 *>(a.wp + m * a.kp + c0) = make_uint4(word[0], word[1], word[2], word[3]);
            continue;
        }
        const int64_t r = t / chunks_per_row;
        const int32_t c16 = (int32_t)(t - r * chunks_per_row);
        const int64_t ig = r / a.kp;
        const int32_t k = (int32_t)(r - ig * a.kp);
        uint8_t *dst = a.cols + r * a.ldb + 16 * (int64_t)c16;
        if (k >= a.k) {   // a padding row
            const uint32_t pw4 = pad * 0x01010101u;
            if constexpr (ALIGNED16) {
                *reinterpret_cast<uint4 *>(dst) = make_uint4(pw4, pw4, pw4, pw4);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) reinterpret_cast<uint32_t *>(dst)[q] = pw4;
            }
            continue;
        }
        const int64_t img = ig / a.groups;
        const int32_t g = (int32_t)(ig - img * a.groups);
        const int32_t c = k / taps, kk = k - c * taps, kh = kk / a.kw, kw = kk - kh * a.kw;
        const uint8_t *plane = a.x + (img * a.cin + (int64_t)g * a.cin_g + c) * (int64_t)a.h * a.w;
        // Column n = 16 * c16 + e; its (oh, ow) advance one column at a time.
        int32_t n = 16 * c16, row_o = n / a.ow, col_o = n - row_o * a.ow;
        uint32_t word[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t wv = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t v = pad;
                if (n < ncols) {
                    const int64_t ih = (int64_t)row_o * a.sh + (int64_t)kh * a.dh - a.ph;
                    const int64_t iw = (int64_t)col_o * a.sw + (int64_t)kw * a.dw - a.pw;
                    if (ih >= 0 && ih < a.h && iw >= 0 && iw < a.w) v = plane[ih * a.w + iw];
                }
                wv |= v << (8 * e);
                n++;
                if (++col_o == a.ow) {
                    col_o = 0;
                    row_o++;
                }
            }
            word[q] = wv;
        }
        if constexpr (ALIGNED16) {
            *reinterpret_cast<uint4 *>(dst) = make_uint4(word[0], word[1], word[2], word[3]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) reinterpret_cast<uint32_t *>(dst)[q] = word[q];
        }
    }
}

// K3: the window is 3 x 3 (known at compile time), so the nine taps' loads are all issued before the first is used
// (a tap in the padding loads the plane's first byte and adds nothing); otherwise a loop over the window.
template <bool XS, bool WS, bool K3>
__global__ __launch_bounds__(kConvThreads) void k_conv_depthwise(ConvDepthwiseArgs a)
{
    const int64_t plane = (int64_t)a.oh * a.ow;
    const int64_t total = (int64_t)a.batch * a.cout * plane;
    const int32_t cout_g = a.cout / a.cin;   // output channels of one input channel
    const int32_t xz = a.xz ? byte_val(*a.xz, XS) : 0;
    for (int64_t t = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kConvThreads) {
        const int64_t nm = t / plane;
        const int32_t p = (int32_t)(t - nm * plane);
        const int64_t n = nm / a.cout;
        const int32_t m = (int32_t)(nm - n * a.cout);
        const int32_t i = p / a.ow, j = p - (p / a.ow) * a.ow;
        const uint8_t *xp = a.x + (n * a.cin + m / cout_g) * (int64_t)a.h * a.w;
        const uint8_t *wp = a.wt + (int64_t)m * a.kh * a.kw;
        const int32_t wz = a.wz ? byte_val(a.wz[a.wz_per_channel ? m : 0], WS) : 0;
        uint32_t acc = 0;
        if constexpr (K3) {
            int64_t off[9];
            bool in[9];
#pragma unroll
            for (int q = 0; q < 9; q++) {
                const int64_t ih = (int64_t)i * a.sh + (int64_t)(q / 3) * a.dh - a.ph;
                const int64_t iw = (int64_t)j * a.sw + (int64_t)(q % 3) * a.dw - a.pw;
                in[q] = ih >= 0 && ih < a.h && iw >= 0 && iw < a.w;
                off[q] = in[q] ? ih * a.w + iw : 0;
            }
            uint8_t xv[9], wv[9];
#pragma unroll
            for (int q = 0; q < 9; q++) {
                xv[q] = xp[off[q]];
                wv[q] = wp[q];
            }
#pragma unroll
            for (int q = 0; q < 9; q++)
                if (in[q]) acc += (uint32_t)(byte_val(xv[q], XS) - xz) * (uint32_t)(byte_val(wv[q], WS) - wz);
            a.y[t] = (int32_t)acc;
            continue;
        }
        for (int32_t kh = 0; kh < a.kh; kh++) {
            const int64_t ih = (int64_t)i * a.sh + (int64_t)kh * a.dh - a.ph;
            if (ih < 0 || ih >= a.h) continue;
            for (int32_t kw = 0; kw < a.kw; kw++) {
                const int64_t iw = (int64_t)j * a.sw + (int64_t)kw * a.dw - a.pw;
                if (iw < 0 || iw >= a.w) continue;
                const int32_t xv = byte_val(xp[ih * a.w + iw], XS) - xz;
                const int32_t wv = byte_val(wp[kh * a.kw + kw], WS) - wz;
                acc += (uint32_t)xv * (uint32_t)wv;
            }
        }
        a.y[t] = (int32_t)acc;
    }
}

int64_t conv_grid(int64_t threads)
{
    return std::max<int64_t>(1, std::min<int64_t>((threads + kConvThreads - 1) / kConvThreads, int64_t(1) << 20));
}

}  // namespace

hipError_t launch_conv_pack(const ConvPackArgs &a, hipStream_t s, const char **kernel)
{
    *kernel = "conv-pack16";
    const int64_t total = (int64_t)a.images * a.groups * a.kp * (a.ldb / 16) + (int64_t)a.wrows * (a.kp / 16);
    if (total == 0) return hipSuccess;
    const dim3 grid((uint32_t)conv_grid(total)), block(kConvThreads);
    if (((uintptr_t)a.cols & 15) == 0) hipLaunchKernelGGL(k_conv_pack<true>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(k_conv_pack<false>, grid, block, 0, s, a);
    return hipGetLastError();
}

hipError_t launch_conv_depthwise(const ConvDepthwiseArgs &a, hipStream_t s, const char **kernel)
{
    *kernel = "conv-depthwise-i8";
    const int64_t total = (int64_t)a.batch * a.cout * a.oh * a.ow;
    if (total == 0) return hipSuccess;
    const dim3 grid((uint32_t)conv_grid(total)), block(kConvThreads);
#define OG_DW(XS, WS)                                                                                     \
    do {                                                                                                 \
        if (a.kh == 3 && a.kw == 3) hipLaunchKernelGGL((k_conv_depthwise<XS, WS, true>), grid, block, 0, s, a);  \
        else hipLaunchKernelGGL((k_conv_depthwise<XS, WS, false>), grid, block, 0, s, a);                       \
    } while (0)
    if (a.x_signed) {
        if (a.w_signed) OG_DW(true, true);
        else OG_DW(true, false);
    } else {
        if (a.w_signed) OG_DW(false, true);
        else OG_DW(false, false);
    }
#undef OG_DW
    return hipGetLastError();
}

}  // namespace og
