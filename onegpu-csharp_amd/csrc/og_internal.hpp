// Internal declarations shared by the HIP translation units of libonegpu_hip.so: the resolved argument blocks the
// kernels take, their launchers, and the device helpers common to them. Everything here is gfx950 (CDNA4) code.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "onegpu_hip.h"

namespace og {

// One int8 product after validation: base pointers with the caller's offsets already applied, strides in bytes (A, B)
// and elements (C), zero points as pointers to their first element (nullptr when absent).
struct GemmArgs {
    const uint8_t *A;
    const uint8_t *B;
    void *C;
    const uint8_t *ZA;
    const uint8_t *ZB;
    const int32_t *bias;
    const float *scale;
    const float *fbias;
    const float *act_scale;   // EPI_SCALE_PRODUCT: the column scale is fl(*act_scale * scale[n or 0])
    int64_t strideA, strideB, strideC;
    // Bytes readable from B (all batches). The aligned K x N kernels load B's rows a dword at a time, so with N not a
    // multiple of 4 they read up to round4(N) in the last row: they run only when that stays inside this extent.
    int64_t b_bytes;
    int32_t M, N, K, batch;
    int32_t lda, ldb;
    uint32_t flags;  // OG_GEMM_*
    uint32_t epi;    // OG_EPI_*, plus EPI_REQUANT / EPI_REQUANT_U8 below
    int32_t zp_y;    // the output zero point of a requantized product
    // A float product's range output (og_int8_gemm_float_ranged), or nullptr: each workgroup that stores C writes the
    // NaN-ignoring minimum and maximum of the values it stored to ranges[2 slot], ranges[2 slot + 1], its slot a number
    // below the kernel's range_groups (product_range_groups).
    float *ranges;
};

// Pairs a ranged product may write: its caller's buffer holds 2 * kRangesMax floats (OG_RANGES_MAX).
constexpr int kRangesMax = 1024;

// Library-internal epilogue bits (above the public OG_EPI_* ones): C is 8-bit and each sum is requantized with the
// multiplier at `scale` and the zero point zp_y; uint8 output when EPI_REQUANT_U8, else int8.
constexpr uint32_t EPI_REQUANT = 0x100u, EPI_REQUANT_U8 = 0x200u;
// Library-internal: the float result's column scale is the product fl(*act_scale * scale[n or 0]).
constexpr uint32_t EPI_SCALE_PRODUCT = 0x400u;

// Device workspace owned by a context: the partial sums of the few-rows kernels and the dynamic quantizer's
// per-workgroup ranges. Sized once at og_init; the partial sums grow (outside any launch) when a larger few-rows product
// arrives.
struct Workspace {
    int32_t *partials;       // split-k partial sums (int32)
    uint64_t partial_bytes;
    float *dq_ranges;        // 2 * kDqMaxGroups floats: the dynamic quantizer's per-workgroup ranges
};

constexpr int kDqMaxGroups = 256;

// og_int8_gemm_noalloc's fixed scratch (one array a device): the few-rows kernel's count words, then partial sums.
constexpr uint64_t kNoAllocScratchBytes = 16ull << 20, kNoAllocWordBytes = 64ull << 10;
// Looks up the array's device address on `device` (current) once, clearing its count words; later calls return it.
hipError_t noalloc_scratch_setup(int device, hipStream_t s, void **out);


// Kernel choice for a product, as og_int8_gemm_kernel_name reports it.
enum class GemmKernel { Portable, Tiled, Skinny, SkinnyDirect, RowTiles, RowXcd };

// The (min, max) pairs a float product writes from its epilogue when GemmArgs::ranges is set: the direct kernels one a
// workgroup, the split-k summing pass one a workgroup, the one-launch few-rows kernel one a column slab; 0 for the
// kernels without a range epilogue (the caller then runs a range pass over C).
uint32_t direct_range_groups(const GemmArgs &g, bool large);
uint32_t direct_split_range_groups(const GemmArgs &g);
uint32_t gemv_xcd_range_groups(const GemmArgs &g);
GemmKernel choose_gemm_kernel(int32_t M, int32_t N, int32_t K, int32_t batch, uint32_t flags);
const char *gemm_kernel_name(GemmKernel k);

// Launchers (one per kernel family); each returns the launch status. `kernel` receives the name of the kernel run.
hipError_t launch_gemm_portable(const GemmArgs &g, hipStream_t s, const char **kernel);
// The MFMA tiled product: the aligned kernel when tiled_fast_ok(g), else the generic one.
hipError_t launch_gemm_tiled(const GemmArgs &g, hipStream_t s, const char **kernel);
hipError_t launch_gemm_generic(const GemmArgs &g, hipStream_t s, const char **kernel);
// The kernel fed by LDS DMA (16-byte aligned operands, K a multiple of 64), 256 x 256 tiles for large products, else
// 128 x 128; launch_gemm_tiled picks it when it applies.
hipError_t launch_gemm_direct(const GemmArgs &g, hipStream_t s, const char **kernel, bool large);
bool direct_ok(const GemmArgs &g);
// Split-k of the 128 x 128 direct kernel for grids that fill under half the chip: direct_split gives the number of k
// slices (1: no split); the slices' int32 sums go to ws.partials (step 0), a second pass adds them and applies the
// bias and the epilogue (step 1).
constexpr int64_t kSplitTargetTiles = 256, kSplitMaxBytes = int64_t(256) << 20;
int direct_split(const GemmArgs &g);
uint64_t direct_split_workspace_bytes(const GemmArgs &g, int ks);
hipError_t launch_gemm_direct_split(const GemmArgs &g, const Workspace &ws, hipStream_t s, const char **kernel, int ks,
                                    int step);
// Whether B's last row can be read in whole dwords up to round4(N) (K x N layout; always true for N % 4 == 0).
inline bool b_dwords_ok(const GemmArgs &g)
{
    if ((g.flags & OG_GEMM_TRANSPOSE_B) || g.N % 4 == 0 || g.K == 0) return true;
    return (int64_t)(g.batch - 1) * g.strideB + (int64_t)(g.K - 1) * g.ldb + ((g.N + 3) & ~3) <= g.b_bytes;
}
bool tiled_fast_ok(const GemmArgs &g);
bool tiled_uses_large(int32_t M, int32_t N, int32_t batch);
// Few rows (M <= 16), B stored K x N: split-k partial sums into ws.partials, then a pass that adds them up, corrects for
// the zero points and applies the epilogue. `slices` is the split chosen by skinny_slices().
hipError_t launch_gemm_skinny(const GemmArgs &g, const Workspace &ws, hipStream_t s, const char **kernel, int step);
int skinny_slices(int32_t M, int32_t N, int32_t K, int32_t batch);
uint64_t skinny_workspace_bytes(int32_t M, int32_t N, int32_t K, int32_t batch);
// Few rows (M <= 16), B stored K x N, one workgroup per 256 x 256 tile of B writing its part into ws.partials (step 0),
// then a pass that adds the parts, corrects for the zero points and applies the epilogue (step 1).
bool gemv_tiles_ok(const GemmArgs &g);
uint64_t gemv_tiles_workspace_bytes(const GemmArgs &g);
hipError_t launch_gemv_tiles(const GemmArgs &g, const Workspace &ws, hipStream_t s, const char **kernel, int step);
// The same tiles in one launch: every tile but the last row band of a column slab stores its part into `parts` and
// counts it in the slab's word of `words`; the last row band's tile waits for the count, adds the parts and stores C.
// The tiles of a slab run on one XCD (ids equal modulo 8), so the parts pass through that XCD's L2 alone. `words`
// (gemv_xcd_words 64-bit words: a poison word, then one a slab) must be zero before the launch and the slab words are
// zero again after it; `flag` is set to 1 if a slab's tiles did not share an XCD, 2 if a slab's parts were never all
// counted within `spin_limit` polls (its columns of C not written), 3 if an earlier launch on these words failed (the
// poison word was set: nothing was read); after 1 or 2 the poison word is set and every word must be cleared.
constexpr uint32_t kGemvSpinLimit = 1u << 22;
bool gemv_xcd_ok(const GemmArgs &g);
uint64_t gemv_xcd_workspace_bytes(const GemmArgs &g);
uint64_t gemv_xcd_words(const GemmArgs &g);
hipError_t launch_gemv_xcd(const GemmArgs &g, int32_t *parts, unsigned long long *words, uint32_t *flag,
                           uint32_t spin_limit, hipStream_t s, const char **kernel);
// out[x] = the XCD (HW_REG_XCC_ID) workgroup x of a `groups`-workgroup launch ran on.
hipError_t launch_xcc_probe(uint32_t *out, uint32_t groups, hipStream_t s);

struct EpilogueArgs {
    const int32_t *acc;
    void *out;
    const int32_t *bias;
    const float *scale;
    const float *fbias;
    uint32_t count, n, mode, flags;
    int32_t zero_point;
    uint32_t out_byte_offset;  // mode 2: byte offset of out within its allocation, for vector stores
};
hipError_t launch_int8_epilogue(const EpilogueArgs &e, hipStream_t s, const char **kernel);

struct DqArgs {
    const float *x;
    uint8_t *y;
    float *scale;
    uint8_t *zero;
    uint32_t count;
};
hipError_t launch_dynamic_quantize(const DqArgs &d, const Workspace &ws, hipStream_t s, const char **kernel, int step);
// DynamicQuantizeLinear's quantize pass alone, over `groups` (min, max) pairs at `ranges` (at most kRangesMax; the
// buffer holds 2 * kRangesMax floats) that cover x: a ranged product's, or launch_range_pass's.
hipError_t launch_dynamic_quantize_ranged(const DqArgs &d, const float *ranges, uint32_t groups, hipStream_t s,
                                          const char **kernel);
// DynamicQuantizeLinear's range pass alone over count floats at x, into `ranges`; *groups = the pairs written.
hipError_t launch_range_pass(const float *x, uint32_t count, float *ranges, hipStream_t s, const char **kernel,
                             uint32_t *groups);

struct DequantArgs {
    const void *x;
    const float *scale;
    const void *zero;
    void *out;
    uint32_t count, axis_len, inner;
    bool per_axis, has_zero;
};
hipError_t launch_dequantize(const DequantArgs &d, int kind, bool f16_out, hipStream_t s, const char **kernel);
// n passes of one count, axis and zero-point form (their buffers independent) in ceil(n / kDqBatch) launches.
constexpr int kDqBatch = 64;   // 64 argument blocks of 48 bytes: within the 4 KB of kernel arguments
hipError_t launch_dequantize_batch(const DequantArgs *d, int n, int kind, bool f16_out, hipStream_t s,
                                   const char **kernel);
hipError_t launch_quantize(const DequantArgs &d, bool is_signed, bool f16_in, hipStream_t s, const char **kernel);

// ONNX Gather along one axis as a copy of byte rows: output row (o, i) of row_bytes bytes is data row
// (o, index[i]); rows = outer * count. An invalid index gives a zero row and its position in *status (atomic minimum).
struct GatherArgs {
    const uint8_t *data;
    const void *idx;
    uint8_t *out;
    uint32_t *status;   // nullptr: invalid indices only give zeros
    int64_t rows, count;
    uint32_t axis_len;
    int64_t row_bytes;
    bool wide;          // int64 indices
};
hipError_t launch_gather(const GatherArgs &a, hipStream_t s, const char **kernel);

// ConvInteger's column matrix for `images` images from x (image 0 of the chunk): per image and group K rows of ldb
// bytes (ldb a multiple of 16, at least oh * ow), image-major then group; padding and padding columns hold *xz (0 when
// absent).
struct ConvPackArgs {
    const uint8_t *x;
    const uint8_t *xz;
    uint8_t *cols;
    int32_t images, groups, k, cin, cin_g, h, w, oh, ow, kh, kw, sh, sw, dh, dw, ph, pw;
    int64_t ldb;
    // K padded to kp (>= k) rows: rows k .. kp - 1 of every column matrix hold x's zero point, and the weights
    // [wrows x k] are copied to wp as [wrows x kp] with zeros past k (wrows = 0: no copy; wp 16-byte aligned).
    int32_t kp, wrows;
    const uint8_t *wt;
    uint8_t *wp;
};
hipError_t launch_conv_pack(const ConvPackArgs &a, hipStream_t s, const char **kernel);

// ConvInteger with one input channel a group: y[n, m, i, j] from input channel m / (cout / cin) directly.
struct ConvDepthwiseArgs {
    const uint8_t *x, *wt, *xz, *wz;
    int32_t *y;
    int32_t batch, cin, cout, h, w, oh, ow, kh, kw, sh, sw, dh, dw, ph, pw;
    bool x_signed, w_signed, wz_per_channel;
};
hipError_t launch_conv_depthwise(const ConvDepthwiseArgs &a, hipStream_t s, const char **kernel);

hipError_t launch_fill_bytes(void *dst, uint8_t value, uint64_t bytes, hipStream_t s);
hipError_t launch_synth(int kind, uint64_t seed, uint32_t tensor, void *out, uint64_t count, double lo, double hi,
                        hipStream_t s);
hipError_t launch_col_absmax_scale(const float *w, uint32_t rows, uint32_t cols, float divisor, float *scale,
                                   hipStream_t s);
hipError_t launch_scale_product(const float *a, const float *b, uint32_t n, float *out, hipStream_t s);
// Reads B [K x N] (dense rows, N a multiple of 16) once in the few-rows one-launch kernel's tiles and loads, and does
// nothing else (int8_gemv_xcd.hip): that kernel's streaming floor.
hipError_t launch_stream_tiles(const uint8_t *B, int32_t K, int32_t N, uint32_t *sink, hipStream_t s);

// ------------------------------------------------------------------ device helpers

#if defined(__HIPCC__)
// Four signed bytes times four signed bytes, summed, plus c (v_dot4_i32_i8); no clamping, so the sum wraps.
__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c)
{
    return __builtin_amdgcn_sdot4((int32_t)a, (int32_t)b, c, false);
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value {hi, lo} (selectors 0-3 pick lo, 4-7 hi).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4 x 4 byte transpose: r[i] holds row i (byte j = column j); afterwards c[j] holds column j (byte i = row i).
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t &c0,
                                             uint32_t &c1, uint32_t &c2, uint32_t &c3)
{
    uint32_t lo01 = perm(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
    uint32_t hi01 = perm(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
    uint32_t lo23 = perm(r3, r2, 0x05010400u);
    uint32_t hi23 = perm(r3, r2, 0x07030602u);
    c0 = perm(lo23, lo01, 0x05040100u);
    c1 = perm(lo23, lo01, 0x07060302u);
    c2 = perm(hi23, hi01, 0x05040100u);
    c3 = perm(hi23, hi01, 0x07060302u);
}

__device__ __forceinline__ int32_t sext8(uint32_t b) { return (int32_t)(int8_t)(uint8_t)b; }

// A workgroup of THREADS threads combines its threads' (mn, mx) (fminf / fmaxf: a NaN never wins, and the kernels' float
// results are never signalling NaNs) and thread 0 stores them to ranges[2 slot], [2 slot + 1]. `lds` holds 2 * THREADS
// / 64 floats nobody else uses until the call returns; every thread of the workgroup calls it.
template <int THREADS>
__device__ __forceinline__ void store_workgroup_range(float mn, float mx, float *lds, float *ranges, uint32_t slot)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, o));
        mx = fmaxf(mx, __shfl_xor(mx, o));
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        lds[2 * wave] = mn;
        lds[2 * wave + 1] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < THREADS / 64; w++) {
            mn = fminf(mn, lds[2 * w]);
            mx = fmaxf(mx, lds[2 * w + 1]);
        }
        ranges[2 * slot] = mn;
        ranges[2 * slot + 1] = mx;
    }
}

// The column scale of a float result: scale[n or 0], or its product with the activation scale.
__device__ __forceinline__ float column_scale(const GemmArgs &g, int32_t col)
{
    const float s = g.scale[(g.epi & OG_EPI_SCALE_PER_COL) ? col : 0];
    return (g.epi & EPI_SCALE_PRODUCT) ? __fmul_rn(*g.act_scale, s) : s;
}

// QLinearMatMul's requantization of one sum (bias already added; Int8Epilogue.hlsl:54-68): v = fl(float(sum) * mult);
// NaN to the lowest value; else round half to even, clamp to [lo - zp, hi - zp], add zp. Returns the byte.
__device__ __forceinline__ uint32_t requantize_byte(uint32_t sum, float mult, int32_t zp, bool u8)
{
    const int32_t lo = u8 ? 0 : -128, hi = u8 ? 255 : 127;
    const float v = __fmul_rn((float)(int32_t)sum, mult);
    if ((__float_as_uint(v) & 0x7FFFFFFFu) > 0x7F800000u) return (uint32_t)lo & 0xFFu;   // NaN
    const float r = fminf(fmaxf(rintf(v), (float)(lo - zp)), (float)(hi - zp));
    return (uint32_t)((int32_t)r + zp) & 0xFFu;
}

// The float result of a sum (Int8GemmEpilogue.hlsli:17-42): fl(fl(float(sum + bias)) * scale), then + float bias as a
// separate rounding.
__device__ __forceinline__ float sum_to_float(const GemmArgs &g, int32_t col, uint32_t sum)
{
    if (g.epi & OG_EPI_INT_BIAS) sum += (uint32_t)g.bias[col];
    float f = __fmul_rn((float)(int32_t)sum, column_scale(g, col));
    if (g.epi & OG_EPI_FLOAT_BIAS) f = __fadd_rn(f, g.fbias[col]);
    return f;
}

// The int32 sum as the reference's StoreValue leaves it (Int8GemmEpilogue.hlsli:17-42): the raw sum; + int bias;
// or fl(fl(float(sum + bias)) * scale), then + float bias as a separate rounding.
__device__ __forceinline__ void store_sum(const GemmArgs &g, int64_t ci, int32_t col, uint32_t sum)
{
    uint32_t epi = g.epi;
    if (epi & OG_EPI_INT_BIAS) sum += (uint32_t)g.bias[col];
    if (!(epi & OG_EPI_FLOAT)) {
        static_cast<int32_t *>(g.C)[ci] = (int32_t)sum;
        return;
    }
    const float s = column_scale(g, col);
    float f = __fmul_rn((float)(int32_t)sum, s);
    if (epi & OG_EPI_FLOAT_BIAS) f = __fadd_rn(f, g.fbias[col]);
    static_cast<float *>(g.C)[ci] = f;
}

// A requantized product's byte (+ int bias, then requantize_byte with the multiplier and zp_y).
__device__ __forceinline__ void store_requantized(const GemmArgs &g, int64_t ci, int32_t col, uint32_t sum)
{
    const uint32_t epi = g.epi;
    if (epi & OG_EPI_INT_BIAS) sum += (uint32_t)g.bias[col];
    const float mult = g.scale[(epi & OG_EPI_SCALE_PER_COL) ? col : 0];
    static_cast<uint8_t *>(g.C)[ci] = (uint8_t)requantize_byte(sum, mult, g.zp_y, (epi & EPI_REQUANT_U8) != 0);
}

// store_sum and store_requantized with the column's int bias already added to `sum` and its scale (multiplier) and
// float bias fetched, for kernels that store many values of one column.
__device__ __forceinline__ void store_sum_col(const GemmArgs &g, int64_t ci, uint32_t sum, float sc, float fb)
{
    if (!(g.epi & OG_EPI_FLOAT)) {
        static_cast<int32_t *>(g.C)[ci] = (int32_t)sum;
        return;
    }
    float f = __fmul_rn((float)(int32_t)sum, sc);
    if (g.epi & OG_EPI_FLOAT_BIAS) f = __fadd_rn(f, fb);
    static_cast<float *>(g.C)[ci] = f;
}

__device__ __forceinline__ void store_requantized_col(const GemmArgs &g, int64_t ci, uint32_t sum, float mult, float)
{
    static_cast<uint8_t *>(g.C)[ci] = (uint8_t)requantize_byte(sum, mult, g.zp_y, (g.epi & EPI_REQUANT_U8) != 0);
}

// Either of the two, as the product's epilogue bits say (for kernels that store few values a thread).
__device__ __forceinline__ void store_value(const GemmArgs &g, int64_t ci, int32_t col, uint32_t sum)
{
    if (g.epi & EPI_REQUANT) store_requantized(g, ci, col, sum);
    else store_sum(g, ci, col, sum);
}

// Zero point in the signed domain: an unsigned operand's bytes move by -128 (s = u ^ 0x80), and so does its zero point.
__device__ __forceinline__ int32_t signed_zero(const uint8_t *z, int32_t idx, bool per, bool is_signed)
{
    int32_t v = z ? (is_signed ? sext8(z[per ? idx : 0]) : (int32_t)z[per ? idx : 0]) : 0;
    return is_signed ? v : v - 128;
}
#endif

}  // namespace og
