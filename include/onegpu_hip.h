/*
 * onegpu_hip.h — the C ABI of the MI355X (gfx950) int8 quantized-matmul library.
 *
 * This is the drop-in boundary for one path of recursive-ai-oss/onegpu-csharp: the Int8Gemm family (ONNX MatMulInteger,
 * MatMulIntegerToFloat, QLinearMatMul), DynamicQuantizeLinear, and DequantizeLinear/QuantizeLinear. The reference
 * records these as compute dispatches through WideKernelPipeline.Record / KernelPipeline.Record
 * (src/RecursiveAI.OneGpu.Kernels/WideKernelPipeline.cs:73-115, KernelSupport.cs:236-287): a push-constant block plus
 * storage-buffer bindings. Each entry point below replaces one such family of dispatches; its parameter block keeps the
 * reference's push-constant words, word for word, and each binding becomes an og_buffer (device address + byte size).
 *
 * Conventions
 *  - Plain C: no C++ or framework types cross the boundary. Every pointer in an og_buffer is a device address the caller
 *    allocated (og_alloc or hipMalloc); the caller owns it. A NULL ptr means "operand absent" (the reference binds a dummy).
 *  - Offsets are counted as in the reference: bytes for uint8/int8 operands, elements for int32/float32/float16 ones.
 *  - Every compute call is asynchronous on the context's stream, in call order ("nothing runs until Submit" is the host
 *    layer's business). Nothing is allocated on a warm call.
 *  - Every call validates its arguments before launching anything and returns an og_status. On OG_ERR_INVALID_ARG,
 *    og_last_error_argument() names the argument at fault (the host maps it to GpuKernelShapeException(operation, argument,
 *    message)); OG_ERR_UNSUPPORTED maps to GpuUnsupportedException, OG_ERR_OUT_OF_MEMORY to GpuOutOfMemoryException,
 *    OG_ERR_DEVICE_LOST to GpuDeviceLostException, OG_ERR_LAUNCH_FAILED to GpuCommandFailedException.
 *  - Like the reference families, a context is not thread-safe (src/RecursiveAI.OneGpu.Kernels/Int8Gemm.cs:122).
 *  - Workspace: a context owns its partial-sum workspace and the few-rows kernel's arrival words. A product that needs
 *    more than the context holds grows them first; growth is refused with OG_ERR_INVALID_ARG (argument "workspace")
 *    while the context's stream is being captured into a HIP graph, so capture a product only after one of at least
 *    its size has run on the context. Replaced workspaces stay allocated until og_destroy, so a graph captured earlier
 *    never replays into freed memory.
 */
#ifndef ONEGPU_HIP_H
#define ONEGPU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OG_ABI_VERSION 1

typedef struct og_ctx og_ctx;

typedef enum og_status {
    OG_OK = 0,
    OG_ERR_INVALID_ARG = 1,
    OG_ERR_UNSUPPORTED = 2,
    OG_ERR_OUT_OF_MEMORY = 3,
    OG_ERR_DEVICE_LOST = 4,
    OG_ERR_LAUNCH_FAILED = 5,
    OG_ERR_NO_DEVICE = 6
} og_status;

/* One storage-buffer binding: the buffer's device address and its size in bytes. */
typedef struct og_buffer {
    void *ptr;
    uint64_t bytes;
} og_buffer;

/* ------------------------------------------------------------------ device, memory, ordering */

/* Opens device `device_ordinal` with one stream of its own. Replaces the HIP half of a GpuDevice
 * (src/RecursiveAI.OneGpu/GpuDevice.cs:27-254): the queue the families record onto. */
int og_init(int device_ordinal, og_ctx **out);
int og_destroy(og_ctx *ctx);
int og_device_count(int *count);
/* Adapter name (GpuDevice.Adapter.Name) and limits (GpuComputeCapabilities, ComputeCapabilities.cs:86-203). */
int og_device_name(og_ctx *ctx, char *buf, size_t len);
int og_device_limits(og_ctx *ctx, uint64_t *max_buffer_bytes, uint32_t *compute_units, uint32_t *lds_bytes_per_group);
/* The hipStream_t the context records on, for callers that interleave their own work. */
int og_stream(og_ctx *ctx, void **hip_stream);
/* Waits for everything recorded so far (GpuDevice.WaitIdle); reports a failed launch as OG_ERR_LAUNCH_FAILED, and so
 * a one-launch few-rows product whose column slab did not run on one XCD (its output may then be wrong), that gave up
 * waiting for a slab's parts (those columns unwritten), or that found the count words left by such a failure and did
 * not run. It then clears the count words (the context's and the device's fixed ones) and the context uses the
 * two-launch form from then on. */
int og_sync(og_ctx *ctx);
/* Buffers (GpuDevice.CreateBuffer / GpuBuffer<T>.Dispose, GpuBufferOfT.cs:11-89). */
int og_alloc(og_ctx *ctx, uint64_t bytes, void **dptr);
int og_free(og_ctx *ctx, void *dptr);
/* Copies in stream order (GpuBuffer.Write / ReadAsync, GpuBufferOfT.cs:71-75). The d2h copy completes before it returns. */
int og_memcpy_h2d(og_ctx *ctx, void *dst, const void *src, uint64_t bytes);
int og_memcpy_d2h(og_ctx *ctx, void *dst, const void *src, uint64_t bytes);
int og_memcpy_d2d(og_ctx *ctx, void *dst, const void *src, uint64_t bytes);
/* Byte fill by a kernel (not hipMemsetAsync), so a fill can sit inside a captured HIP graph. */
int og_fill_bytes(og_ctx *ctx, void *dst, uint8_t value, uint64_t bytes);

/* Per-dispatch timing, the HIP counterpart of GpuCommandEncoder.BeginPassTiming / EndPassTiming and
 * GpuDevice.TryReadTimestamps (Resources.cs:216-222, GpuDevice.cs:109): while timing is on, every kernel the context
 * launches is bracketed by a pair of events on its stream. og_timing_read waits for them and returns milliseconds. */
int og_timing_begin(og_ctx *ctx, int max_dispatches);
int og_timing_end(og_ctx *ctx, int *dispatches);
int og_timing_read(og_ctx *ctx, int index, float *ms, const char **kernel_name);
/* One event pair around everything recorded between the two calls (GpuCommandEncoder.BeginPassTiming /
 * EndPassTiming around a whole run of passes, Resources.cs:216-222): back-to-back launches stay back to back.
 * og_timing_region_end waits for the stop event and returns the elapsed milliseconds. */
int og_timing_region_begin(og_ctx *ctx);
int og_timing_region_end(og_ctx *ctx, float *ms);

/* ------------------------------------------------------------------ Int8Gemm */

/* Int8GemmParams, the 19 push-constant words of the reference product kernels
 * (src/RecursiveAI.OneGpu.Kernels/Shaders/Int8GemmDot.hlsl:17-40; filled by Int8Gemm.Multiply, Int8Gemm.cs:616-635). */
typedef struct og_int8_gemm_params {
    uint32_t M, N, K;
    uint32_t OffA;      /* byte offset of A */
    uint32_t OffB;      /* byte offset of B */
    uint32_t OffC;      /* element offset of C */
    uint32_t StrideA;   /* bytes between the A of consecutive batches; 0 shares A */
    uint32_t StrideB;   /* bytes between the B of consecutive batches; 0 shares B */
    uint32_t StrideC;   /* elements between the C of consecutive batches (the reference passes M * N) */
    uint32_t Lda;       /* row stride of A in bytes, >= K */
    uint32_t Ldb;       /* row stride of the stored B in bytes, >= N (or >= K with TransposeB) */
    uint32_t Flags;     /* OG_GEMM_* below */
    uint32_t OffZA;     /* byte offset of the zero point of A */
    uint32_t OffZB;     /* byte offset of the zero point of B */
    uint32_t Epi;       /* OG_EPI_* below */
    uint32_t OffBias;   /* element offset of the int32 bias */
    uint32_t OffScale;  /* element offset of the float32 scale */
    uint32_t OffFBias;  /* element offset of the float32 bias */
    uint32_t GridX;     /* the reference's folded-grid width; ignored here (the library sizes its own grids) */
} og_int8_gemm_params;

/* Flags bits 0-9 keep the reference's meaning (Int8GemmDot.hlsl:30-32). Bits 7-9 describe how the reference folded its
 * grid and aligned its word loads; this library derives both from the actual addresses, so they are ignored. */
#define OG_GEMM_A_INT8        0x001u  /* A is int8 (else uint8) */
#define OG_GEMM_B_INT8        0x002u  /* B is int8 (else uint8) */
#define OG_GEMM_TRANSPOSE_B   0x004u  /* B stored N x K */
#define OG_GEMM_ZA            0x008u  /* zero point of A present */
#define OG_GEMM_ZA_PER_ROW    0x010u  /* ... one per row of A */
#define OG_GEMM_ZB            0x020u  /* zero point of B present */
#define OG_GEMM_ZB_PER_COL    0x040u  /* ... one per column of B */
/* Library bits, no counterpart in the reference: kernel choice, for Int8GemmOptions and tests. */
#define OG_GEMM_PORTABLE      0x400u  /* run the portable integer kernel (Int8GemmOptions.AllowPackedDot = false) */
#define OG_GEMM_NO_SKINNY     0x800u  /* never use the few-rows kernel (M <= 16) */
#define OG_GEMM_NO_DIRECT     0x1000u /* never use the few-rows kernel's single-pass form (always split k) */
#define OG_GEMM_LARGE_TILE    0x2000u /* take the 256 x 256 tile kernels whatever the size (with NO_SKINNY: every shape) */
#define OG_GEMM_NO_STREAM     0x4000u /* never use the tiled few-rows kernel (the split-k one instead) */
#define OG_GEMM_TWO_PASS      0x8000u /* the tiled few-rows kernel in two launches (its parts added by a second kernel) */

/* Epi (Int8GemmEpilogue.hlsli:1-12): bit 0 float32 result, bit 1 int32 bias per column, bit 2 scale per column (else one),
 * bit 3 float32 bias per column. 0 stores the raw int32 sums. */
#define OG_EPI_FLOAT          0x1u
#define OG_EPI_INT_BIAS       0x2u
#define OG_EPI_SCALE_PER_COL  0x4u
#define OG_EPI_FLOAT_BIAS     0x8u

/* One product, Batch independent batches (Batch is the reference's dispatch z, Int8Gemm.cs:638):
 * C[b, m, n] = sum_k (A[b, m, k] - za)(B[b, k, n] - zb), int32 wrapping modulo 2^32, then the epilogue Epi asks for:
 * the int32 sum (+ bias), or fl(fl(float(sum + bias)) * scale) (+ fbias as a separate rounding). C is int32 or float32.
 * Replaces Int8Gemm.Multiply's dispatch (Int8Gemm.cs:554-639), i.e. the body of EncodeInt32 (230-253) and EncodeFloat
 * (270-314). A, B: uint8/int8 bytes; ZA/ZB: zero points in the operand's own type; bias: int32; scale, fbias: float32. */
int og_int8_gemm(og_ctx *ctx, const og_int8_gemm_params *params, uint32_t batch, og_buffer A, og_buffer B, og_buffer C,
                 og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer scale, og_buffer fbias);

/* og_int8_gemm that allocates nothing: no counterpart in the reference. For callers that cannot allocate device
 * memory (work captured into a HIP graph, serving loops, harnesses that forbid hipMalloc). The same product, kernels
 * and result; the scratch its kernels need (split-k and few-rows partial sums, the few-rows kernel's count words)
 * comes from one fixed array of OG_NOALLOC_SCRATCH_BYTES per device instead of the context's workspace. A product
 * that needs more fails with OG_ERR_UNSUPPORTED before anything is launched. Every call on a device shares that
 * device's array (whatever the context), so calls that overlap on one device race. */
#define OG_NOALLOC_SCRATCH_BYTES (16u << 20)
int og_int8_gemm_noalloc(og_ctx *ctx, const og_int8_gemm_params *params, uint32_t batch, og_buffer A, og_buffer B,
                         og_buffer C, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer scale, og_buffer fbias);

/* The kernel og_int8_gemm would run for these parameters (a stable name, e.g. "mfma-i8-tile256x256x64"), the HIP
 * counterpart of Int8Gemm.Variant (Int8Gemm.cs:214-215). Validates nothing; writes at most len bytes. */
int og_int8_gemm_kernel_name(const og_int8_gemm_params *params, uint32_t batch, char *buf, size_t len);

/* Int8EpilogueParams, 11 words (src/RecursiveAI.OneGpu.Kernels/Shaders/Int8Epilogue.hlsl:15-28). */
typedef struct og_int8_epilogue_params {
    uint32_t Count;     /* sums to finish */
    uint32_t OffAcc;    /* element offset of the int32 sums */
    uint32_t OffOut;    /* element offset of the output (bytes for mode 2) */
    uint32_t GridX;     /* ignored */
    uint32_t N;         /* columns: bias, scale and float bias are indexed by element % N */
    uint32_t Mode;      /* 0 int32 (+bias), 1 float32, 2 uint8/int8 requantized, 3 add float bias in place */
    uint32_t Flags;     /* bit 0 int bias present, bit 1 scale per column, bit 3 output uint8 (else int8) */
    uint32_t OffBias, OffScale, OffFBias;
    int32_t ZeroPoint;  /* output zero point of mode 2 */
} og_int8_epilogue_params;

/* The pass after the sums (Int8Gemm.Finish, Int8Gemm.cs:649-682): mode 2 is QLinearMatMul's requantization
 * clamp(round_half_even(float(sum + bias) * multiplier) + zeroPoint), NaN to the lowest value (Int8Epilogue.hlsl:54-68). */
int og_int8_epilogue(og_ctx *ctx, const og_int8_epilogue_params *params, og_buffer acc, og_buffer out, og_buffer bias,
                     og_buffer scale, og_buffer fbias);

/* MatMulIntegerToFloat with the scale product folded into the product's epilogue: the column scale is
 * fl(act_scale * scale[n or 0]), the f32 product the reference makes with a separate elementwise Mul before EncodeFloat
 * (Int8Tests.cs:738-745: DynamicQuantizeLinear's scale times the per-column weight scale), and each result is then what
 * og_int8_gemm with OG_EPI_FLOAT writes with that scale vector: fl(fl(float(sum + bias)) * s_n) (+ fbias as a separate
 * rounding). Replaces the Mul dispatch + Int8Gemm.EncodeFloat (Int8Gemm.cs:270-314) pair with one launch. params as
 * for og_int8_gemm with OG_EPI_FLOAT set; act_scale is one float32 at element act_offset of its buffer (e.g.
 * og_dynamic_quantize's scale output). */
int og_int8_gemm_float_scaled(og_ctx *ctx, const og_int8_gemm_params *params, uint32_t batch, og_buffer A, og_buffer B,
                              og_buffer C, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer act_scale,
                              uint32_t act_offset, og_buffer scale, og_buffer fbias);

/* Int8Gemm.EncodeRequantized (Int8Gemm.cs:336-363) in one launch: the product of og_int8_gemm and the mode-2 pass of
 * og_int8_epilogue, with the requantization applied where the product stores its sums, so the int32 sums never reach
 * memory and no scratch is used. Replaces the Multiply (554-639) + Finish (649-682) pair; each output byte equals what
 * the pair writes. params as for og_int8_gemm, except: C is Y, 8-bit, and OffC and StrideC count bytes; Epi may hold
 * only OG_EPI_INT_BIAS and OG_EPI_SCALE_PER_COL (the multiplier is one value, or one per column, at OffScale of
 * multiplier); zero_point_y lies in the output type's range; y_signed chooses int8 (else uint8) output. Bytes of Y
 * outside the product are not touched. */
int og_int8_gemm_requantized(og_ctx *ctx, const og_int8_gemm_params *params, uint32_t batch, og_buffer A, og_buffer B,
                             og_buffer Y, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer multiplier,
                             int32_t zero_point_y, uint32_t y_signed);

/* ------------------------------------------------------------------ DynamicQuantizeLinear */

/* DqParams, 7 words (src/RecursiveAI.OneGpu.Kernels/Shaders/DynamicQuantize.hlsl:13-22). GridX and Groups are the
 * reference's dispatch sizes and are ignored: the library sizes its own grid. */
typedef struct og_dq_params {
    uint32_t Count;     /* elements, >= 1 */
    uint32_t OffX;      /* element offset of the float32 input */
    uint32_t OffY;      /* byte offset of the uint8 output */
    uint32_t GridX;
    uint32_t Groups;
    uint32_t OffScale;  /* element offset of the float32 scale written */
    uint32_t OffZero;   /* byte offset of the uint8 zero point written (neighbouring bytes untouched) */
} og_dq_params;

/* DynamicQuantizeLinear on float32 (DynamicQuantizeKernels.Encode, DynamicQuantizeKernels.cs:59-90):
 * lo = min(0, min x), hi = max(0, max x), scale = (hi - lo) / 255 correctly rounded, zp = clamp(rne(-(lo / scale)), 0, 255),
 * y = clamp(rne(x / scale) + zp, 0, 255), NaN to 0; an all-zero range gives (1, 0). Uses a fixed workspace inside ctx. */
int og_dynamic_quantize(og_ctx *ctx, const og_dq_params *params, og_buffer X, og_buffer Y, og_buffer scale, og_buffer zero);

/* ------------------------------------------------------------------ quantizing a product's output without a read pass
 * (no counterpart in the reference: there, DynamicQuantizeLinear of a layer's float output starts with the DqMinMax
 * dispatch, a read of the whole tensor, DynamicQuantize.hlsl:35-69). */

/* (min, max) pairs a ranged product may write; its `ranges` buffer holds 2 * OG_RANGES_MAX float32. */
#define OG_RANGES_MAX 1024u

/* og_int8_gemm with OG_EPI_FLOAT (or, with act_scale given, og_int8_gemm_float_scaled) whose kernels also record the
 * range of the float values they store: *groups (min, max) pairs at `ranges` (8-byte aligned, 2 * OG_RANGES_MAX
 * float32) whose NaN-ignoring minimum and maximum are those of C. C is dense (StrideC = M * N when batch > 1) and holds
 * at most 2^31 - 1 elements. The direct MFMA kernels, the split-k summing pass and the one-launch few-rows kernel write
 * the pairs from their epilogue (one a workgroup, or a column slab); the other kernels are followed by a range pass
 * over C. C is bit for bit what og_int8_gemm (og_int8_gemm_float_scaled) writes. */
int og_int8_gemm_float_ranged(og_ctx *ctx, const og_int8_gemm_params *params, uint32_t batch, og_buffer A, og_buffer B,
                              og_buffer C, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer act_scale,
                              uint32_t act_offset, og_buffer scale, og_buffer fbias, og_buffer ranges,
                              uint32_t *groups);

/* og_dynamic_quantize of x whose range a ranged product recorded (its ranges and groups): the quantize pass alone, one
 * launch, no read pass. y, scale and zero point are bit for bit og_dynamic_quantize's when the pairs cover x (as
 * og_int8_gemm_float_ranged's cover its C). */
int og_dynamic_quantize_ranged(og_ctx *ctx, const og_dq_params *params, og_buffer X, og_buffer Y, og_buffer scale,
                               og_buffer zero, og_buffer ranges, uint32_t groups);

/* ------------------------------------------------------------------ DequantizeLinear / QuantizeLinear */

/* DequantizeParams / QuantizeParams, 9 words (Dequantize.hlsl:9-20, Quantize.hlsl:10-21). The tensor is seen as
 * [outer, AxisLen, Inner]; Flags bit 0 per axis, bit 1 zero point given. GridX is ignored. */
typedef struct og_dequant_params {
    uint32_t Count, OffX, OffO, OffS, OffZ, GridX, Flags, AxisLen, Inner;
} og_dequant_params;

#define OG_KIND_U8  0
#define OG_KIND_I8  1
#define OG_KIND_I32 2

/* y = fl((float)(x - zp) * scale[a]) with the subtraction wrapping in 32 bits; f16_out rounds that to binary16 (RNE).
 * Replaces DequantizeKernels.Encode<TIn, TOut> (DequantizeKernels.cs:64-150) and its DequantizeOp dispatch. */
int og_dequantize(og_ctx *ctx, int kind, int f16_out, const og_dequant_params *params, og_buffer X, og_buffer scale,
                  og_buffer zero, og_buffer out);

/* n DequantizeLinear passes of one count, axis and zero-point form (buffers and offsets their own) in one launch:
 * no counterpart in the reference, where each pass is a dispatch of its own. For recorders that see consecutive
 * passes, such as the per-batch rescale after a batched product whose batches have their own column scales; the
 * host mirror's encoder batches consecutive passes through it. Passes run together, so a pass's output may not
 * overlap another pass's operands (OG_ERR_INVALID_ARG, argument "output"); at most OG_DEQUANT_BATCH_MAX a call. */
#define OG_DEQUANT_BATCH_MAX 256u
int og_dequantize_batch(og_ctx *ctx, int kind, int f16_out, uint32_t n, const og_dequant_params *params,
                        const og_buffer *X, const og_buffer *scale, const og_buffer *zero, const og_buffer *out);

/* y = saturate(rne(x / scale[a]) + zp) with correctly rounded division, NaN to the lowest value; f16_in widens binary16
 * input exactly. Replaces DequantizeKernels.EncodeQuantize<TIn, TOut> (DequantizeKernels.cs:204-272). */
int og_quantize(og_ctx *ctx, int is_signed, int f16_in, const og_dequant_params *params, og_buffer X, og_buffer scale,
                og_buffer zero, og_buffer out);

/* ------------------------------------------------------------------ ConvInteger */

/* ConvProblem's fields (src/RecursiveAI.OneGpu.Kernels/ConvProblem.cs:107-235) and the operands' types: NCHW input,
 * OIHW weights, strides, dilations, asymmetric padding, groups. Offsets count elements (bytes of x and w, int32 of y);
 * the output extent is floor((in + padBegin + padEnd - dilation * (kernel - 1) - 1) / stride) + 1 per axis. */
typedef struct og_conv_params {
    uint32_t Batch, InChannels, Height, Width, OutChannels, KernelHeight, KernelWidth;
    uint32_t StrideHeight, StrideWidth, DilationHeight, DilationWidth;
    uint32_t PadTop, PadLeft, PadBottom, PadRight, Groups;
    uint32_t OffsetX, OffsetW, OffsetY;
    uint32_t Flags;       /* OG_CONV_* */
    uint32_t OffXZero;    /* element offset of x's zero point (one value) */
    uint32_t OffWZero;    /* element offset of w's zero point (one value, or one per output channel) */
    uint32_t GemmFlags;   /* OG_GEMM_PORTABLE / NO_SKINNY / NO_DIRECT / LARGE_TILE / NO_STREAM for the products */
} og_conv_params;

#define OG_CONV_X_INT8          0x1u  /* x is int8 (else uint8) */
#define OG_CONV_W_INT8          0x2u  /* w is int8 (else uint8) */
#define OG_CONV_XZ              0x4u  /* x has a zero point */
#define OG_CONV_WZ              0x8u  /* w has a zero point */
#define OG_CONV_WZ_PER_CHANNEL  0x10u /* ... one per output channel */
#define OG_CONV_NO_DEPTHWISE    0x20u /* convolutions with one input channel a group through the column matrix too */

/* Bytes of column scratch one image needs: Groups * Kp * ldb with K = InChannels / Groups * KernelHeight * KernelWidth,
 * ldb = OutHeight * OutWidth rounded up to 16 (ConvIntegerKernels.ScratchBytesPerImage, ConvIntegerKernels.cs:78-89,
 * which rounds to 4) and Kp = K, or, when 64 <= K and K % 64 != 0, K rounded up to 64 plus 16 + OutChannels * Kp
 * rounded up to 256 bytes for the weights in rows of Kp bytes. A scratch of n such figures holds n images' columns.
 * 0 when the geometry is invalid. */
uint64_t og_conv_integer_scratch_bytes(const og_conv_params *params);

/* ONNX ConvInteger: y[n, m, oh, ow] = sum over c, kh, kw of (x - xz) * (w - wz[m]) in 32-bit wrap-around; taps in the
 * padding add nothing. Replaces ConvIntegerKernels.Encode's dispatches (ConvIntegerKernels.cs:97-253): per chunk of
 * images that fits the scratch (bytes from scratch_offset, a multiple of 4), the column matrix is packed and then
 * multiplied, one batched product per group (the reference records one product per image and group). With one input
 * channel a group (depthwise) the library convolves directly, and a 1 x 1 window with unit strides and no padding
 * whose image rows are whole 16-byte multiples from a 16-byte aligned start multiplies the input as it lies; neither
 * uses the scratch (it may be absent). */
int og_conv_integer(og_ctx *ctx, const og_conv_params *params, og_buffer x, og_buffer w, og_buffer y, og_buffer xz,
                    og_buffer wz, og_buffer scratch, uint64_t scratch_offset);

/* ------------------------------------------------------------------ Gather (the int8 embedding lookup) */

/* GatherParams, 9 words (src/RecursiveAI.OneGpu.Kernels/Shaders/Gather.hlsl:6-17). The data tensor is seen as
 * [outer, AxisLen, Inner] elements, the output as [outer, IdxCount, Inner]; Count = outer * IdxCount * Inner. Offsets
 * count elements (indices: index elements). Flags bit 0: int64 indices (else int32). GridX is ignored. */
typedef struct og_gather_params {
    uint32_t Count, OffData, OffOut, OffIdx, GridX, Flags, Inner, IdxCount, AxisLen;
} og_gather_params;

/* out[o, i, n] = data[o, index[i], n] for elements of elem_bytes bytes (1: uint8/int8, 2: half, 4, 8); a negative
 * index counts from the end of the axis. An index outside [-AxisLen, AxisLen) reads nothing: its output elements are
 * zero and, when status is given (one uint32, initialised to 0xFFFFFFFF by the caller), the smallest such position is
 * recorded there with an atomic minimum. Output bytes outside the gathered range are left as they are. The output
 * must not overlap the data. Replaces GatherKernels.EncodeGather's dispatch (GatherKernels.cs:66-118, Gather.hlsl). */
int og_gather(og_ctx *ctx, uint32_t elem_bytes, const og_gather_params *params, og_buffer data, og_buffer indices,
              og_buffer out, og_buffer status);

/* ------------------------------------------------------------------ diagnostics */

const char *og_last_error(og_ctx *ctx);           /* text of the last failure (thread-local when ctx is NULL) */
const char *og_last_error_argument(og_ctx *ctx);  /* the argument at fault for OG_ERR_INVALID_ARG, else "" */
const char *og_last_kernel(og_ctx *ctx);          /* name of the last kernel launched on ctx */
const char *og_version(void);

/* ------------------------------------------------------------------ benchmark and test utilities
 * (no counterpart in the reference: synthetic data made on the device, so large inputs need no host round trip) */

/* Counter-based SplitMix64 stream `tensor` under `seed`, element i written to out[offset + i]:
 * kind 0: bytes uniform in [lo, hi] (as int8 or uint8 bits); kind 1: int32 uniform in [lo, hi];
 * kind 2: float32 N(lo = mean, hi = stddev) by Box-Muller in double. */
int og_util_synth(og_ctx *ctx, int kind, uint64_t seed, uint32_t tensor, og_buffer out, uint64_t offset, uint64_t count,
                  double lo, double hi);
/* scale[n] = fl(max_k |w[k, n]|) / divisor over a dense float32 [rows, cols] tensor (symmetric weight scales). */
int og_util_col_absmax_scale(og_ctx *ctx, og_buffer W, uint32_t rows, uint32_t cols, float divisor, og_buffer scale);
/* out[i] = fl(a[0] * b[i]) for i < n (the on-device scale product of the dynamic int8 chain). */
int og_util_scale_product(og_ctx *ctx, og_buffer a, og_buffer b, uint32_t n, og_buffer out);
/* Reads B [K x N] (dense int8 rows, N a multiple of 16, K * N < 2^31) once, in the tiles, workgroups and loads of
 * the one-launch few-rows product ("mfma-i8-rows16-xcd"), and does nothing else: the streaming floor that product is
 * measured against (kernel name "stream-tiles"). `sink` (4 bytes) is written only on an unlikely checksum. */
int og_util_stream_tiles(og_ctx *ctx, og_buffer B, uint32_t K, uint32_t N, og_buffer sink);

/* ------------------------------------------------------------------ test hooks
 * (no counterpart in the reference: they let a test drive the failure path of the one-launch few-rows product,
 * "mfma-i8-rows16-xcd", from the host, with every kernel still ending normally) */

/* Polls of a column slab's part count before that kernel's finishing tile gives up on ctx's later products (default
 * 4194304). 0: the finishing tile gives up at once, leaving its columns of C unwritten; og_sync then reports
 * OG_ERR_LAUNCH_FAILED, clears the count words and the context uses the two-launch form. */
int og_test_set_spin_limit(og_ctx *ctx, uint32_t polls);
/* How many of the count words are non-zero: ctx's own, and the device's fixed ones (og_int8_gemm_noalloc). Waits for
 * ctx's stream. */
int og_test_nonzero_words(og_ctx *ctx, uint64_t *context_words, uint64_t *fixed_words);

#ifdef __cplusplus
}
#endif
#endif /* ONEGPU_HIP_H */
