/*
 * CPU oracle for the int8 quantized-matmul path: a plain-C restatement of the reference's own CPU references
 * (the C# test oracles that define bit-exactness for MatMulInteger, QLinearMatMul, MatMulIntegerToFloat,
 * DynamicQuantizeLinear, DequantizeLinear and QuantizeLinear), plus the reference's deterministic test-data generators.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library, the host layer) links or calls this code; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only as the checker.
 *
 * Every function names the reference file:line it restates. Paths are relative to the reference repository root;
 * "tests/K" is tests/RecursiveAI.OneGpu.Kernels.Tests and "shaders" is src/RecursiveAI.OneGpu.Kernels/Shaders.
 */
#ifndef ONEGPU_ORACLE_H
#define ONEGPU_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The shape of one batch of products, with the meaning of Int8GemmProblem (src/RecursiveAI.OneGpu.Kernels/Int8Gemm.cs:43-95):
 * A is M x K (row stride Lda), B is K x N or, with TransposeB, N x K (row stride Ldb); Lda/Ldb 0 mean dense; offsets and
 * strides are in bytes for A and B and in elements for C; C is dense [Batch, M, N] at OffsetC. */
typedef struct {
    int32_t M, N, K, Batch, TransposeB, Lda, Ldb, OffsetA, OffsetB, OffsetC, StrideA, StrideB;
} ora_problem;

/* --- generators (bit-identical to the reference tests' data) --- */
void ora_bytes(uint8_t *out, int64_t len, int32_t seed);                                  /* tests/K/Int8Tests.cs:36-47 */
void ora_rig_random(float *out, int64_t n, int32_t seed, float lo, float hi);            /* tests/K/Rig.cs:8-19 */
void ora_dq_input(float *out, int64_t count, int32_t seed, int32_t kind);                 /* tests/K/Int8Tests.cs:627-647 */
void ora_dequant_input_i32(int32_t *out, int64_t n, int32_t seed);                        /* tests/K/DequantizeTests.cs:8-32 (int) */
void ora_dequant_input_bytes(uint8_t *out, int64_t n, int32_t seed);                      /* tests/K/DequantizeTests.cs:8-32 (byte/sbyte) */
void ora_quantize_input(float *out, int64_t n, int32_t seed, int32_t special);            /* tests/K/DequantizeTests.cs:159-177 */

/* Counter-based SplitMix64 streams for the benchmark configurations: value i of tensor `tensor` under `seed`. */
uint64_t ora_splitmix64(uint64_t x);
void ora_synth_uniform_i32(int32_t *out, int64_t n, uint64_t seed, uint32_t tensor, int32_t lo, int32_t hi);
void ora_synth_normal_f32(float *out, int64_t n, uint64_t seed, uint32_t tensor, float mean, float stddev);

/* --- the product --- */
/* Definition form: C = sum_k (A - za)(B - zb), int32 with wrap-around (tests/K/Int8Tests.cs:52-82). za/zb may be NULL (0);
 * *_vec selects one value per row of A / column of B; *_off is the element offset of the first zero point.
 * c receives the dense Batch*M*N sums (not offset). threads <= 1 runs on the calling thread. */
void ora_int8_gemm(const ora_problem *p, const uint8_t *a, int32_t a_signed, const uint8_t *b, int32_t b_signed,
                   const uint8_t *za, int32_t za_vec, int32_t za_off, const uint8_t *zb, int32_t zb_vec, int32_t zb_off,
                   int32_t *c, int32_t threads);

/* Signed-domain identity form (shaders/Int8GemmDot.hlsl:1-11, 134-140): s = u ^ 0x80, z' = z - 128,
 * sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w' (mod 2^32). An independent second computation. */
void ora_int8_gemm_identity(const ora_problem *p, const uint8_t *a, int32_t a_signed, const uint8_t *b, int32_t b_signed,
                            const uint8_t *za, int32_t za_vec, int32_t za_off, const uint8_t *zb, int32_t zb_vec, int32_t zb_off,
                            int32_t *c);

/* The same sums for a subset of rows (row indices over Batch*M), for checking large products by sampling. */
void ora_int8_gemm_rows(const ora_problem *p, const uint8_t *a, int32_t a_signed, const uint8_t *b, int32_t b_signed,
                        const uint8_t *za, int32_t za_vec, int32_t za_off, const uint8_t *zb, int32_t zb_vec, int32_t zb_off,
                        const int64_t *rows, int64_t nrows, int32_t *c, int32_t threads);

/* --- what follows the sums --- */
/* MatMulIntegerToFloat: f = (float)(sum + ib) * scale; then f += fb (tests/K/Int8Tests.cs:356-373). bias/fbias may be NULL. */
void ora_float_epilogue(const int32_t *sums, int64_t count, int32_t n, const int32_t *ibias, const float *scale,
                        int32_t scale_vec, const float *fbias, float *out);
/* QLinearMatMul requantization of one sum (tests/K/Int8Tests.cs:84-97). */
int32_t ora_requant(int32_t acc, float mult, int32_t zero, int32_t is_unsigned);
void ora_requant_array(const int32_t *sums, int64_t count, int32_t n, const int32_t *ibias, const float *mult,
                       int32_t mult_vec, int32_t zero, int32_t is_unsigned, uint8_t *out);

/* --- DynamicQuantizeLinear (tests/K/Int8Tests.cs:576-615) --- */
void ora_dynamic_quantize(const float *x, int64_t n, uint8_t *y, float *scale, uint8_t *zp);
/* The reference kernel's integer long division (shaders/DivExact.hlsli:4-99), to show it equals IEEE division. */
float ora_div_exact(float x, float s);

/* --- DequantizeLinear / QuantizeLinear --- */
uint16_t ora_f2h(float f);                               /* shaders/Common.hlsl:52-92 */
float ora_h2f(uint16_t h);                               /* shaders/Common.hlsl:30-48 */
/* kind 0 u8, 1 i8, 2 i32; y = (float)(x - zp) * scale[a], a = (j / inner) % axis_len when per_axis
 * (tests/K/DequantizeTests.cs:67-74). f16_out writes binary16 bits via ora_f2h into out16, else float into out32. */
void ora_dequantize(int32_t kind, const void *x, int64_t count, int32_t per_axis, int64_t axis_len, int64_t inner,
                    const float *scale, const void *zero, int32_t f16_out, float *out32, uint16_t *out16);
/* One QuantizeLinear value (tests/K/DequantizeTests.cs:147-157). */
int32_t ora_quantize_one(float x, float scale, int32_t zero, int32_t lo, int32_t hi);
void ora_quantize(const float *x, int64_t count, int32_t per_axis, int64_t axis_len, int64_t inner, const float *scale,
                  const uint8_t *zero, int32_t is_signed, uint8_t *out);

/* --- ConvInteger (tests/K/ConvIntegerTests.cs:42-89, Reference) --- */
/* NCHW input, OIHW weights, strides, dilations, asymmetric padding (top/left given; the output extent oh x ow is the
 * caller's), groups. y[n, m, i, j] = sum over c, kh, kw of (x - xz) * (w - wz[m]) in 32-bit wrap-around; taps in the
 * padding add nothing. xz: one byte or NULL; wz: one byte, or one per output channel (wz_vec), or NULL. */
typedef struct ora_conv {
    int32_t Batch, InChannels, Height, Width, OutChannels, KernelHeight, KernelWidth;
    int32_t StrideHeight, StrideWidth, DilationHeight, DilationWidth, PadTop, PadLeft, Groups;
    int32_t OutHeight, OutWidth;
} ora_conv;
void ora_conv_integer(const ora_conv *p, const uint8_t *x, int32_t x_signed, const uint8_t *w, int32_t w_signed,
                      const uint8_t *xz, const uint8_t *wz, int32_t wz_vec, int32_t *y, int32_t threads);

#ifdef __cplusplus
}
#endif
#endif
