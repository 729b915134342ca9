/*
 * CPU oracle for the int8 quantized-matmul path. TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg as the checker; never linked into or called by the product.
 *
 * Each function restates, in plain C, the reference's own CPU reference that its tests treat as the specification, and
 * cites it. Paths: "tests/K" = tests/RecursiveAI.OneGpu.Kernels.Tests, "shaders" = src/RecursiveAI.OneGpu.Kernels/Shaders.
 *
 * Build with -ffp-contract=off (no fused multiply-add): the C# references round every float operation separately.
 * int32 wrap-around is done in uint32_t so that no signed overflow occurs.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* C# MathF.Round(float): round half to even. */
static inline float round_even(float v) { return rintf(v); }

/* ------------------------------------------------------------------ generators */

/* tests/K/Int8Tests.cs:36-47 (identical in Int8ScratchTests.cs:6-17). */
void ora_bytes(uint8_t *out, int64_t len, int32_t seed)
{
    uint32_t s = (uint32_t)seed * 2654435761u + 7u;
    for (int64_t i = 0; i < len; i++) {
        s = s * 1664525u + 1013904223u;
        out[i] = (uint8_t)(s >> 24);
    }
}

/* tests/K/Rig.cs:8-19: lo + (hi - lo) * ((s >> 8) / 16777216f), float32 steps. */
void ora_rig_random(float *out, int64_t n, int32_t seed, float lo, float hi)
{
    uint32_t s = (uint32_t)seed * 2654435761u + 12345u;
    for (int64_t i = 0; i < n; i++) {
        s = s * 1664525u + 1013904223u;
        float t = (float)(s >> 8) / 16777216.0f;
        out[i] = lo + (hi - lo) * t;
    }
}

/* tests/K/Int8Tests.cs:633-647: the seven DynamicQuantizeLinear input distributions. */
void ora_dq_input(float *out, int64_t count, int32_t seed, int32_t kind)
{
    uint32_t s = (uint32_t)seed * 2654435761u + 99u;
    for (int64_t i = 0; i < count; i++) {
        s = s * 1664525u + 1013904223u;
        float t = (float)(s >> 8) / 16777216.0f;
        float u = (t * 2.0f) - 1.0f;
        float x;
        switch (kind) {
        case 0: x = u * 4.7f; break;
        case 1: x = (u + 1.0f) * 3.3f; break;
        case 2: x = -((u + 1.0f) * 0.0123f); break;
        case 3: { float c = (u * u) * u; x = c * 100.0f + 0.001f; break; }
        case 4: x = round_even(u * 127.0f) * 0.125f; break;
        case 5: x = 0.0f; break;
        default: x = u * 1e-3f; break;
        }
        out[i] = x;
    }
}

/* tests/K/DequantizeTests.cs:8-32, int32 branch: extremes every 17th / 19th element, else (int)h >> (i % 7). */
void ora_dequant_input_i32(int32_t *out, int64_t n, int32_t seed)
{
    uint32_t h = (uint32_t)seed * 2654435761u + 1u;
    for (int64_t i = 0; i < n; i++) {
        h = h * 1664525u + 1013904223u;
        out[i] = (i % 17 == 0) ? INT32_MIN : (i % 19 == 0) ? INT32_MAX : ((int32_t)h >> (i % 7));
    }
}

/* tests/K/DequantizeTests.cs:8-32, byte and sbyte branches: (byte)(h >> 16) (the sbyte is the same bits). */
void ora_dequant_input_bytes(uint8_t *out, int64_t n, int32_t seed)
{
    uint32_t h = (uint32_t)seed * 2654435761u + 1u;
    for (int64_t i = 0; i < n; i++) {
        h = h * 1664525u + 1013904223u;
        out[i] = (uint8_t)(h >> 16);
    }
}

/* tests/K/DequantizeTests.cs:159-177: random values plus ties, saturating values and (special) NaN, infinities,
 * a subnormal and signed zeros. */
void ora_quantize_input(float *out, int64_t n, int32_t seed, int32_t special)
{
    ora_rig_random(out, n, seed, -40.0f, 40.0f);
    for (int64_t i = 0; i < n; i++) {
        int32_t ii = (int32_t)i;
        switch (ii % 13) {
        case 3: out[i] = (float)(ii % 5 - 2) * 0.25f; break;
        case 5: out[i] = (float)(ii % 2 == 0 ? 1 : -1) * (100.0f + (float)ii); break;
        case 7: out[i] = (float)(ii % 9 - 4) + 0.5f; break;
        case 9:
            if (special) {
                int r = ii % 4;
                out[i] = r == 0 ? u2f(0xFFC00000u) /* C# float.NaN */ : r == 1 ? INFINITY : r == 2 ? -INFINITY : 1e-42f;
            }
            break;
        case 11:
            if (special) out[i] = (ii % 2 == 0) ? 0.0f : -0.0f;
            break;
        default: break;
        }
    }
}

uint64_t ora_splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static inline uint64_t synth_key(uint64_t seed, uint32_t tensor) { return ora_splitmix64((seed << 32) ^ (uint64_t)tensor); }

/* Uniform integers in [lo, hi] by the multiply-shift map of the top 32 bits. */
void ora_synth_uniform_i32(int32_t *out, int64_t n, uint64_t seed, uint32_t tensor, int32_t lo, int32_t hi)
{
    uint64_t key = synth_key(seed, tensor);
    uint64_t range = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (int64_t i = 0; i < n; i++) {
        uint64_t x = ora_splitmix64(key + (uint64_t)i);
        out[i] = (int32_t)((int64_t)lo + (int64_t)(((x >> 32) * range) >> 32));
    }
}

/* N(mean, stddev) by Box-Muller in double from two 53-bit uniforms, rounded once to float. */
void ora_synth_normal_f32(float *out, int64_t n, uint64_t seed, uint32_t tensor, float mean, float stddev)
{
    uint64_t key = synth_key(seed, tensor);
    for (int64_t i = 0; i < n; i++) {
        uint64_t x = ora_splitmix64(key + (uint64_t)i);
        uint64_t y = ora_splitmix64(x ^ 0xD1B54A32D192ED03ull);
        double u1 = (double)((x >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(y >> 11) * 0x1.0p-53;
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)((double)mean + (double)stddev * z);
    }
}

/* ------------------------------------------------------------------ the product */

static inline int32_t val(uint8_t b, int32_t is_signed) { return is_signed ? (int32_t)(int8_t)b : (int32_t)b; }

static int32_t lda_of(const ora_problem *p) { return p->Lda == 0 ? (p->K > 0 ? p->K : 1) : p->Lda; }
static int32_t ldb_of(const ora_problem *p)
{
    int32_t cols = p->TransposeB ? p->K : p->N;
    return p->Ldb == 0 ? (cols > 0 ? cols : 1) : p->Ldb;
}

typedef struct {
    const ora_problem *p;
    const uint8_t *a, *b, *za, *zb;
    int32_t a_signed, b_signed, za_vec, za_off, zb_vec, zb_off;
    const int64_t *rows;   /* NULL: all rows */
    int64_t row_begin, row_end;
    int32_t *c;
} gemm_job;

/* One output row (row = batch * M + m), as tests/K/Int8Tests.cs:57-80: arow[k] = A - zA; acc += arow[k] * (B - zB) with wrap. */
static void gemm_row(const gemm_job *j, int64_t row, int32_t *crow, int32_t *arow, uint32_t *acc, int32_t *zbv)
{
    const ora_problem *p = j->p;
    int64_t bt = row / p->M, m = row % p->M;
    int32_t lda = lda_of(p), ldb = ldb_of(p);
    int32_t zA = j->za ? val(j->za[j->za_off + (j->za_vec ? m : 0)], j->a_signed) : 0;
    const uint8_t *arow_src = j->a + p->OffsetA + bt * (int64_t)p->StrideA + m * (int64_t)lda;
    for (int32_t k = 0; k < p->K; k++) arow[k] = val(arow_src[k], j->a_signed) - zA;
    const uint8_t *bbase = j->b + p->OffsetB + bt * (int64_t)p->StrideB;
    if (!p->TransposeB) {
        /* k outer, n inner: the same terms summed in the same k order per element, vectorisable. */
        for (int32_t n = 0; n < p->N; n++) acc[n] = 0u;
        for (int32_t k = 0; k < p->K; k++) {
            const uint8_t *brow = bbase + (int64_t)k * ldb;
            int32_t av = arow[k];
            if (j->b_signed) {
                for (int32_t n = 0; n < p->N; n++) acc[n] += (uint32_t)(av * ((int32_t)(int8_t)brow[n] - zbv[n]));
            } else {
                for (int32_t n = 0; n < p->N; n++) acc[n] += (uint32_t)(av * ((int32_t)brow[n] - zbv[n]));
            }
        }
        for (int32_t n = 0; n < p->N; n++) crow[n] = (int32_t)acc[n];
    } else {
        for (int32_t n = 0; n < p->N; n++) {
            const uint8_t *bcol = bbase + (int64_t)n * ldb;
            int32_t zB = zbv[n];
            uint32_t s = 0u;
            for (int32_t k = 0; k < p->K; k++) s += (uint32_t)(arow[k] * (val(bcol[k], j->b_signed) - zB));
            crow[n] = (int32_t)s;
        }
    }
}

static void *gemm_worker(void *arg)
{
    gemm_job *j = (gemm_job *)arg;
    const ora_problem *p = j->p;
    int32_t *arow = (int32_t *)malloc(sizeof(int32_t) * (size_t)(p->K > 0 ? p->K : 1));
    uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(p->N > 0 ? p->N : 1));
    int32_t *zbv = (int32_t *)malloc(sizeof(int32_t) * (size_t)(p->N > 0 ? p->N : 1));
    for (int32_t n = 0; n < p->N; n++) zbv[n] = j->zb ? val(j->zb[j->zb_off + (j->zb_vec ? n : 0)], j->b_signed) : 0;
    for (int64_t r = j->row_begin; r < j->row_end; r++) {
        int64_t row = j->rows ? j->rows[r] : r;
        gemm_row(j, row, j->c + r * (int64_t)p->N, arow, acc, zbv);
    }
    free(arow);
    free(acc);
    free(zbv);
    return NULL;
}

static void gemm_run(gemm_job base, int64_t nrows, int32_t threads)
{
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (nrows < threads) threads = (int32_t)(nrows > 0 ? nrows : 1);
    pthread_t tid[64];
    gemm_job jobs[64];
    int64_t per = (nrows + threads - 1) / threads;
    int started = 0;
    for (int32_t t = 0; t < threads; t++) {
        jobs[t] = base;
        jobs[t].row_begin = (int64_t)t * per;
        jobs[t].row_end = jobs[t].row_begin + per < nrows ? jobs[t].row_begin + per : nrows;
        if (jobs[t].row_begin >= jobs[t].row_end) continue;
        if (threads == 1 || pthread_create(&tid[t], NULL, gemm_worker, &jobs[t]) != 0) {
            gemm_worker(&jobs[t]);
            jobs[t].row_end = -1; /* ran inline */
        } else {
            started++;
        }
    }
    for (int32_t t = 0; t < threads; t++) {
        if (jobs[t].row_begin < jobs[t].row_end) pthread_join(tid[t], NULL);
    }
    (void)started;
}

/* tests/K/Int8Tests.cs:52-82 (Reference). */
void ora_int8_gemm(const ora_problem *p, const uint8_t *a, int32_t a_signed, const uint8_t *b, int32_t b_signed,
                   const uint8_t *za, int32_t za_vec, int32_t za_off, const uint8_t *zb, int32_t zb_vec, int32_t zb_off,
                   int32_t *c, int32_t threads)
{
    int64_t nrows = (int64_t)p->Batch * p->M;
    if (nrows <= 0 || p->N <= 0) return;
    gemm_job j = {p, a, b, za, zb, a_signed, b_signed, za_vec, za_off, zb_vec, zb_off, NULL, 0, 0, c};
    gemm_run(j, nrows, threads);
}

void ora_int8_gemm_rows(const ora_problem *p, const uint8_t *a, int32_t a_signed, const uint8_t *b, int32_t b_signed,
                        const uint8_t *za, int32_t za_vec, int32_t za_off, const uint8_t *zb, int32_t zb_vec, int32_t zb_off,
                        const int64_t *rows, int64_t nrows, int32_t *c, int32_t threads)
{
    if (nrows <= 0 || p->N <= 0) return;
    gemm_job j = {p, a, b, za, zb, a_signed, b_signed, za_vec, za_off, zb_vec, zb_off, rows, 0, 0, c};
    gemm_run(j, nrows, threads);
}

/* shaders/Int8GemmDot.hlsl:1-11 and 134-140: the signed-domain rewrite, computed independently of the definition. */
void ora_int8_gemm_identity(const ora_problem *p, const uint8_t *a, int32_t a_signed, const uint8_t *b, int32_t b_signed,
                            const uint8_t *za, int32_t za_vec, int32_t za_off, const uint8_t *zb, int32_t zb_vec, int32_t zb_off,
                            int32_t *c)
{
    int32_t lda = lda_of(p), ldb = ldb_of(p);
    uint8_t flip_a = a_signed ? 0 : 0x80, flip_b = b_signed ? 0 : 0x80;
    for (int64_t bt = 0; bt < p->Batch; bt++) {
        for (int32_t m = 0; m < p->M; m++) {
            /* z' = z - 128 for an unsigned operand (its bytes move by -128), z for a signed one. */
            int32_t zr = za ? val(za[za_off + (za_vec ? m : 0)], a_signed) : 0;
            if (!a_signed) zr -= 128;
            const uint8_t *ar = a + p->OffsetA + bt * (int64_t)p->StrideA + (int64_t)m * lda;
            for (int32_t n = 0; n < p->N; n++) {
                int32_t wc = zb ? val(zb[zb_off + (zb_vec ? n : 0)], b_signed) : 0;
                if (!b_signed) wc -= 128;
                uint32_t dot = 0, sum_s = 0, sum_t = 0;
                for (int32_t k = 0; k < p->K; k++) {
                    int64_t bi = p->OffsetB + bt * (int64_t)p->StrideB + (p->TransposeB ? (int64_t)n * ldb + k : (int64_t)k * ldb + n);
                    int32_t s = (int32_t)(int8_t)(uint8_t)(ar[k] ^ flip_a);
                    int32_t t = (int32_t)(int8_t)(uint8_t)(b[bi] ^ flip_b);
                    dot += (uint32_t)(s * t);
                    sum_s += (uint32_t)s;
                    sum_t += (uint32_t)t;
                }
                uint32_t r = dot - (uint32_t)wc * sum_s - (uint32_t)zr * sum_t + (uint32_t)p->K * (uint32_t)zr * (uint32_t)wc;
                c[(bt * p->M + m) * (int64_t)p->N + n] = (int32_t)r;
            }
        }
    }
}

/* ------------------------------------------------------------------ epilogues */

/* tests/K/Int8Tests.cs:356-373: acc = sum + ib (wrap); f = (float)acc * scale; f += fb. Two separate roundings. */
void ora_float_epilogue(const int32_t *sums, int64_t count, int32_t n, const int32_t *ibias, const float *scale,
                        int32_t scale_vec, const float *fbias, float *out)
{
    for (int64_t i = 0; i < count; i++) {
        int32_t col = (int32_t)(i % n);
        int32_t acc = sums[i];
        if (ibias) acc = (int32_t)((uint32_t)acc + (uint32_t)ibias[col]);
        float f = (float)acc * scale[scale_vec ? col : 0];
        if (fbias) f = f + fbias[col];
        out[i] = f;
    }
}

/* tests/K/Int8Tests.cs:84-97 (Requant). */
int32_t ora_requant(int32_t acc, float mult, int32_t zero, int32_t is_unsigned)
{
    int32_t lo = is_unsigned ? 0 : -128, hi = is_unsigned ? 255 : 127;
    float v = (float)acc * mult;
    if (isnan(v)) return lo;
    float r = round_even(v);
    float cmin = (float)(lo - zero), cmax = (float)(hi - zero);
    r = r < cmin ? cmin : (r > cmax ? cmax : r);  /* Math.Clamp(float, float, float) */
    return (int32_t)r + zero;
}

void ora_requant_array(const int32_t *sums, int64_t count, int32_t n, const int32_t *ibias, const float *mult,
                       int32_t mult_vec, int32_t zero, int32_t is_unsigned, uint8_t *out)
{
    for (int64_t i = 0; i < count; i++) {
        int32_t col = (int32_t)(i % n);
        int32_t acc = sums[i];
        if (ibias) acc = (int32_t)((uint32_t)acc + (uint32_t)ibias[col]);
        out[i] = (uint8_t)ora_requant(acc, mult[mult_vec ? col : 0], zero, is_unsigned);
    }
}

/* ------------------------------------------------------------------ DynamicQuantizeLinear */

/* tests/K/Int8Tests.cs:576-615 (DynamicReference, "onemodel's DynamicQuantizeLinear"). */
void ora_dynamic_quantize(const float *x, int64_t n, uint8_t *y, float *scale_out, uint8_t *zp_out)
{
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    /* Math.Min(0f, min) and Math.Max(0f, max) (IEEE 754-2019 minimum/maximum: -0 < +0). NaN cannot reach them here
     * because a NaN never wins a < or > compare. The sign of a zero bound cannot change scale or zero point. */
    float lo = mn <= 0.0f ? mn : 0.0f;
    float hi = mx > 0.0f ? mx : 0.0f;
    float scale = (hi - lo) / 255.0f;
    int32_t zp = 0;
    if (scale != 0.0f && isfinite(scale)) {
        float z = round_even(0.0f - (lo / scale));
        zp = z < 0.0f ? 0 : (z > 255.0f ? 255 : (int32_t)z);
    }
    if (scale == 0.0f) {
        memset(y, 0, (size_t)n);
        *scale_out = 1.0f;
        *zp_out = 0;
        return;
    }
    for (int64_t i = 0; i < n; i++) {
        float v = round_even(x[i] / scale) + (float)zp;
        y[i] = isnan(v) ? 0 : (v < 0.0f ? 0 : (v > 255.0f ? 255 : (uint8_t)(int32_t)v));
    }
    *scale_out = scale;
    *zp_out = (uint8_t)zp;
}

/* shaders/DivExact.hlsli:4-26 (Unpack): 24-bit mantissa with its top bit set, subnormals normalised. */
static void unpack(uint32_t bits, uint32_t *m, int32_t *e)
{
    *e = (int32_t)((bits >> 23) & 255u);
    *m = bits & 0x7FFFFFu;
    if (*e == 0) {
        *e = 1;
        while (*m < 0x800000u) { *m <<= 1; *e -= 1; }
    } else {
        *m |= 0x800000u;
    }
}

/* shaders/DivExact.hlsli:28-99 (DivExact): long division, 26 quotient bits plus sticky, round to nearest even. */
float ora_div_exact(float x, float s)
{
    uint32_t xb = f2u(x), sb = f2u(s);
    uint32_t xa = xb & 0x7FFFFFFFu, sa = sb & 0x7FFFFFFFu;
    if (xa == 0u && sa != 0u && sa <= 0x7F800000u) return u2f((xb ^ sb) & 0x80000000u);
    if (xa == 0u || sa == 0u || xa >= 0x7F800000u || sa >= 0x7F800000u) return x / s;
    uint32_t ma, mb;
    int32_t ea, eb;
    unpack(xa, &ma, &ea);
    unpack(sa, &mb, &eb);
    uint32_t r = ma, q = 0u;
    if (r >= mb) { q = 1u; r -= mb; }
    for (int i = 0; i < 26; i++) {
        r <<= 1;
        q <<= 1;
        if (r >= mb) { q |= 1u; r -= mb; }
    }
    int32_t e = ea - eb + 127;
    uint32_t shift = 2u;
    if (q >= 0x4000000u) shift = 3u; else e -= 1;
    uint32_t m = q >> shift, rest = q & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    int sticky = r != 0u;
    if (rest > half || (rest == half && (sticky || (m & 1u) != 0u))) {
        m += 1u;
        if (m == 0x1000000u) { m >>= 1; e += 1; }
    }
    if (e < 1 || e > 254) return x / s;
    return u2f(((xb ^ sb) & 0x80000000u) | ((uint32_t)e << 23) | (m & 0x7FFFFFu));
}

/* ------------------------------------------------------------------ (de)quantize */

/* shaders/Common.hlsl:52-92 (F2H): binary32 to binary16, round to nearest even, overflow to infinity, NaN to quiet NaN. */
uint16_t ora_f2h(float f)
{
    uint32_t x = f2u(f);
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

/* shaders/Common.hlsl:32-49 (H2F): binary16 to binary32, exact. */
float ora_h2f(uint16_t h)
{
    uint32_t s = ((uint32_t)h & 0x8000u) << 16, e = ((uint32_t)h >> 10) & 31u, m = (uint32_t)h & 1023u;
    if (e == 0u) return u2f(f2u((float)m * (1.0f / 16777216.0f)) | s);
    if (e == 31u) return u2f(s | 0x7F800000u | (m << 13));
    return u2f(s | ((e + 112u) << 23) | (m << 13));
}

static inline int32_t load_q(int32_t kind, const void *p, int64_t i)
{
    if (kind == 0) return (int32_t)((const uint8_t *)p)[i];
    if (kind == 1) return (int32_t)((const int8_t *)p)[i];
    return ((const int32_t *)p)[i];
}

/* tests/K/DequantizeTests.cs:67-74: want = (float)unchecked(x - zp) * scale[a]; half output is (Half)want (RNE). */
void ora_dequantize(int32_t kind, const void *x, int64_t count, int32_t per_axis, int64_t axis_len, int64_t inner,
                    const float *scale, const void *zero, int32_t f16_out, float *out32, uint16_t *out16)
{
    for (int64_t j = 0; j < count; j++) {
        int64_t a = per_axis ? (j / inner) % axis_len : 0;
        int32_t zp = zero ? load_q(kind, zero, a) : 0;
        int32_t d = (int32_t)((uint32_t)load_q(kind, x, j) - (uint32_t)zp);
        float want = (float)d * scale[a];
        if (f16_out) out16[j] = ora_f2h(want); else out32[j] = want;
    }
}

/* tests/K/DequantizeTests.cs:147-157 (QuantizeOne): v = round_half_even(x / scale) + zp in float32; NaN to lo; clamp. */
int32_t ora_quantize_one(float x, float scale, int32_t zero, int32_t lo, int32_t hi)
{
    float v = round_even(x / scale) + (float)zero;
    if (isnan(v)) return lo;
    return v < (float)lo ? lo : (v > (float)hi ? hi : (int32_t)v);
}

void ora_quantize(const float *x, int64_t count, int32_t per_axis, int64_t axis_len, int64_t inner, const float *scale,
                  const uint8_t *zero, int32_t is_signed, uint8_t *out)
{
    int32_t lo = is_signed ? -128 : 0, hi = is_signed ? 127 : 255;
    for (int64_t j = 0; j < count; j++) {
        int64_t a = per_axis ? (j / inner) % axis_len : 0;
        int32_t zp = zero ? (is_signed ? (int32_t)(int8_t)zero[a] : (int32_t)zero[a]) : 0;
        out[j] = (uint8_t)ora_quantize_one(x[j], scale[a], zp, lo, hi);
    }
}


/* ------------------------------------------------------------------ ConvInteger */

typedef struct conv_job {
    const ora_conv *p;
    const uint8_t *x, *w, *xz, *wz;
    int32_t x_signed, w_signed, wz_vec;
    int32_t *y;
    int64_t row_begin, row_end;   /* rows are (n, m) pairs */
} conv_job;

/* tests/K/ConvIntegerTests.cs:42-89: one output plane per (image, output channel). */
static void *conv_worker(void *arg)
{
    const conv_job *j = (const conv_job *)arg;
    const ora_conv *p = j->p;
    const int32_t oh = p->OutHeight, ow = p->OutWidth;
    const int32_t cin_g = p->InChannels / p->Groups, cout_g = p->OutChannels / p->Groups;
    const int32_t xzv = j->xz ? val(j->xz[0], j->x_signed) : 0;
    for (int64_t row = j->row_begin; row < j->row_end; row++) {
        const int64_t n = row / p->OutChannels, m = row % p->OutChannels, g = m / cout_g;
        const int32_t wzv = j->wz ? val(j->wz[j->wz_vec ? m : 0], j->w_signed) : 0;
        for (int32_t i = 0; i < oh; i++) {
            for (int32_t jj = 0; jj < ow; jj++) {
                uint32_t acc = 0;
                for (int32_t c = 0; c < cin_g; c++) {
                    for (int32_t kh = 0; kh < p->KernelHeight; kh++) {
                        const int64_t ih = (int64_t)i * p->StrideHeight + (int64_t)kh * p->DilationHeight - p->PadTop;
                        if (ih < 0 || ih >= p->Height) continue;
                        for (int32_t kw = 0; kw < p->KernelWidth; kw++) {
                            const int64_t iw = (int64_t)jj * p->StrideWidth + (int64_t)kw * p->DilationWidth - p->PadLeft;
                            if (iw < 0 || iw >= p->Width) continue;
                            const int64_t xi = ((n * p->InChannels + g * cin_g + c) * p->Height + ih) * p->Width + iw;
                            const int64_t wi = ((m * cin_g + c) * p->KernelHeight + kh) * p->KernelWidth + kw;
                            const int32_t xv = val(j->x[xi], j->x_signed) - xzv;
                            const int32_t wv = val(j->w[wi], j->w_signed) - wzv;
                            acc += (uint32_t)xv * (uint32_t)wv;
                        }
                    }
                }
                j->y[((n * p->OutChannels + m) * oh + i) * ow + jj] = (int32_t)acc;
            }
        }
    }
    return NULL;
}

void ora_conv_integer(const ora_conv *p, const uint8_t *x, int32_t x_signed, const uint8_t *w, int32_t w_signed,
                      const uint8_t *xz, const uint8_t *wz, int32_t wz_vec, int32_t *y, int32_t threads)
{
    const int64_t rows = (int64_t)p->Batch * p->OutChannels;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (rows < threads) threads = (int32_t)(rows > 0 ? rows : 1);
    pthread_t tid[64];
    conv_job jobs[64];
    int started[64] = {0};
    const int64_t per = (rows + threads - 1) / threads;
    for (int32_t t = 0; t < threads; t++) {
        jobs[t] = (conv_job){p, x, w, xz, wz, x_signed, w_signed, wz_vec, y, (int64_t)t * per, 0};
        jobs[t].row_end = jobs[t].row_begin + per < rows ? jobs[t].row_begin + per : rows;
        if (jobs[t].row_begin >= jobs[t].row_end) continue;
        if (threads > 1 && pthread_create(&tid[t], NULL, conv_worker, &jobs[t]) == 0) started[t] = 1;
        else conv_worker(&jobs[t]);
    }
    for (int32_t t = 0; t < threads; t++)
        if (started[t]) pthread_join(tid[t], NULL);
}
