// The large-product int8 MFMA kernel: operands go from HBM straight into a ring of LDS stages (buffer_load ... lds,
// no staging registers), and B stored K x N is read in its own layout with the gfx950 transpose read
// ds_read_b64_tr_b8, so no VALU transposition is needed.
//
//  - Tile 256 x 256 x 64 per stage, 4 waves (2 x 2) of 128 x 128, v_mfma_i32_16x16x64_i8, NS stages in flight.
//  - Operands stay unsigned in LDS; each MFMA fragment is moved to the signed domain (s = u ^ 0x80) after it is read,
//    and the zero points are applied at the store from byte sums of the fragments:
//        sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w'   (mod 2^32; Int8GemmDot.hlsl:1-11 rearranges the same)
//  - LDS layouts (16-byte chunks, conflict-free for the fragment reads as measured with SQ_LDS_BANK_CONFLICT):
//      A (and B stored N x K): row r of 64 bytes, chunk q at position q ^ ((r >> 1) & 3);
//      B stored K x N: row k of 256 bytes, chunk c at position c ^ fB(k), fB(k) = (k & 7) | (((k >> 4) & 1) << 3).
//    A buffer load writes 64 lanes x 16 bytes to consecutive LDS, so each lane loads the global chunk that belongs in
//    its slot.
//  - A fragment (lane l: row l % 16, k 16 (l / 16) .. + 15) is one ds_read_b128. A B fragment (lane l: column l % 16,
//    the same 16 k) is two ds_read_b64_tr_b8: within each 16-lane group, lane i < 8 receives byte i of the 8-byte
//    segments the even lanes address and lane 8 + i byte i of the odd lanes' segments, so even lanes address rows
//    k..k+7 at columns n..n+7 and odd lanes the same rows at columns n+8..n+15.
#include <type_traits>

#include "og_internal.hpp"

namespace og {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u4w __attribute__((ext_vector_type(4)));
#define OG_LDS2(p) ((__attribute__((address_space(3))) v2i *)(p))

namespace {

constexpr int DBM = 256, DBN = 256, DBK = 64, DTHREADS = 256;
constexpr int A_STAGE = DBM * DBK;   // bytes
constexpr int B_STAGE = DBK * DBN;
constexpr int LOADS_A = A_STAGE / 16 / DTHREADS;   // 16-byte buffer loads per thread per stage
constexpr int LOADS_B = B_STAGE / 16 / DTHREADS;
constexpr int LOADS = LOADS_A + LOADS_B;

// Buffer resource words for `bytes` bytes at `base` (raw buffer: no stride, no swizzle; reads past the range
// return zero).
__device__ __forceinline__ u4w drsrc(const uint8_t *base, int64_t bytes)
{
    const uint32_t n = bytes <= 0 ? 0u : (bytes >= 0xFFFFFFFFll ? 0xFFFFFFFFu : (uint32_t)bytes);
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return (u4w){(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, n, 0x00020000u};
}

// LDS byte address of a __shared__ location.
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// One LDS DMA: lane l's 16 bytes at rsrc + voff land at LDS address lds + 16 l. Issued from inline assembly so that
// the compiler neither reorders LDS accesses across it nor adds waits of its own for it: the stages below wait for
// exactly the loads they need (vmcnt counts these loads in issue order).
__device__ __forceinline__ void dma16(u4w rsrc, uint32_t lds, uint32_t voff)
{
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

__device__ __forceinline__ int a_pos(int r, int q) { return q ^ ((r >> 1) & 3); }
__device__ __forceinline__ int b_pos(int k, int c) { return c ^ ((k & 7) | (((k >> 4) & 1) << 3)); }

// Waits until at most N of this wave's DMA loads are outstanding, then meets the other waves. A compiler barrier as
// well: no LDS access moves across it.
template <int N>
__device__ __forceinline__ void wait_vm_barrier()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// This wave's LDS accesses done, then meet the other waves.
__device__ __forceinline__ void wait_lgkm_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

}  // namespace

template <int NS, bool TRANS_B, bool SUM_A, bool SUM_B>
__global__ __launch_bounds__(DTHREADS) void k_gemm_direct(GemmArgs g, int32_t tiles_n, int32_t tiles_m)
{
    // One array per stage (fixed LDS addresses for every stage of the unrolled loop).
    __shared__ __attribute__((aligned(1024))) uint8_t A0[A_STAGE], A1[A_STAGE], A2[NS > 2 ? A_STAGE : 16], A3[NS > 3 ? A_STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t B0[B_STAGE], B1[B_STAGE], B2[NS > 2 ? B_STAGE : 16], B3[NS > 3 ? B_STAGE : 16];
    __shared__ __attribute__((aligned(16))) int32_t RowSum[SUM_A ? DBM : 1];
    __shared__ __attribute__((aligned(16))) int32_t RowZ[SUM_B ? DBM : 1];
    __shared__ int32_t ColSum[SUM_B ? DBN : 1];
    __shared__ int32_t ColW[SUM_A ? DBN : 1];
    __shared__ int32_t ColIB[DBN];
    __shared__ float ColSc[DBN], ColFb[DBN];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g4 = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;

    // Tile order: an XCD-contiguous run of tiles, walked in groups of 8 row-tiles (see the aligned kernel).
    const int64_t tiles = (int64_t)tiles_n * tiles_m;
    const int64_t nblocks = tiles * g.batch;
    int64_t bid = blockIdx.x;
    if ((nblocks & 7) == 0) bid = (bid & 7) * (nblocks >> 3) + (bid >> 3);
    const int32_t batch = (int32_t)(bid / tiles);
    const int64_t t = bid % tiles;
    int32_t tm, tn;
    {
        const int32_t GROUP = 8;
        const int64_t per_group = (int64_t)GROUP * tiles_n;
        const int32_t first_m = (int32_t)(t / per_group * GROUP);
        const int32_t gsize = min(tiles_m - first_m, GROUP);
        const int64_t in = t % per_group;
        tm = first_m + (int32_t)(in % gsize);
        tn = (int32_t)(in / gsize);
    }
    const int32_t m0 = tm * DBM, n0 = tn * DBN;
    const int32_t lda = g.lda, ldb = g.ldb, K = g.K;
    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    const uint32_t flip_a = a_signed ? 0u : 0x80808080u, flip_b = b_signed ? 0u : 0x80808080u;

    // The epilogue's per-row and per-column parameters, fetched now so that their latency hides behind the loop:
    // thread t holds row m0 + t's zero point and column n0 + t's zero point, int bias, scale and float bias (in the
    // signed domain; an absent zero point of an unsigned operand is -128 there, of a signed one 0).
    const uint32_t epi = g.epi;
    const int32_t my_m = min(m0 + tid, g.M - 1), my_n = min(n0 + tid, g.N - 1);
    // Raw zero-point bytes (0 when absent); moved to the signed domain after the loop, so nothing waits for them here.
    const uint32_t za_raw = (SUM_B && g.ZA) ? g.ZA[(g.flags & OG_GEMM_ZA_PER_ROW) ? my_m : 0] : 0u;
    const uint32_t zb_raw = (SUM_A && g.ZB) ? g.ZB[(g.flags & OG_GEMM_ZB_PER_COL) ? my_n : 0] : 0u;
    const int32_t my_ib = (epi & OG_EPI_INT_BIAS) ? g.bias[my_n] : 0;
    const float my_sc = (epi & OG_EPI_FLOAT) ? g.scale[(epi & OG_EPI_SCALE_PER_COL) ? my_n : 0] : 0.0f;
    const float my_fb = (epi & OG_EPI_FLOAT_BIAS) ? g.fbias[my_n] : 0.0f;

    // This tile's operand ranges: loads past the last valid byte return zeros. With K = 0 the operands may be absent
    // and nothing is read (the prologue still issues its loads, over empty ranges).
    const uint8_t *a_base = g.A + batch * g.strideA + (int64_t)m0 * lda;
    const int64_t a_valid = K > 0 ? (int64_t)(min(g.M - m0, DBM) - 1) * lda + K : 0;
    const uint8_t *b_base;
    int64_t b_valid, b_step;
    if constexpr (TRANS_B) {
        b_base = g.B + batch * g.strideB + (int64_t)n0 * ldb;
        b_valid = K > 0 ? (int64_t)(min(g.N - n0, DBN) - 1) * ldb + K : 0;
        b_step = 1;
    } else {
        b_base = g.B + batch * g.strideB + n0;
        b_valid = K > 0 ? (int64_t)(K - 1) * ldb + min(g.N - n0, DBN) : 0;
        b_step = ldb;
    }

    // Per-thread global offsets of the chunks that land in this thread's LDS slots (the same at every stage).
    uint32_t off_a[LOADS_A], off_b[LOADS_B];
#pragma unroll
    for (int i = 0; i < LOADS_A; i++) {
        const int s = (i * 4 + wave) * 64 + lane, r = s >> 2, p = s & 3;
        off_a[i] = (uint32_t)r * (uint32_t)lda + 16u * (uint32_t)a_pos(r, p);
    }
#pragma unroll
    for (int i = 0; i < LOADS_B; i++) {
        const int s = (i * 4 + wave) * 64 + lane;
        if constexpr (TRANS_B) {
            const int r = s >> 2, p = s & 3;
            off_b[i] = (uint32_t)r * (uint32_t)ldb + 16u * (uint32_t)a_pos(r, p);
        } else {
            const int k = s >> 4, p = s & 15;
            off_b[i] = (uint32_t)k * (uint32_t)ldb + 16u * (uint32_t)b_pos(k, p);
        }
    }

    auto issue = [&](uint8_t *as, uint8_t *bs, int32_t k0) {
        const u4w ar = drsrc(a_base + k0, a_valid - k0);
        const u4w br = drsrc(b_base + (int64_t)k0 * b_step, b_valid - (int64_t)k0 * b_step);
        const uint32_t la = lds_addr(as) + wave * 1024, lb = lds_addr(bs) + wave * 1024;
#pragma unroll
        for (int i = 0; i < LOADS_A; i++) dma16(ar, la + i * 4096, off_a[i]);
#pragma unroll
        for (int i = 0; i < LOADS_B; i++) dma16(br, lb + i * 4096, off_b[i]);
    };

    v4i acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = (v4i){0, 0, 0, 0};
    int32_t rs[8], cs[8];   // this lane's byte sums of its A rows / B columns (k-group g4)
#pragma unroll
    for (int i = 0; i < 8; i++) { rs[i] = 0; cs[i] = 0; }

    // One stage: B fragments for the wave's 8 column blocks stay in registers, A fragments stream one ahead.
    auto compute = [&](const uint8_t *as, const uint8_t *bs) {
        v4i bf[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int nl = wn * 128 + 16 * j;   // first column of the block
            uint32_t w[4];
            if constexpr (TRANS_B) {
                const int r = nl + i16;
                v4i v = *reinterpret_cast<const v4i *>(bs + r * 64 + 16 * a_pos(r, g4));
                w[0] = (uint32_t)v.x; w[1] = (uint32_t)v.y; w[2] = (uint32_t)v.z; w[3] = (uint32_t)v.w;
            } else {
                const int c = nl >> 4;   // 16-byte chunk of the block's columns
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int k = 16 * g4 + 8 * h + (i16 >> 1);
                    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                        OG_LDS2(bs + k * DBN + 16 * b_pos(k, c) + 8 * (i16 & 1)));
                    w[2 * h] = (uint32_t)v.x;
                    w[2 * h + 1] = (uint32_t)v.y;
                }
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                w[q] ^= flip_b;
                if (SUM_B && wm == 0) cs[j] = dot4(w[q], 0x01010101u, cs[j]);
            }
            bf[j] = (v4i){(int32_t)w[0], (int32_t)w[1], (int32_t)w[2], (int32_t)w[3]};
        }
        auto read_a = [&](int i) {
            const int r = wm * 128 + 16 * i + i16;
            const v4i v = *reinterpret_cast<const v4i *>(as + r * 64 + 16 * a_pos(r, g4));
            return (v4i){v.x ^ (int32_t)flip_a, v.y ^ (int32_t)flip_a, v.z ^ (int32_t)flip_a, v.w ^ (int32_t)flip_a};
        };
        v4i a_cur = read_a(0);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const v4i a_next = i + 1 < 8 ? read_a(i + 1) : a_cur;
            if (SUM_A && wn == 0)
                rs[i] = dot4((uint32_t)a_cur.w, 0x01010101u, dot4((uint32_t)a_cur.z, 0x01010101u,
                             dot4((uint32_t)a_cur.y, 0x01010101u, dot4((uint32_t)a_cur.x, 0x01010101u, rs[i]))));
#pragma unroll
            for (int j = 0; j < 8; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_cur, bf[j], acc[i][j], 0, 0, 0);
            a_cur = a_next;
        }
    };

    // The last stage of a K that is not a multiple of 64 holds bytes past K (the rest of a row, or rows past K read
    // as zeros). Each is overwritten with the byte the signed-domain flip turns into 0 (0x80 for an unsigned operand,
    // 0 for a signed one), so they add nothing to the products or the byte sums. valid = K - k0 in 1 .. 63.
    const uint32_t pad_a = flip_a & 0xFFu, pad_b = flip_b & 0xFFu;
    // Keeps the first n bytes of a 16-byte chunk and fills the rest with `pad` (n clamped to 0..16).
    auto keep_fill = [](uint4 v, int32_t n, uint32_t pad) {
        auto one = [&](uint32_t w, int32_t m) {
            const uint32_t keep = m >= 4 ? 0xFFFFFFFFu : (m <= 0 ? 0u : ((1u << (8 * m)) - 1u));
            return (w & keep) | (pad * 0x01010101u & ~keep);
        };
        return make_uint4(one(v.x, n), one(v.y, n - 4), one(v.z, n - 8), one(v.w, n - 12));
    };
    auto patch_tail = [&](uint8_t *as, uint8_t *bs, int32_t valid) {
        {   // A: thread tid owns row tid (64 bytes)
            const int r = tid;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint4 *p = reinterpret_cast<uint4 *>(&as[r * 64 + 16 * a_pos(r, q)]);
                *p = keep_fill(*p, valid - 16 * q, pad_a);
            }
        }
        if constexpr (TRANS_B) {
            const int r = tid;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint4 *p = reinterpret_cast<uint4 *>(&bs[r * 64 + 16 * a_pos(r, q)]);
                *p = keep_fill(*p, valid - 16 * q, pad_b);
            }
        } else {   // B: rows k >= valid, 256 bytes each; thread tid fills 64 bytes
            const int k = tid >> 2, part = tid & 3;
            if (k >= valid) {
                const uint32_t w = pad_b * 0x01010101u;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<uint4 *>(&bs[k * DBN + 64 * part + 16 * e]) = make_uint4(w, w, w, w);
            }
        }
        wait_lgkm_barrier();
    };

    const int32_t nk = (K + DBK - 1) / DBK;
    const bool ragged = (K % DBK) != 0;
    // Prologue: stages 0 .. NS - 2 in flight.
    issue(A0, B0, 0);
    if (NS > 2) issue(A1, B1, DBK);
    if (NS > 3) issue(A2, B2, 2 * DBK);

    // Stage u of a round of NS: wait for its loads (NS - 2 later stages may still be in flight), barrier (everyone's
    // loads landed and everyone is done reading the buffer about to be refilled), refill that buffer NS - 1 stages
    // ahead (past K the loads return zeros), patch a ragged last stage, compute.
#define OG_STAGE(U, AS, BS, ANEXT, BNEXT)                                                      \
    if (kt + (U) < nk) {                                                                       \
        wait_vm_barrier<LOADS * (NS - 2)>();                                                   \
        issue(ANEXT, BNEXT, (kt + (U) + NS - 1) * DBK);                                        \
        if (ragged && kt + (U) == nk - 1) patch_tail(AS, BS, K - (kt + (U)) * DBK);          \
        compute(AS, BS);                                                                       \
    }
    for (int32_t kt = 0; kt < nk; kt += NS) {
        if constexpr (NS == 4) {
            OG_STAGE(0, A0, B0, A3, B3)
            OG_STAGE(1, A1, B1, A0, B0)
            OG_STAGE(2, A2, B2, A1, B1)
            OG_STAGE(3, A3, B3, A2, B2)
        } else if constexpr (NS == 3) {
            OG_STAGE(0, A0, B0, A2, B2)
            OG_STAGE(1, A1, B1, A0, B0)
            OG_STAGE(2, A2, B2, A1, B1)
        } else {
            OG_STAGE(0, A0, B0, A1, B1)
            OG_STAGE(1, A1, B1, A0, B0)
        }
    }
#undef OG_STAGE
    wait_vm<0>();

    // Byte sums: the four k-groups of a row / column sit in lanes l, l + 16, l + 32, l + 48.
    if (SUM_A && wn == 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int32_t v = rs[i] + __shfl_xor(rs[i], 16);
            v += __shfl_xor(v, 32);
            if (g4 == 0) RowSum[wm * 128 + 16 * i + i16] = v;
        }
    }
    if (SUM_B && wm == 0) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int32_t v = cs[j] + __shfl_xor(cs[j], 16);
            v += __shfl_xor(v, 32);
            if (g4 == 0) ColSum[wn * 128 + 16 * j + i16] = v;
        }
    }
    if (SUM_B) RowZ[tid] = a_signed ? sext8(za_raw) : (int32_t)za_raw - 128;
    if (SUM_A) ColW[tid] = b_signed ? sext8(zb_raw) : (int32_t)zb_raw - 128;
    ColIB[tid] = my_ib;
    ColSc[tid] = my_sc;
    ColFb[tid] = my_fb;
    wait_lgkm_barrier();

    // Store. With z' = zero of A's row, w' = zero of B's column, s_m / t_n the byte sums of the row / column:
    //     C = acc - w' s_m - z' (t_n - K w')   (+ int bias; float: fl(fl(float(C)) * scale) (+ float bias))
    // MFMA 16 x 16 output layout: lane l holds rows 4 (l / 16) + r, column l % 16 of each block.
    const uint32_t Ku = (uint32_t)K;
    uint32_t wz[8], ct[8], ib[8];
    float sc[8], fb[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int nl = wn * 128 + 16 * j + i16;
        wz[j] = SUM_A ? (uint32_t)ColW[nl] : 0u;
        ct[j] = SUM_B ? (uint32_t)ColSum[nl] - Ku * wz[j] : 0u;
        ib[j] = (uint32_t)ColIB[nl];
        sc[j] = ColSc[nl];
        fb[j] = ColFb[nl];
    }
    int32_t *const Cb = static_cast<int32_t *>(g.C) + batch * g.strideC;   // int32 and float32 results alike
    const int32_t ncol0 = n0 + wn * 128 + i16;
    const int32_t M = g.M, N = g.N;
    auto store_all = [&](auto float_tag, bool has_fb) {
        constexpr bool F = decltype(float_tag)::value;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int ml = wm * 128 + 16 * i + 4 * g4;
            const v4i ssv = SUM_A ? *reinterpret_cast<const v4i *>(&RowSum[ml]) : (v4i){0, 0, 0, 0};
            const v4i zzv = SUM_B ? *reinterpret_cast<const v4i *>(&RowZ[ml]) : (v4i){0, 0, 0, 0};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int32_t m = m0 + ml + r;
                if (m >= M) continue;
                int32_t *const row = Cb + m * N;   // batch * M * N < 2^31 (checked at the boundary)
                const uint32_t ss = (uint32_t)ssv[r], zz = (uint32_t)zzv[r];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int32_t n = ncol0 + 16 * j;
                    if (n >= N) continue;
                    const uint32_t v = (uint32_t)acc[i][j][r] - wz[j] * ss - zz * ct[j] + ib[j];
                    if constexpr (F) {
                        float f = __fmul_rn((float)(int32_t)v, sc[j]);
                        if (has_fb) f = __fadd_rn(f, fb[j]);
                        row[n] = __float_as_int(f);
                    } else {
                        row[n] = (int32_t)v;
                    }
                }
            }
        }
    };
    if (epi & OG_EPI_FLOAT) {
        if (epi & OG_EPI_FLOAT_BIAS) store_all(std::true_type{}, true);
        else store_all(std::true_type{}, false);
    } else {
        store_all(std::false_type{}, false);
    }
}

// The direct kernel's conditions: 16-byte aligned rows for both operands, each batch's operands under 2^31 bytes.
bool direct_ok(const GemmArgs &g)
{
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    const int64_t lim = 0x7FFFFFFFll;
    if (((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 15) != 0) return false;
    if (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 15) != 0) return false;
    if ((int64_t)g.M * g.lda > lim) return false;
    if ((int64_t)(trans_b ? g.N : g.K) * g.ldb > lim) return false;
    return true;
}

hipError_t launch_gemm_direct(const GemmArgs &g, hipStream_t s, const char **kernel)
{
    const int32_t tn = (g.N + DBN - 1) / DBN, tm = (g.M + DBM - 1) / DBM;
    const int64_t blocks = (int64_t)tn * tm * g.batch;
    *kernel = "mfma-i8-direct256x256x64";
    if (blocks <= 0) return hipSuccess;
    const bool trans_b = g.flags & OG_GEMM_TRANSPOSE_B;
    const bool a_signed = g.flags & OG_GEMM_A_INT8, b_signed = g.flags & OG_GEMM_B_INT8;
    const bool sum_a = (g.flags & OG_GEMM_ZB) || !b_signed;
    const bool sum_b = (g.flags & OG_GEMM_ZA) || !a_signed;
    dim3 grid((uint32_t)blocks), block(DTHREADS);
#define OG_D(T, SA, SB) hipLaunchKernelGGL((k_gemm_direct<4, T, SA, SB>), grid, block, 0, s, g, tn, tm)
    if (trans_b) {
        if (sum_a && sum_b) OG_D(true, true, true);
        else if (sum_a) OG_D(true, true, false);
        else if (sum_b) OG_D(true, false, true);
        else OG_D(true, false, false);
    } else {
        if (sum_a && sum_b) OG_D(false, true, true);
        else if (sum_a) OG_D(false, true, false);
        else if (sum_b) OG_D(false, false, true);
        else OG_D(false, false, false);
    }
#undef OG_D
    return hipGetLastError();
}

}  // namespace og
