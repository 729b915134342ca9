// The large-product int8 MFMA kernel: operands go from HBM straight into a ring of LDS stages (buffer_load ... lds,
// no staging registers), and B stored K x N is read in its own layout with the gfx950 transpose read
// ds_read_b64_tr_b8, so no VALU transposition is needed.
//
//  - Tile 256 x 256 per workgroup (large products) or 128 x 128 (medium ones), 64 deep per stage, a ring of 5 stages
//    filling the 160 KB of LDS (half of it at 128, two workgroups a CU). K must be a multiple of 64 (other products
//    take the register-staged kernel). 8 waves, two a SIMD, so while one waits (at the stage barrier, for a fragment
//    read) the other keeps the matrix core busy: at 256, 4 x 2 waves of 64 x 128 (2 x 4 blocks of
//    v_mfma_i32_32x32x32_i8; 128 accumulator registers a wave leave room for both in the SIMD's register file), at
//    128, 2 x 4 waves of 64 x 32 (2 x 1 blocks). A 256 tile that needs both operands' byte sums runs on 4 waves
//    (2 x 2 of 128 x 128, one a SIMD, accumulators in AGPRs): on 8 its registers would spill.
//  - The 32 x 32 x 32 MFMA (32 cycles) does the work of two 16 x 16 x 64 ones with the same fragment reads, and leaves
//    room for about seven other instructions: the DMA of a later stage (2 instructions a load), the fragment reads,
//    one flip per unsigned fragment, and the operands' byte sums (v_sad_u8, which issues beside an MFMA where v_dot4
//    does not).
//  - Operands stay as stored in LDS; each MFMA fragment of an unsigned operand is moved to the signed domain
//    (s = u ^ 0x80) after it is read, and the zero points are applied at the store from the byte sums:
//        sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w'   (mod 2^32; Int8GemmDot.hlsl:1-11 rearranges the same)
//  - LDS layouts (16-byte chunks):
//      A (and B stored N x K): row r of 64 bytes, chunk q at position q ^ ((r >> 2) & 3);
//      B stored K x N: row k of 256 bytes, chunk c at position c ^ fB(k), fB(k) = 2 (k & 7) | ((k >> 4) & 1)
//      (128-byte rows at the 128 tile: c ^ (k & 7)).
//    A buffer load writes 64 lanes x 16 bytes to consecutive LDS, so each lane loads the global chunk that belongs in
//    its slot.
//  - An A fragment (lane l: row l % 32, k 16 (l / 32) .. + 15 of a 32-deep half stage) is one ds_read_b128. A B
//    fragment (lane l: column l % 32, the same 16 k) is two ds_read_b64_tr_b8: within each 16-lane group, lane i < 8
//    receives byte i of the 8-byte segments the even lanes address and lane 8 + i byte i of the odd lanes' segments,
//    so even lanes address rows k..k+7 at columns n..n+7 and odd lanes the same rows at columns n+8..n+15. A and B
//    give byte b of a lane the same k, which is all the MFMA's sum needs.
#pragma once

#include <type_traits>

#include "og_internal.hpp"

namespace og {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u4w __attribute__((ext_vector_type(4)));
#define OG_LDS2(p) ((__attribute__((address_space(3))) v2i *)(p))

namespace {

constexpr int DBK = 64;
constexpr int NS = 5;                                   // stages in the ring

// The shape of a BT x BT tile (BT = 256 or 128) on WAVES waves (4: one a SIMD; 8: two a SIMD): WGM x WGN waves of
// WTM x WTN (4 x 2 at 256 on 8 waves, 2 x 4 at 128 on 8 waves, else 2 x 2), each FM x FN blocks of 32 x 32; a stage of
// 64 k in NB blocks of 2 row blocks x FN column blocks (HB blocks per 32-deep half).
template <int BT, int WAVES>
struct DCfg {
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int A_STAGE = BT * DBK, B_STAGE = DBK * BT, STAGE = A_STAGE + B_STAGE;   // bytes
    static constexpr int LOADS_A = A_STAGE / 16 / THREADS, LOADS_B = B_STAGE / 16 / THREADS;   // 16-byte loads a thread
    static constexpr int LOADS = LOADS_A + LOADS_B;
    static constexpr int WGN = (WAVES == 8 && BT == 128) ? 4 : 2, WGM = WAVES / WGN;
    static constexpr int WTM = BT / WGM, WTN = BT / WGN, FM = WTM / 32, FN = WTN / 32;
    static constexpr int HB = FM / 2, NB = 2 * HB, BPB = FN / HB;
    static_assert(BT == 256 || BT == 128, "tile");
    static_assert(WAVES == 4 || WAVES == 8, "waves");
    static_assert(FM >= 2 && FN >= 1 && LOADS_A >= 1 && LOADS_B >= 1, "shape");
};

// Buffer resource words for `bytes` bytes at `base` (raw buffer: no stride, no swizzle; reads past the range
// return zero).
__device__ __forceinline__ u4w drsrc(const uint8_t *base, int32_t bytes)
{
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return (u4w){(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, (uint32_t)max(bytes, 0), 0x00020000u};
}

// LDS byte address of a __shared__ location.
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// One LDS DMA: lane l's 16 bytes at rsrc + voff land at LDS address base + OFF + 16 l. Issued from inline assembly
// so that the compiler neither reorders LDS accesses across it nor adds waits of its own for it: the stages wait for
// exactly the loads they need (vmcnt counts these loads in issue order). The address is formed outside the
// assembly (an s_add there would change SCC behind the compiler's back) and moved into M0 with s_mov, which leaves
// SCC alone. M0 is written without being saved: the compiler reserves M0 and these kernels give it nothing to hold
// across a DMA (no indexed register access, s_sendmsg, GWS or LDS-DMA intrinsics; checked in the disassembly of
// every kernel that includes this file: M0 is written only here). The resource words are uniform; readfirstlane states
// so, which keeps them in scalar registers where the compiler's uniformity analysis alone would not (the epilogue's
// store loop, inlined into the 4-wave kernels, otherwise leaves it unsure).
template <int OFF>
__device__ __forceinline__ void dma16(u4w rsrc, uint32_t base, uint32_t voff)
{
    const u4w r = {(uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc.x),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc.y),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc.z),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc.w)};
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(base + (uint32_t)OFF),
                 "v"(voff), "s"(r) : "memory");
}

// LDS serves 256 bytes a cycle: a 16-byte fragment read takes 16 lanes at a time (rows r .. r + 15 of A: the
// position must differ across r & 3 and (r >> 2) & 3), a transpose read of 8 bytes 32 lanes (8 rows of B x two
// neighbouring chunks c and c ^ 1: at 256-byte rows the 16 positions must all differ, so the rows take even offsets
// and the chunk pair fills the odd ones). rocprofv3 counts no bank conflicts with these (SQ_LDS_BANK_CONFLICT = 0).
__device__ __forceinline__ int a_pos(int r, int q) { return q ^ ((r >> 2) & 3); }
template <int BT>
__device__ __forceinline__ int b_pos(int k, int c)
{
    if constexpr (BT == 256) return c ^ ((2 * (k & 7)) | ((k >> 4) & 1));
    else return c ^ (k & 7);   // 128-byte rows: the row's parity picks the bank half, k & 7 the rest
}

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

// Both: at most N DMA loads outstanding and no LDS access, then meet the other waves.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm_barrier()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

template <bool FLIP>
__device__ __forceinline__ v4i to_signed(v4i v)
{
    if constexpr (FLIP) return v ^ (int32_t)0x80808080;
    else return v;
}

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }

// Sum of the 16 bytes of a fragment read as unsigned, added to acc (v_sad_u8 against zero). Applied to biased bytes
// (signed-domain value + 128, i.e. value ^ 0x80): the signed sum is the biased sum minus 128 per byte.
__device__ __forceinline__ uint32_t sad16(v4i v, uint32_t acc)
{
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.x, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.y, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.z, 0u, acc);
    return __builtin_amdgcn_sad_u8((uint32_t)v.w, 0u, acc);
}

// a * b mod 2^32 for the epilogue's corrections (a zero point times a byte sum): with SMALL both are under 2^23 in
// magnitude, so the 24-bit multiply (full rate) gives the exact product; otherwise the 32-bit one (quarter rate).
template <bool SMALL>
__device__ __forceinline__ uint32_t zmul(uint32_t a, uint32_t b)
{
    if constexpr (SMALL) return (uint32_t)__mul24((int32_t)a, (int32_t)b);
    else return a * b;
}

// Calls f(integral_constant<I>) for I = B .. E - 1.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

}  // namespace

// FLIP_A / FLIP_B: the operand is unsigned (moved to the signed domain fragment by fragment). SUM_A / SUM_B: the row
// sums of A / column sums of B are needed (the other operand's zero point in the signed domain can be non-zero).
// PP: the 256 tile on 8 waves in ping-pong order (below) instead of the block-interleaved stage loop.
template <int BT, bool TRANS_B, bool SUM_A, bool SUM_B, bool FLIP_A, bool FLIP_B, int WAVES = 4, bool PP = false>
// ksplit > 1: the product is cut along K into slices of kslice bytes (a multiple of 64); g.batch counts batch entries
// times slices, and slice kc of batch entry b computes the int32 sums of its k range with the zero points applied
// (every correction term is linear in the slice) into batch entry b * ksplit + kc of C, which is then a dense int32
// partial buffer (the caller adds the slices and applies the epilogue). ksplit = 1: the whole product.
__global__ __launch_bounds__(64 * WAVES) void k_gemm_direct(GemmArgs g, int32_t tiles_n, int32_t tiles_m, int32_t ksplit,
                                                          int32_t kslice)
{
    using D = DCfg<BT, WAVES>;
    constexpr int DBM = BT, DBN = BT, A_STAGE = D::A_STAGE, STAGE = D::STAGE, LOADS_A = D::LOADS_A;
    constexpr int LOADS_B = D::LOADS_B, LOADS = D::LOADS, WTM = D::WTM, WTN = D::WTN, FM = D::FM, FN = D::FN;
    constexpr int HB = D::HB, NB = D::NB, BPB = D::BPB, WGM = D::WGM, WGN = D::WGN, THREADS = D::THREADS;
    // The ring of NS stages, A (BT x 64) then B (64 x BT) each: all 160 KB of LDS at BT = 256, half at 128 (two
    // workgroups a CU). After the loop its start holds the epilogue's per-row and per-column arrays.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i32 = lane & 31, h2 = lane >> 5;   // MFMA roles: row / column within a 32-block, k half
    const int i16 = lane & 15, g4 = lane >> 4;   // transpose-read roles
    const int wm = wave / WGN, wn = wave % WGN;

    // Tile order: the hardware deals workgroups round-robin to the 8 XCDs; remap so that each XCD gets one contiguous
    // run of tiles, walked in groups of 8 row tiles, and the A and B tiles the run reuses stay in its L2.
    const int64_t tiles = (int64_t)tiles_n * tiles_m;
    const int64_t nblocks = tiles * g.batch;
    int64_t bid = blockIdx.x;
    if ((nblocks & 7) == 0) bid = (bid & 7) * (nblocks >> 3) + (bid >> 3);
    const int32_t bsplit = (int32_t)(bid / tiles);           // batch entry of C
    const int32_t kc = bsplit % ksplit, batch = bsplit / ksplit;   // k slice; batch entry of A and B
    const int32_t K0 = kc * kslice;
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
    const int32_t lda = g.lda, ldb = g.ldb, K = max(0, min(kslice, g.K - K0));   // an empty slice adds zero
    constexpr bool a_signed = !FLIP_A, b_signed = !FLIP_B;

    // The epilogue's per-row and per-column parameters, fetched now so that their latency hides behind the loop:
    // thread t < BT holds row m0 + t's zero point and column n0 + t's zero point, int bias, scale and float bias.
    const uint32_t epi = g.epi;
    const int32_t my_m = min(m0 + tid, g.M - 1), my_n = min(n0 + tid, g.N - 1);
    // Raw zero-point bytes (0 when absent); moved to the signed domain after the loop, so nothing waits for them here.
    const uint32_t za_raw = (SUM_B && g.ZA) ? g.ZA[(g.flags & OG_GEMM_ZA_PER_ROW) ? my_m : 0] : 0u;
    const uint32_t zb_raw = (SUM_A && g.ZB) ? g.ZB[(g.flags & OG_GEMM_ZB_PER_COL) ? my_n : 0] : 0u;
    const int32_t my_ib = (epi & OG_EPI_INT_BIAS) ? g.bias[my_n] : 0;
    const float my_sc = (epi & (OG_EPI_FLOAT | EPI_REQUANT)) ? column_scale(g, my_n) : 0.0f;
    const float my_fb = (epi & OG_EPI_FLOAT_BIAS) ? g.fbias[my_n] : 0.0f;

    // This tile's operand ranges (under 2^31 bytes, as the launcher checks): loads past the last valid byte return
    // zeros. With K = 0 the operands may be absent and nothing is read (the prologue still issues its loads, over
    // empty ranges).
    const uint8_t *a_base = g.A + batch * g.strideA + (int64_t)m0 * lda + K0;
    const int32_t a_valid = K > 0 ? (min(g.M - m0, DBM) - 1) * lda + K : 0;
    const uint8_t *b_base;
    int32_t b_valid, b_step;
    if constexpr (TRANS_B) {
        b_base = g.B + batch * g.strideB + (int64_t)n0 * ldb + K0;
        b_valid = K > 0 ? (min(g.N - n0, DBN) - 1) * ldb + K : 0;
        b_step = 1;
    } else {
        b_base = g.B + batch * g.strideB + n0 + (int64_t)K0 * ldb;
        b_valid = K > 0 ? (K - 1) * ldb + ((min(g.N - n0, DBN) + 3) & ~3) : 0;   // whole dwords (b_dwords_ok)
        b_step = ldb;
    }

    // Per-thread global offsets of the chunks that land in this thread's LDS slots (the same at every stage): load i
    // of a wave fills 1 KB at i * WAVES KB + wave * 1 KB of the operand's tile.
    uint32_t off_a[LOADS_A], off_b[LOADS_B];
#pragma unroll
    for (int i = 0; i < LOADS_A; i++) {
        const int s = (i * WAVES + wave) * 64 + lane, r = s >> 2, p = s & 3;
        off_a[i] = (uint32_t)r * (uint32_t)lda + 16u * (uint32_t)a_pos(r, p);
    }
#pragma unroll
    for (int i = 0; i < LOADS_B; i++) {
        const int s = (i * WAVES + wave) * 64 + lane;
        if constexpr (TRANS_B) {
            const int r = s >> 2, p = s & 3;
            off_b[i] = (uint32_t)r * (uint32_t)ldb + 16u * (uint32_t)a_pos(r, p);
        } else {
            const int k = s / (DBN / 16), p = s % (DBN / 16);
            off_b[i] = (uint32_t)k * (uint32_t)ldb + 16u * (uint32_t)b_pos<BT>(k, p);
        }
    }
    const uint32_t wave_lds = lds_addr(smem) + (uint32_t)wave * 1024u;

    // The DMA of the stage at depth k0 into ring buffer U: load I < LOADS_A is A's, the rest B's. A k0 past K (the loads
    // beyond the last stage) is clamped to K, which keeps the offsets in range; those loads are never used.
    struct StageRsrc {
        u4w a, b;
    };
    auto stage_rsrc = [&](int32_t k0) {
        k0 = min(k0, K);
        return StageRsrc{drsrc(a_base + k0, a_valid - k0), drsrc(b_base + k0 * b_step, b_valid - k0 * b_step)};
    };
    auto dma = [&](auto u_tag, auto i_tag, const StageRsrc &rr) {
        constexpr int U = decltype(u_tag)::value, I = decltype(i_tag)::value;
        if constexpr (I < LOADS_A) dma16<U * STAGE + I * WAVES * 1024>(rr.a, wave_lds, off_a[I]);
        else dma16<U * STAGE + A_STAGE + (I - LOADS_A) * WAVES * 1024>(rr.b, wave_lds, off_b[I - LOADS_A]);
    };

    // Fragments as stored (unsigned operands not yet flipped) from ring buffer u. A: row block i (32 rows) at k half
    // ks; lane l holds row 32 i + l % 32, k 32 ks + 16 (l / 32) .. + 15: one ds_read_b128.
    auto read_a = [&](int u, int i, int ks) {
        const int r = wm * WTM + 32 * i + i32;
        return *reinterpret_cast<const v4i *>(smem + u * STAGE + r * 64 + 16 * a_pos(r, 2 * ks + h2));
    };
    // B: column block j (32 columns) at k half ks; lane l holds column 32 j + l % 32 and the same 16 k as A.
    auto read_b = [&](int u, int j, int ks) -> v4i {
        const uint8_t *bs = smem + u * STAGE + A_STAGE;
        if constexpr (TRANS_B) {
            const int r = wn * WTN + 32 * j + i32;
            return *reinterpret_cast<const v4i *>(bs + r * 64 + 16 * a_pos(r, 2 * ks + h2));
        } else {
            // Each 16-lane group g transposes 16 columns (16 (g & 1) .. + 15 of the block) x 8 rows per read; groups
            // 2 and 3 take the second 16 k.
            const int c = (wn * WTN + 32 * j + 16 * (g4 & 1)) >> 4;   // 16-byte chunk of the group's columns
            v2i h[2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int k = 32 * ks + 16 * (g4 >> 1) + 8 * hh + (i16 >> 1);
                h[hh] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(OG_LDS2(bs + k * DBN + 16 * b_pos<BT>(k, c) + 8 * (i16 & 1)));
            }
            return (v4i){h[0].x, h[0].y, h[1].x, h[1].y};
        }
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    // This lane's biased byte sums (its k half, 16 bytes per fragment) of the wave's A row blocks / B column blocks.
    // Biased bytes: an unsigned operand's bytes as stored, a signed one's with the top bit flipped.
    uint32_t rs[FM], cs[FN];
#pragma unroll
    for (int i = 0; i < FM; i++) rs[i] = 0;
#pragma unroll
    for (int j = 0; j < FN; j++) cs[j] = 0;
    const int32_t nk = K / DBK;   // K is a multiple of DBK here

    if constexpr (PP) {
        // Ping-pong: waves 0-3 (group 0, rows 0-127 of the tile) and 4-7 (group 1, rows 128-255) put one wave of each
        // group on every SIMD, and the two groups take turns: while one group's waves issue a stage's 16 MFMAs (512
        // cycles of the SIMD's matrix core), the other group's read their fragments of the stage they multiply next,
        // move them to the signed domain, form their byte sums and issue their share of later stages' DMA. A barrier
        // ends each such phase, two a stage, so the matrix core of every SIMD always has one wave feeding it.
        //   phase 2t:     group 0 multiplies stage t;  group 1 issues half of an A pair and reads stage t;
        //   phase 2t + 1: group 1 multiplies stage t;  group 0 issues B of stage t + 4 and reads stage t + 1.
        // LDS: A in 3 pair slots of 256 rows x 128 bytes (two stages: each row a whole 128-byte line, where a 64-byte
        // stage would fetch half lines), then B in 4 stage slots of 64 x 256 bytes. Pair q (stages 2q, 2q + 1) goes
        // into slot q % 3 in halves of 128 rows, at phases 4q - 8 and 4q - 6, after both groups are done with pair
        // q - 3 (read last in phase 4q - 10); B of stage t + 4 goes into slot t % 4 in phase 2t + 1, after group 1 read
        // B of stage t in phase 2t. Stage t + 1 must have landed before phase 2t + 1, where group 0 reads it: at the
        // end of phase 2t each group waits for its own loads of it, then meets the other.
        // A pair slot: row r's 16-byte chunk c (k 16 c .. + 15 of the pair) at position c ^ ((r >> 1) & 7): the rows
        // of one parity fill one 128-byte half of the 256 bytes LDS serves a cycle, so a fragment read (16 rows, one
        // chunk) is conflict-free, and a DMA instruction writes 8 whole rows.
        static_assert(BT == 256 && WAVES == 8 && FM == 2 && FN == 4 && WGN == 2 && NS * STAGE == 163840, "the layout");
        constexpr int GL = 4;   // DMA loads of a group's thread a phase (16 KB over 256 threads)
        constexpr int A_PAIR = 2 * A_STAGE, B_OFF = 3 * A_PAIR, B_SLOT = D::B_STAGE;
        static_assert(B_OFF + 4 * B_SLOT == NS * STAGE && A_STAGE / 16 / 256 == GL && B_SLOT / 16 / 256 == GL, "slots");
        auto pp = [&](auto wm_tag, auto wn_tag) {
            constexpr int WM = decltype(wm_tag)::value, WN = decltype(wn_tag)::value, GRP = WM >> 1;
            // Byte sums: row block WN of this wave's rows, column block WM of its columns (one wave each).
            constexpr int SAR = SUM_A ? WN : -1, SBR = SUM_B ? WM : -1;
            const int lw = wave & 3;
            const uint32_t lds_l = lds_addr(smem) + (uint32_t)lw * 1024u;
            // This thread's global chunk offsets. Group 1, A: load i of local wave lw fills 1 KB at (4 i + lw) KB of
            // a half pair (rows 8 (4 i + lw) + lane / 8, position lane % 8). Group 0, B: 1 KB at (4 i + lw) KB of a
            // stage.
            uint32_t off_g[GL];
#pragma unroll
            for (int i = 0; i < GL; i++) {
                const int s = (i * 4 + lw) * 64 + lane;
                if constexpr (GRP == 1) {
                    const int r = s >> 3, q = (s & 7) ^ ((r >> 1) & 7);
                    off_g[i] = (uint32_t)r * (uint32_t)lda + 16u * (uint32_t)q;
                } else if constexpr (TRANS_B) {
                    const int r = s >> 2, q = s & 3;
                    off_g[i] = (uint32_t)r * (uint32_t)ldb + 16u * (uint32_t)a_pos(r, q);
                } else {
                    const int k = s / (DBN / 16), q = s % (DBN / 16);
                    off_g[i] = (uint32_t)k * (uint32_t)ldb + 16u * (uint32_t)b_pos<BT>(k, q);
                }
            }
            // Half h of A pair q (rows 128 h .. + 127, k 128 q .. + 127) into its slot; B of stage st into slot U.
            auto issue_a = [&](int32_t q, auto h_tag) {
                constexpr int H = decltype(h_tag)::value;
                const int32_t k0 = min(128 * q, K), r0 = H * 128 * lda;
                const u4w ra = drsrc(a_base + r0 + k0, a_valid - r0 - k0);
                const uint32_t base = lds_l + (uint32_t)(q % 3) * (uint32_t)A_PAIR;
                static_for<0, GL>([&](auto i_tag) {
                    constexpr int I = decltype(i_tag)::value;
                    dma16<H * A_STAGE + I * 4096>(ra, base, off_g[I]);
                });
            };
            auto issue_b = [&](auto u_tag, int32_t st) {
                constexpr int U = decltype(u_tag)::value;
                const int32_t k0 = min(st * DBK, K);
                const u4w rb = drsrc(b_base + k0 * b_step, b_valid - k0 * b_step);
                static_for<0, GL>([&](auto i_tag) {
                    constexpr int I = decltype(i_tag)::value;
                    dma16<B_OFF + U * B_SLOT + I * 4096>(rb, lds_l, off_g[I]);
                });
            };
            // Fragment reads of stage t: A from pair slot (t / 2) % 3, its half t % 2 (lane l: row 32 i + l % 32 of
            // the wave's rows, chunk 4 (t % 2) + 2 ks + l / 32); B from slot t % 4 as before.
            auto read_a_pp = [&](uint32_t slot, int half, int i, int ks) {
                const int r = wm * WTM + 32 * i + i32, c = 4 * half + 2 * ks + h2;
                return *reinterpret_cast<const v4i *>(smem + slot + r * 128 + 16 * (c ^ ((r >> 1) & 7)));
            };
            auto read_b_pp = [&](int u, int j, int ks) -> v4i {
                const uint8_t *bs = smem + B_OFF + u * B_SLOT;
                if constexpr (TRANS_B) {
                    const int r = wn * WTN + 32 * j + i32;
                    return *reinterpret_cast<const v4i *>(bs + r * 64 + 16 * a_pos(r, 2 * ks + h2));
                } else {
                    const int c = (wn * WTN + 32 * j + 16 * (g4 & 1)) >> 4;
                    v2i h[2];
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const int k = 32 * ks + 16 * (g4 >> 1) + 8 * hh + (i16 >> 1);
                        h[hh] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(OG_LDS2(bs + k * DBN + 16 * b_pos<BT>(k, c) + 8 * (i16 & 1)));
                    }
                    return (v4i){h[0].x, h[0].y, h[1].x, h[1].y};
                }
            };
            // The fragments of the next stage this wave multiplies, in the signed domain: [k half][block].
            v4i af[2][2], bf[2][FN];
            auto fetch = [&](int32_t t, auto u_tag) {
                constexpr int U = decltype(u_tag)::value, H = U & 1;
                const uint32_t slot = (uint32_t)((t >> 1) % 3) * (uint32_t)A_PAIR;
                v4i ar[2][2], br[2][FN];
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
#pragma unroll
                    for (int i = 0; i < 2; i++) ar[ks][i] = read_a_pp(slot, H, i, ks);
#pragma unroll
                    for (int j = 0; j < FN; j++) br[ks][j] = read_b_pp(U, j, ks);
                }
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    if constexpr (SAR >= 0)
                        rs[SAR] = sad16(FLIP_A ? ar[ks][SAR] : (ar[ks][SAR] ^ (int32_t)0x80808080), rs[SAR]);
                    if constexpr (SBR >= 0)
                        cs[SBR] = sad16(FLIP_B ? br[ks][SBR] : (br[ks][SBR] ^ (int32_t)0x80808080), cs[SBR]);
#pragma unroll
                    for (int i = 0; i < 2; i++) af[ks][i] = to_signed<FLIP_A>(ar[ks][i]);
#pragma unroll
                    for (int j = 0; j < FN; j++) bf[ks][j] = to_signed<FLIP_B>(br[ks][j]);
                }
            };
            auto multiply = [&]() {
#pragma unroll
                for (int ks = 0; ks < 2; ks++)
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 0; j < FN; j++) acc[i][j] = mfma32(af[ks][i], bf[ks][j], acc[i][j]);
            };
            // Stage t (U = t % 4).
            auto stage = [&](auto u_tag, int32_t t) {
                constexpr int U = decltype(u_tag)::value, H = U & 1;
                // phase 2t
                if constexpr (GRP == 0) {
                    multiply();
                    __builtin_amdgcn_sched_barrier(0);
                    wait_vm_lgkm_barrier<2 * GL>();   // B of stage t + 1 landed (t + 2, t + 3 may be in flight)
                } else {
                    issue_a((t >> 1) + 2, std::integral_constant<int, H>{});
                    fetch(t, u_tag);
                    __builtin_amdgcn_sched_barrier(0);
                    // A of stage t + 1 landed: pair (t + 1) / 2, whose halves were issued at stages t - 3, t - 2 (t odd)
                    // or t - 4, t - 3 (t even).
                    wait_vm_lgkm_barrier<(H ? 2 : 3) * GL>();
                }
                __builtin_amdgcn_sched_barrier(0);
                // phase 2t + 1
                if constexpr (GRP == 1) {
                    multiply();
                } else {
                    issue_b(u_tag, t + 4);
                    if (t + 1 < nk) fetch(t + 1, std::integral_constant<int, (U + 1) % 4>{});   // (past the last: nothing)
                }
                __builtin_amdgcn_sched_barrier(0);
                wait_lgkm_barrier();
                __builtin_amdgcn_sched_barrier(0);
            };
            // Prologue: group 1 issues A pairs 0 and 1 (stages 0-3), group 0 B of stages 0-3; stage 0 landed (group 1:
            // pair 0 of its 16 loads; group 0: B of stage 0 of its 16); group 0 reads it.
            if constexpr (GRP == 1) {
                issue_a(0, std::integral_constant<int, 0>{});
                issue_a(0, std::integral_constant<int, 1>{});
                issue_a(1, std::integral_constant<int, 0>{});
                issue_a(1, std::integral_constant<int, 1>{});
                wait_vm_barrier<2 * GL>();
            } else {
                static_for<0, 4>([&](auto u_tag) { issue_b(u_tag, decltype(u_tag)::value); });
                wait_vm_barrier<3 * GL>();
                if (nk > 0) fetch(0, std::integral_constant<int, 0>{});   // (K = 0: no stage, no byte sums)
            }
            __builtin_amdgcn_sched_barrier(0);
            wait_lgkm_barrier();
            __builtin_amdgcn_sched_barrier(0);
            for (int32_t kt = 0; kt < nk; kt += 4) {
                static_for<0, 4>([&](auto u_tag) {
                    if (kt + decltype(u_tag)::value < nk) stage(u_tag, kt + decltype(u_tag)::value);
                });
            }
        };
        // One instantiation per wave role (wm, and wn when A's row sums are needed), uniform across each wave.
        static_for<0, 4>([&](auto wm_tag) {
            if (wm == decltype(wm_tag)::value) {
                if constexpr (SUM_A) {
                    static_for<0, 2>([&](auto wn_tag) {
                        if (wn == decltype(wn_tag)::value) pp(wm_tag, wn_tag);
                    });
                } else {
                    pp(wm_tag, std::integral_constant<int, 0>{});
                }
            }
        });
    } else {
    // How far ahead the DMA runs. With one block a k half (HB = 1) a stage's buffer is read only in its first block,
    // so once the waves meet in stage s (each having finished its LDS reads) the buffer of stage s itself can take stage
    // s + NS: every buffer of the ring holds a stage in flight. With more blocks a k half, the second half's first
    // blocks still read stage s's A, so the refill goes one stage later, into the buffer of stage s - 1.
    constexpr int AHEAD = HB == 1 ? NS : NS - 1;
    // Prologue: stages 0 .. AHEAD - 1 in flight; stage 0 landed, its first k half of B and the first block's A read.
    static_for<0, AHEAD>([&](auto u_tag) {
        const StageRsrc r = stage_rsrc(decltype(u_tag)::value * DBK);
        static_for<0, LOADS>([&](auto i_tag) { dma(u_tag, i_tag, r); });
    });
    wait_vm_barrier<LOADS * (AHEAD - 1)>();
    // B fragments in the signed domain, [k half][column block]; the current block's A fragments as stored and signed.
    v4i bf[2][FN], a_st[2], a_cur[2];
#pragma unroll
    for (int j = 0; j < FN; j++) bf[0][j] = to_signed<FLIP_B>(read_b(0, j, 0));
#pragma unroll
    for (int t = 0; t < 2; t++) {
        a_st[t] = read_a(0, t, 0);
        a_cur[t] = to_signed<FLIP_A>(a_st[t]);
    }

    // One stage s in ring buffer U, in NB blocks of 2F MFMAs: block b multiplies A row blocks 2 (b % HB), + 1 at k
    // half b / HB against the FN B column blocks. Block b reads the A fragments of block b + 1 (the last block: the
    // first of stage s + 1) and BPB B fragments: the first half's blocks this stage's second k half, the second half's
    // the next stage's first (whose registers are free once the first half is done). At the first block of the second
    // half the waves wait for stage s + 1 (this wave's loads landed, then everyone's) and meet: from then on nobody
    // reads the buffer DU, so the second half's blocks issue the loads of stage s + AHEAD into it. Stages
    // past the last still wait and read (their loads cover empty or unused ranges and what is read is not used), so
    // every stage is the same.
    // SAR / SBR: the row / column byte sums this wave forms: those of its row blocks i with i % WGN == SAR and of its
    // column blocks j with j % WGM == SBR (-1: none). So each row block's sums come from one wave of its row of waves
    // and each column block's from one wave of its column, spread evenly, and no wave repeats another's.
    auto run_stage = [&](auto u_tag, int32_t s, auto sa_tag, auto sb_tag) {
        constexpr int U = decltype(u_tag)::value, DU = (U + AHEAD) % NS, NU = (U + 1) % NS;
        constexpr int SAR = decltype(sa_tag)::value, SBR = decltype(sb_tag)::value;
        const StageRsrc rr = stage_rsrc((s + AHEAD) * DBK);
        static_for<0, NB>([&](auto b_tag) {
            constexpr int b = decltype(b_tag)::value, ks = b / HB, i0 = 2 * (b % HB);
            constexpr int rks = b < HB ? 1 : 0, rj = BPB * (b % HB), RU = b < HB ? U : NU;
            constexpr int nb = (b + 1) % NB, AU = b < NB - 1 ? U : NU;
            // At 256, the compiler's MFMA / LDS-read interleave for small products within the block (1-3.6% faster on
            // the 256 tile's products than its default order; the 128 tile measured no better with it, and strategy
            // 1, the single-wave one, does not compile here).
            if constexpr (BT == 256) __builtin_amdgcn_iglp_opt(0);
            constexpr int LPB = LOADS / HB;   // loads per second-half block
            if constexpr (b == HB) {
                wait_vm_lgkm_barrier<LOADS * (AHEAD - 2)>();   // stages s + 2 .. s + AHEAD - 1 may still be in flight
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (b >= HB) {
                static_for<0, LPB>([&](auto q_tag) {
                    dma(std::integral_constant<int, DU>{}, std::integral_constant<int, LPB * (b - HB) + decltype(q_tag)::value>{}, rr);
                });
            }
            v4i bn[BPB];
#pragma unroll
            for (int q = 0; q < BPB; q++) bn[q] = read_b(RU, rj + q, rks);
            v4i a_nx[2];
            a_nx[0] = read_a(AU, 2 * (nb % HB), nb / HB);
            a_nx[1] = read_a(AU, 2 * (nb % HB) + 1, nb / HB);
            static_for<0, 2>([&](auto t_tag) {
                constexpr int t = decltype(t_tag)::value;
                if constexpr (SAR >= 0 && (i0 + t) % WGN == SAR)
                    rs[i0 + t] = FLIP_A ? sad16(a_st[t], rs[i0 + t]) : sad16(a_cur[t] ^ (int32_t)0x80808080, rs[i0 + t]);
            });
            static_for<0, BPB>([&](auto q_tag) {
                constexpr int q = decltype(q_tag)::value;
                if constexpr (SBR >= 0 && (rj + q) % WGM == SBR)
                    cs[rj + q] = sad16(bf[ks][rj + q] ^ (int32_t)0x80808080, cs[rj + q]);
            });
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[i0 + t][j] = mfma32(a_cur[t], bf[ks][j], acc[i0 + t][j]);
#pragma unroll
            for (int q = 0; q < BPB; q++) bf[rks][rj + q] = to_signed<FLIP_B>(bn[q]);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                a_st[t] = a_nx[t];
                a_cur[t] = to_signed<FLIP_A>(a_nx[t]);
            }
            // At 128 the blocks stay in order and the compiler interleaves freely within one (with two waves a SIMD
            // the other wave fills what one wave's order leaves idle; a fixed MFMA / VALU interleave measured slower).
            // At 256 the interleave strategy above also schedules across blocks (0.2-2% faster than with the blocks
            // kept apart); only the stage wait above stays a scheduling boundary.
            if constexpr (BT != 256) __builtin_amdgcn_sched_barrier(0);
        });
    };
    static_assert(NS == 5, "the loop below is unrolled for 5 stages");
    auto main_loop = [&](auto sa_tag, auto sb_tag) {
        for (int32_t kt = 0; kt < nk; kt += NS) {
            static_for<0, NS>([&](auto u_tag) {
                if (kt + decltype(u_tag)::value < nk) run_stage(u_tag, kt + decltype(u_tag)::value, sa_tag, sb_tag);
            });
        }
    };
    // The loop is instantiated per wave role (wm, wn are uniform across a wave), so each wave carries only its own share
    // of the byte sums: no wave waits at the stage barrier for another's extra VALU work, and none is spent twice.
    auto with_roles = [&](auto sa_tag) {
        if constexpr (SUM_B) {
            static_for<0, D::WGM>([&](auto r_tag) {
                if (wm == decltype(r_tag)::value) main_loop(sa_tag, r_tag);
            });
        } else {
            main_loop(sa_tag, std::integral_constant<int, -1>{});
        }
    };
    if constexpr (SUM_A) {
        static_for<0, D::WGN>([&](auto r_tag) {
            if (wn == decltype(r_tag)::value) with_roles(r_tag);
        });
    } else {
        with_roles(std::integral_constant<int, -1>{});
    }
    }
    // Every DMA landed and every wave done with the stage buffers before the epilogue's arrays take their place.
    wait_vm<0>();
    wait_lgkm_barrier();
    int32_t *const RowSum = reinterpret_cast<int32_t *>(smem);
    int32_t *const RowZ = RowSum + DBM;
    int32_t *const ColSum = RowZ + DBM;
    int32_t *const ColW = ColSum + DBN;
    int32_t *const ColIB = ColW + DBN;
    float *const ColSc = reinterpret_cast<float *>(ColIB + DBN);
    float *const ColFb = ColSc + DBN;

    // Byte sums: the two k halves of a row / column sit in lanes l and l + 32. The biased sums cover 64 bytes per
    // stage; the signed sums are 128 less per byte (mod 2^32).
    const uint32_t bias_total = 128u * (uint32_t)DBK * (uint32_t)nk;
    if (SUM_A) {
#pragma unroll
        for (int i = 0; i < FM; i++) {
            if (i % WGN != wn) continue;   // another wave of this row of waves formed these
            const uint32_t v = rs[i] + (uint32_t)__shfl_xor((int32_t)rs[i], 32);
            if (h2 == 0) RowSum[wm * WTM + 32 * i + i32] = (int32_t)(v - bias_total);
        }
    }
    if (SUM_B) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            if (j % WGM != wm) continue;   // another wave of this column of waves formed these
            const uint32_t v = cs[j] + (uint32_t)__shfl_xor((int32_t)cs[j], 32);
            if (h2 == 0) ColSum[wn * WTN + 32 * j + i32] = (int32_t)(v - bias_total);
        }
    }
    if (tid < BT) {
        if (SUM_B) RowZ[tid] = a_signed ? sext8(za_raw) : (int32_t)za_raw - 128;
        if (SUM_A) ColW[tid] = b_signed ? sext8(zb_raw) : (int32_t)zb_raw - 128;
        ColIB[tid] = my_ib;
        ColSc[tid] = my_sc;
        ColFb[tid] = my_fb;
    }
    wait_lgkm_barrier();

    // Store. With z' = zero of A's row, w' = zero of B's column, s_m / t_n the byte sums of the row / column:
    //     C = acc - w' s_m - z' (t_n - K w')   (+ int bias; float: fl(fl(float(C)) * scale) (+ float bias))
    // MFMA 32 x 32 output layout: lane l holds column l % 32 and, in register r, row 8 (r / 4) + 4 (l / 32) + r % 4
    // of its block; one store writes two 128-byte row segments.
    const uint32_t Ku = (uint32_t)K;
    // Below 2^15 k a byte sum (and a column sum less K times a zero point) stays under 2^23 in magnitude, so the
    // correction products fit the full-rate 24-bit multiply exactly.
    const bool small_k = K < 32768;
    uint32_t wz[FN], ct[FN], ib[FN];
    float sc[FN], fb[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int nl = wn * WTN + 32 * j + i32;
        wz[j] = SUM_A ? (uint32_t)ColW[nl] : 0u;
        ct[j] = SUM_B ? (uint32_t)ColSum[nl] - Ku * wz[j] : 0u;
        ib[j] = (uint32_t)ColIB[nl];
        sc[j] = ColSc[nl];
        fb[j] = ColFb[nl];
    }
    // int32 and float32 results are 4-byte elements, requantized ones bytes; strideC counts elements either way.
    int32_t *const Cb = static_cast<int32_t *>(g.C) + bsplit * g.strideC;
    uint8_t *const Yb = static_cast<uint8_t *>(g.C) + bsplit * g.strideC;
    const int32_t ncol0 = n0 + wn * WTN + i32;
    const int32_t M = g.M, N = g.N, zp_y = g.zp_y;
    // The NaN-ignoring range of the float values this thread stores (for a ranged float product; 128 tile).
    float rmn = __int_as_float(0x7F800000), rmx = __int_as_float(0xFF800000);
    // MODE 0: int32 (+ bias); 1: float32, `opt` = float bias present; 2: requantized bytes, `opt` = uint8 output.
    // Inlined: as a call it would keep a 1,408-byte stack frame a lane in the 4-wave kernels.
    auto store_all = [&](auto mode_tag, bool opt) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode_tag)::value;
        if constexpr (BT == 128) {
            // Staged through LDS: one store instruction per thread then writes four neighbouring columns (16 bytes, or
            // 4 bytes of a requantized row) where the accumulator layout gives it one column per lane, so a tile takes
            // a quarter of the store instructions, whose issue rate bounds this epilogue. Needs N % 4 == 0 and an
            // aligned C.
            const bool staged = N % 4 == 0 && (MODE == 2 ? ((uintptr_t)Yb & 3) == 0 : ((uintptr_t)Cb & 15) == 0);
            if (staged) {
                // The raw sums, [row][column] with rows of LDT ints (the pad puts the two half-waves' writes of one
                // instruction on different banks), after the epilogue's arrays.
                constexpr int LDT = BT + 4, T_OFF = 4096;
                static_assert(T_OFF >= (2 * DBM + 5 * DBN) * 4 && T_OFF + BT * LDT * 4 <= NS * STAGE, "staging space");
                int32_t *const T = reinterpret_cast<int32_t *>(smem + T_OFF);
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
#pragma unroll
                            for (int j = 0; j < FN; j++)
                                T[(wm * WTM + 32 * i + 8 * q + 4 * h2 + r) * LDT + wn * WTN + 32 * j + i32] = acc[i][j][4 * q + r];
                wait_lgkm_barrier();
                // Thread t: columns 4 (t % 32) .. + 3 of the tile, rows t / 32 + (THREADS / 32) jj.
                const int c4 = 4 * (tid & 31), r0 = tid >> 5;
                uint32_t wz4[4], ct4[4], ib4[4];
                float sc4[4], fb4[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    wz4[e] = SUM_A ? (uint32_t)ColW[c4 + e] : 0u;
                    ct4[e] = SUM_B ? (uint32_t)ColSum[c4 + e] - Ku * wz4[e] : 0u;
                    ib4[e] = (uint32_t)ColIB[c4 + e];
                    sc4[e] = ColSc[c4 + e];
                    fb4[e] = ColFb[c4 + e];
                }
                const int32_t n = n0 + c4;
#pragma unroll 4
                for (int jj = 0; jj < BT / (THREADS / 32); jj++) {
                    const int rl = r0 + (THREADS / 32) * jj;
                    const int32_t m = m0 + rl;
                    if (m >= M || n >= N) continue;   // N % 4 == 0: the four columns are all in or all out
                    const v4i raw = *reinterpret_cast<const v4i *>(&T[rl * LDT + c4]);
                    const uint32_t ss = SUM_A ? (uint32_t)RowSum[rl] : 0u, zz = SUM_B ? (uint32_t)RowZ[rl] : 0u;
                    uint32_t v[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = (uint32_t)raw[e] - wz4[e] * ss - zz * ct4[e] + ib4[e];   // once a 16 bytes
                    const int64_t at = (int64_t)m * N + n;
                    if constexpr (MODE == 1) {
                        float f[4];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            f[e] = __fmul_rn((float)(int32_t)v[e], sc4[e]);
                            if (opt) f[e] = __fadd_rn(f[e], fb4[e]);
                            rmn = fminf(rmn, f[e]);   // (the 128 tile only: this path)
                            rmx = fmaxf(rmx, f[e]);
                        }
                        *reinterpret_cast<v4i *>(Cb + at) =
                            (v4i){__float_as_int(f[0]), __float_as_int(f[1]), __float_as_int(f[2]), __float_as_int(f[3])};
                    } else if constexpr (MODE == 2) {
                        uint32_t word = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) word |= requantize_byte(v[e], sc4[e], zp_y, opt) << (8 * e);
                        *reinterpret_cast<uint32_t *>(Yb + at) = word;
                    } else {
                        *reinterpret_cast<v4i *>(Cb + at) = (v4i){(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3]};
                    }
                }
                return;
            }
        }
        // WHOLE: every row and column of the tile is in range (all tiles but the last row and column of tiles), so
        // no store needs a bounds check: a lane's row address once per row, its column blocks at immediate offsets.
        auto store_rows = [&](auto whole_tag, auto small_tag) {
            constexpr bool WHOLE = decltype(whole_tag)::value, SMALL = decltype(small_tag)::value;
#pragma unroll
            for (int i = 0; i < FM; i++) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int ml = wm * WTM + 32 * i + 8 * q + 4 * h2;
                    const v4i ssv = SUM_A ? *reinterpret_cast<const v4i *>(&RowSum[ml]) : (v4i){0, 0, 0, 0};
                    const v4i zzv = SUM_B ? *reinterpret_cast<const v4i *>(&RowZ[ml]) : (v4i){0, 0, 0, 0};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int32_t m = m0 + ml + r;
                        if (!WHOLE && m >= M) continue;
                        int32_t *const row = Cb + m * N + ncol0;   // batch * M * N < 2^31 (checked at the boundary)
                        uint8_t *const yrow = Yb + m * N + ncol0;
                        const uint32_t ss = (uint32_t)ssv[r], zz = (uint32_t)zzv[r];
#pragma unroll
                        for (int j = 0; j < FN; j++) {
                            if (!WHOLE && ncol0 + 32 * j >= N) continue;
                            const uint32_t v = (uint32_t)acc[i][j][4 * q + r] - zmul<SMALL>(wz[j], ss) -
                                               zmul<SMALL>(zz, ct[j]) + ib[j];
                            if constexpr (MODE == 1) {
                                float f = __fmul_rn((float)(int32_t)v, sc[j]);
                                if (opt) f = __fadd_rn(f, fb[j]);
                                row[32 * j] = __float_as_int(f);
                                if constexpr (BT == 128) {
                                    rmn = fminf(rmn, f);
                                    rmx = fmaxf(rmx, f);
                                }
                            } else if constexpr (MODE == 2) {
                                yrow[32 * j] = (uint8_t)requantize_byte(v, sc[j], zp_y, opt);
                            } else {
                                row[32 * j] = (int32_t)v;
                            }
                        }
                    }
                }
            }
        };
        const bool whole = m0 + DBM <= M && n0 + DBN <= N;
        if (whole) {
            if (small_k) store_rows(std::true_type{}, std::true_type{});
            else store_rows(std::true_type{}, std::false_type{});
        } else {
            if (small_k) store_rows(std::false_type{}, std::true_type{});
            else store_rows(std::false_type{}, std::false_type{});
        }
    };
    if (epi & EPI_REQUANT) {
        store_all(std::integral_constant<int, 2>{}, (epi & EPI_REQUANT_U8) != 0);
    } else if (epi & OG_EPI_FLOAT) {
        if (epi & OG_EPI_FLOAT_BIAS) store_all(std::integral_constant<int, 1>{}, true);
        else store_all(std::integral_constant<int, 1>{}, false);
        if (BT == 128 && g.ranges) {
            // A ranged float product: the workgroup's range of what it stored, in its slot (its workgroup id). (The 256
            // tile has no range epilogue: with it, its registers spill; its ranged products take a range pass.)
            __syncthreads();   // every thread done reading the epilogue's arrays in LDS
            store_workgroup_range<THREADS>(rmn, rmx, reinterpret_cast<float *>(smem), g.ranges, blockIdx.x);
        }
    } else {
        store_all(std::integral_constant<int, 0>{}, false);
    }
}

// The waves a 256 tile runs on: 8 (two a SIMD) when a wave's registers fit in half the SIMD's file; a product that
// needs both operands' byte sums does not fit (the compiler spills inside the loop), so it keeps 4.
template <int BT, bool SA, bool SB, int WAVES>
constexpr int direct_waves()
{
    return (BT == 256 && SA && SB) ? 4 : WAVES;
}

// Whether a 256 tile on 8 waves runs its stages in ping-pong order: not when A's row sums are needed (B has a zero
// point or is unsigned), whose ping-pong form spills registers.
template <int BT, bool SA, bool SB, int WAVES>
constexpr bool direct_pingpong()
{
    return BT == 256 && direct_waves<BT, SA, SB, WAVES>() == 8 && !SA;
}

// One instantiation per operand signedness and needed byte sums (an unsigned operand always needs the other's sums).
template <int BT, bool T, bool FA, bool FB, int WAVES>
inline void launch_direct_flips(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm, int32_t ks,
                                int32_t kslice, bool sa, bool sb)
{
#define OG_D(SA, SB) \
    hipLaunchKernelGGL((k_gemm_direct<BT, T, SA, SB, FA, FB, direct_waves<BT, SA, SB, WAVES>(), \
                                      direct_pingpong<BT, SA, SB, WAVES>()>), grid, \
                       dim3(64 * direct_waves<BT, SA, SB, WAVES>()), 0, s, g, tn, tm, ks, kslice)
    if constexpr (FA && FB) {
        OG_D(true, true);
    } else if constexpr (FA) {
        if (sa) OG_D(true, true);
        else OG_D(false, true);
    } else if constexpr (FB) {
        if (sb) OG_D(true, true);
        else OG_D(true, false);
    } else {
        if (sa && sb) OG_D(true, true);
        else if (sa) OG_D(true, false);
        else if (sb) OG_D(false, true);
        else OG_D(false, false);
    }
#undef OG_D
}

template <int BT, bool T, int WAVES = 4>
inline void launch_direct_t(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm, int32_t ks,
                            int32_t kslice)
{
    const bool fa = !(g.flags & OG_GEMM_A_INT8), fb = !(g.flags & OG_GEMM_B_INT8);
    const bool sa = (g.flags & OG_GEMM_ZB) || fb, sb = (g.flags & OG_GEMM_ZA) || fa;
    if (fa && fb) launch_direct_flips<BT, T, true, true, WAVES>(g, s, grid, tn, tm, ks, kslice, sa, sb);
    else if (fa) launch_direct_flips<BT, T, true, false, WAVES>(g, s, grid, tn, tm, ks, kslice, sa, sb);
    else if (fb) launch_direct_flips<BT, T, false, true, WAVES>(g, s, grid, tn, tm, ks, kslice, sa, sb);
    else launch_direct_flips<BT, T, false, false, WAVES>(g, s, grid, tn, tm, ks, kslice, sa, sb);
}

// Instantiated in translation units of their own (compiled in parallel): B stored N x K at 256, both layouts at 128.
void launch_direct_nk256(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm);
void launch_direct128(const GemmArgs &g, hipStream_t s, dim3 grid, int32_t tn, int32_t tm, int32_t ks, int32_t kslice);

}  // namespace og
