// Few-rows int8 products (M <= 16, B stored K x N) in one launch: the decode-step shape, bound by reading B once.
//
//  - B is cut into tiles of 512 rows x 128 columns, one workgroup each. Every thread issues all its loads at once
//    (16 pieces of 16 bytes of B, each wave instruction eight whole 128-byte row segments, plus the A fragments it
//    needs), so the whole matrix is requested from HBM together: every tile of the C3 shape is resident at once.
//  - Each 64-row step, the four waves write the step's rows into LDS (two 8 KB buffers in turn) and wave w reads back
//    its columns 32 w .. 32 w + 31 transposed (ds_read_b64_tr_b8) as the B operand of v_mfma_i32_16x16x64_i8. The A
//    operand has 16 rows; when M < 16 row M is all ones, so the same MFMA also gives the column sums of B that A's
//    zero point needs (M = 16 runs a second MFMA against ones).
//  - The tiles of column slab q hand their parts (their k-range's sums, column sums and the row sums of A) to the
//    tile of the slab's last row band, the slab's highest workgroup id, dispatched after the others. Every other tile
//    stores its part, waits until the stores are in L2 and counts the part in the slab's word (an L2 atomic). The
//    finishing tile keeps its own sums, fetches its epilogue operands, waits until the other parts are counted (they
//    have all been dispatched, and none waits for anything), reads them, adds them in part order, applies the zero
//    points with the whole K and the epilogue, stores C and clears the word.
//
// No cache write-back is needed. The hardware deals workgroup ids round-robin to the 8 XCDs and each XCD has its own
// L2, so the tiles of one slab are given ids that are equal modulo 8: all of them run on the same XCD, where a store
// that has drained (s_waitcnt vmcnt(0)) is in the one L2 they share: the release of a single-L2 device. The finishing
// tile reads the word with atomics and the parts with agent-scope loads (global_load sc1), which pass its CU's L1 (a
// plain or workgroup-scope load may be answered by a stale L1 line, and buffer_inv sc0 does not clear it), so both
// come from that L2. Each count goes to the 7-bit field of the word that belongs to the XCD the tile ran on
// (HW_REG_XCC_ID), so the finishing tile checks that every tile of its slab shared its L2; if not, it raises a flag in
// host memory that og_sync reports (og_init runs this kernel only after a probe launch has shown the mapping). The
// wait is bounded: past the bound the tile raises the flag and leaves its columns of C unwritten.
//
// A failed hand-off leaves count words behind (tiles still count after the finishing tile gave up, and a slab split
// over two XCDs has counted in two L2s). So the finishing tile that fails also sets the poison word (word 0 of
// `words`, an agent-scope store), and every later launch's finishing tiles read it first (agent scope, coherent
// across the XCDs; a launch starts after the previous one on the stream has ended) and, finding it set, raise the
// flag (3) without reading any part. og_sync clears all the words (poison included) once it has seen the flag.
//        sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w'   (mod 2^32; Int8GemmDot.hlsl:1-11)
#include <algorithm>
#include <type_traits>

#include "og_internal.hpp"

namespace og {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));

// Tile geometry: GX_KT rows x GX_COLS columns of B (64 KB), 256 threads.
constexpr int GX_COLS = 128, GX_KT = 512, GX_THREADS = 256;
constexpr int GX_CPR = GX_COLS / 16;                          // 16-byte chunks a row (8)
constexpr int GX_LOADS = GX_KT * GX_COLS / 16 / GX_THREADS;   // 16-byte loads of B a thread (16)
constexpr int GX_ROWS_PER_LOAD = GX_THREADS / GX_CPR;         // rows one load of every thread covers (32)
constexpr int GX_STEPS = GX_KT / 64;                          // 64-row MFMA steps (8)
constexpr int GX_LPS = 64 / GX_ROWS_PER_LOAD;                 // loads a step (2)
constexpr int GX_CPW = GX_CPR / 4;                            // chunks a wave computes (2)
constexpr int GX_STAGE = 64 * GX_COLS;                        // bytes of one step in LDS
constexpr int GX_RED = 17 * GX_COLS + 16;                     // the finishing tile's sums (ints)
static_assert(GX_CPR == 8 && GX_LPS * GX_ROWS_PER_LOAD == 64, "the staging layout below is for 128-byte rows");

__device__ __forceinline__ v4i gx_load(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);   // nontemporal: B is read once
}

// Position of 16-byte chunk c of staged row k (128-byte rows; the row's parity picks the 128-byte half of the 256
// bytes LDS serves a cycle): the 16 rows x 16 bytes of one transpose read (rows k and k + 16, k % 16 < 8 or >= 8),
// and the 2 rows x 8 chunks of one 16-lane write, fall on different 16-byte slots.
__device__ __forceinline__ int gx_pos(int k, int c) { return c ^ (((k >> 1) & 3) | (((k >> 4) & 1) << 2)); }

__device__ __forceinline__ uint32_t gx_sad16(v4i v, uint32_t acc)
{
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.x, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.y, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.z, 0u, acc);
    return __builtin_amdgcn_sad_u8((uint32_t)v.w, 0u, acc);
}

template <typename F, int... I>
__device__ __forceinline__ void gx_static_for(F &&f, std::integer_sequence<int, I...>)
{
    (f(std::integral_constant<int, I>{}), ...);
}

__device__ __forceinline__ uint32_t gx_xcc_id()
{
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 7u;
}

// LDS writes of every wave done, then all waves meet (no wait for the outstanding loads of B).
__device__ __forceinline__ void gx_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace

// Ints of one tile's part: R = M + 1 rows of GX_COLS sums (rows 0 .. M - 1: sum s t over the tile's k-range; row M:
// the column sums of B), then 16 row sums of A; padded to a 128-byte multiple.
__host__ __device__ inline int64_t gemv_xcd_part(int32_t M) { return (int64_t)(M + 1) * GX_COLS + 32; }

// Workgroup id x: XCD x % 8 takes slabs [x8 * Q / 8, (x8 + 1) * Q / 8) of the Q = batch * slabs column slabs; its
// j-th workgroup (j = x / 8) takes slab j % nq of them (slab-fastest, so the tiles running together cover whole rows
// of B) and row band j / nq. Word 1 + q of `words` counts slab q's stored parts; word 0 is the poison word.
// spin_limit: polls of the count before the finishing tile gives up (0: it gives up at once, without reading the
// count; the library's tests use that to drive the recovery path).
template <bool SUM_A, bool SUM_B, bool FLIP_A, bool FLIP_B, bool ROWS16>
__global__ __launch_bounds__(GX_THREADS) void k_gemv_xcd(GemmArgs g, int32_t slabs, int32_t nkc, int32_t qtotal,
                                                         int32_t *parts, unsigned long long *words, uint32_t *flag,
                                                         uint32_t spin_limit)
{
    __shared__ __attribute__((aligned(1024))) int32_t smem[(2 * GX_STAGE / 4) > GX_RED ? (2 * GX_STAGE / 4) : GX_RED];
    __shared__ uint32_t s_ok;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g4 = lane >> 4;
    const int32_t x8 = (int32_t)(blockIdx.x & 7u), jx = (int32_t)(blockIdx.x >> 3);
    const int32_t q0 = (int32_t)((int64_t)x8 * qtotal / 8), q1 = (int32_t)((int64_t)(x8 + 1) * qtotal / 8);
    const int32_t nq = q1 - q0;
    if (jx >= nq * nkc) return;   // the XCD's share is done (whole workgroup)
    const int32_t q = q0 + jx % nq, kc = jx / nq;
    const int32_t b = q / slabs, slab = q % slabs;
    const int32_t M = g.M, N = g.N, K = g.K, ldb = g.ldb, lda = g.lda;
    const int32_t n0 = slab * GX_COLS, k0 = kc * GX_KT, rows = min(GX_KT, K - k0);

    // All loads issued here, in the order they are waited for: the A fragments (lane: row i16 of A, 16 bytes at
    // k0 + 64 s + 16 g4; rows past M read as zero, bytes past K are masked when used), then the 16 pieces of B (load
    // i: tile row 32 i + 8 wave + lane / 8, chunk lane % 8: each wave instruction reads eight whole 128-byte row
    // segments; rows past K and bytes past the operand read as zero).
    v4i af[GX_STEPS], bv[GX_LOADS];
    {
        const uint8_t *abase = g.A + (int64_t)b * g.strideA + k0;
        const __amdgpu_buffer_rsrc_t ra =
            __builtin_amdgcn_make_buffer_rsrc((void *)abase, (short)0, (M - 1) * lda + rows, 0x00020000);
#pragma unroll
        for (int s = 0; s < GX_STEPS; s++)
            af[s] = __builtin_amdgcn_raw_buffer_load_b128(ra, (uint32_t)(i16 * lda + 64 * s + 16 * g4), 0, 0);
        const uint8_t *bbase = g.B + (int64_t)b * g.strideB + (int64_t)k0 * ldb + n0;
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
            (void *)bbase, (short)0, (rows - 1) * ldb + min(GX_COLS, N - n0), 0x00020000);
        const uint32_t r0 = (uint32_t)(8 * wave + (lane >> 3)) * (uint32_t)ldb + 16u * (uint32_t)(lane & 7);
#pragma unroll
        for (int i = 0; i < GX_LOADS; i++) bv[i] = gx_load(rb, r0 + (uint32_t)(GX_ROWS_PER_LOAD * i) * (uint32_t)ldb);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ROWS16: M = 16 with the column sums needed (no spare row in the MFMA's A operand: a second MFMA against ones).
    constexpr bool ones_mfma = SUM_B && ROWS16;
    const bool ones_row = SUM_B && !ROWS16;
    v4i acc[GX_CPW], accs[GX_CPW];
#pragma unroll
    for (int c = 0; c < GX_CPW; c++) { acc[c] = (v4i){0, 0, 0, 0}; accs[c] = (v4i){0, 0, 0, 0}; }
    uint32_t rsum = 0;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)smem;

    gx_static_for([&](auto s_tag) {
        constexpr int s = decltype(s_tag)::value;
        // Step s: rows 64 s .. 64 s + 63, B loads 2 s and 2 s + 1 of every wave (the compiler waits for exactly
        // those: vmcnt counts the loads in issue order), into buffer s % 2. The barrier of step s - 1 came after every
        // wave's reads of step s - 2 had returned, so the buffer is free.
        uint8_t *const buf = reinterpret_cast<uint8_t *>(smem) + (s & 1) * GX_STAGE;
#pragma unroll
        for (int i = 0; i < GX_LPS; i++) {
            const int r = GX_ROWS_PER_LOAD * i + 8 * wave + (lane >> 3);
            *reinterpret_cast<v4i *>(buf + r * GX_COLS + 16 * gx_pos(r, lane & 7)) = bv[GX_LPS * s + i];
        }
        gx_lds_barrier();
        const bool kv = 64 * s + 16 * g4 < rows;
        const bool av = kv && i16 < M;
        v4i a = af[s];
        if constexpr (!FLIP_A) a = av ? a : (v4i){0, 0, 0, 0};
        if constexpr (SUM_A) rsum = av ? gx_sad16(FLIP_A ? a : (a ^ (int32_t)0x80808080), rsum) : rsum;
        if constexpr (FLIP_A) a = av ? (a ^ (int32_t)0x80808080) : (v4i){0, 0, 0, 0};
        const int32_t one = kv ? 0x01010101 : 0;
        if (ones_row && i16 == M) a = (v4i){one, one, one, one};
        const v4i ones = (v4i){one, one, one, one};
        const uint32_t bl = lds0 + (s & 1) * GX_STAGE;
#pragma unroll
        for (int c = 0; c < GX_CPW; c++) {
            const int chunk = GX_CPW * wave + c;
            v2i h[2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int k = 16 * g4 + 8 * hh + (i16 >> 1);
                h[hh] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(uintptr_t)(
                    bl + k * GX_COLS + 16 * gx_pos(k, chunk) + 8 * (i16 & 1)));
            }
            v4i bf = (v4i){h[0].x, h[0].y, h[1].x, h[1].y};
            if constexpr (FLIP_B) bf ^= (int32_t)0x80808080;
            acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bf, acc[c], 0, 0, 0);
            if constexpr (ones_mfma) accs[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ones, bf, accs[c], 0, 0, 0);
        }
    }, std::make_integer_sequence<int, GX_STEPS>{});

    // A's row sums over the tile: biased byte sums of the four k-groups (lanes l, l + 16, l + 32, l + 48); the signed
    // sum is 128 less a byte.
    uint32_t rowsum = 0;
    if (SUM_A) {
        uint32_t v = rsum + (uint32_t)__shfl_xor((int32_t)rsum, 16);
        v += (uint32_t)__shfl_xor((int32_t)v, 32);
        rowsum = v - 128u * (uint32_t)rows;
    }

    // The part, in the MFMA 16 x 16 layout: lane l holds rows 4 (l / 16) + r of column l % 16 of each block. Rows
    // 0 .. M - 1 are sums, row M (M < 16) the column sums; with M = 16 they come from the second MFMA (all its rows
    // equal). Stored to the workspace (global stores), or, by the finishing tile, into LDS.
    const int32_t R = SUM_B ? M + 1 : M;
    const int64_t pstride = gemv_xcd_part(M);
    auto put_part = [&](int32_t *dst) {
#pragma unroll
        for (int c = 0; c < GX_CPW; c++) {
            const int col = 16 * (GX_CPW * wave + c) + i16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g4 + r;
                if (row < R) dst[row * GX_COLS + col] = acc[c][r];
            }
            if constexpr (ones_mfma)
                if (g4 == 0) dst[16 * GX_COLS + col] = accs[c][0];
        }
        if (SUM_A && wave == 0 && g4 == 0) dst[R * GX_COLS + i16] = (int32_t)rowsum;
    };
    unsigned long long *const poison = words, *const word = words + 1 + q;
    if (kc != nkc - 1) {
        put_part(parts + ((int64_t)q * nkc + kc) * pstride);
        // Counted once this wave's stores are in L2 (vmcnt drains) and every wave's are, in the 7-bit field of the
        // XCD the tile ran on.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0)
            __hip_atomic_fetch_add(word, 1ull << (7 * gx_xcc_id()), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return;
    }
    // Whether an earlier launch failed its hand-off: requested now, used after the epilogue operands are in flight.
    const unsigned long long poisoned =
        tid == 0 ? __hip_atomic_load(poison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    gx_lds_barrier();   // every wave's MFMAs are done, so their reads of the staging buffers too
    put_part(smem);

    // The finishing tile. Its epilogue operands are fetched first, so their latency overlaps the wait: thread t
    // serves column t % GX_COLS and rows t / GX_COLS, + 2, ... (at most 8 rows a thread).
    constexpr int GX_EROWS = GX_THREADS / GX_COLS;
    const int ecol = tid % GX_COLS, erow0 = tid / GX_COLS, en = n0 + ecol;
    const uint32_t epi = g.epi;
    uint32_t wz = 0, ib = 0, zz[16 / GX_EROWS];
    float esc = 0.0f, efb = 0.0f;
    if (en < N) {
        if (SUM_A) {
            const uint32_t w = g.ZB ? g.ZB[(g.flags & OG_GEMM_ZB_PER_COL) ? en : 0] : 0u;
            wz = FLIP_B ? w - 128u : (uint32_t)sext8(w);
        }
        if (epi & OG_EPI_INT_BIAS) ib = (uint32_t)g.bias[en];
        if (epi & EPI_REQUANT) esc = g.scale[(epi & OG_EPI_SCALE_PER_COL) ? en : 0];
        else if (epi & OG_EPI_FLOAT) {
            esc = column_scale(g, en);
            if (epi & OG_EPI_FLOAT_BIAS) efb = g.fbias[en];
        }
    }
#pragma unroll
    for (int j = 0; j < 16 / GX_EROWS; j++) {
        const int m = erow0 + GX_EROWS * j;
        uint32_t z = 0;
        if (SUM_B && m < M) {
            const uint32_t zr = g.ZA ? g.ZA[(g.flags & OG_GEMM_ZA_PER_ROW) ? m : 0] : 0u;
            z = FLIP_A ? zr - 128u : (uint32_t)sext8(zr);
        }
        zz[j] = z;
    }

    // Wait until the other nkc - 1 parts are counted. Each poll is an atomic add to the word's top byte (so it is
    // performed in L2: an idempotent read-modify-write may be compiled to a plain load, which the L1 can answer);
    // bits 0 .. 55 are the eight XCDs' 7-bit counts.
    if (tid == 0) {
        if (poisoned) {
            // The words are stale: raise the flag and leave this slab's columns of C unwritten.
            *flag = 3u;
            s_ok = 0u;
        } else {
            const uint32_t xcc = gx_xcc_id();
            uint32_t polls = 0, total = 0;
            unsigned long long now = 0;
            while (spin_limit != 0) {
                now = __hip_atomic_fetch_add(word, 1ull << 56, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                total = 0;
#pragma unroll
                for (int x = 0; x < 8; x++) total += (uint32_t)(now >> (7 * x)) & 127u;
                if (total == (uint32_t)(nkc - 1) || ++polls >= spin_limit) break;
                __builtin_amdgcn_s_sleep(1);
            }
            const bool done = spin_limit != 0 && total == (uint32_t)(nkc - 1);
            const bool here = (now & ((1ull << 56) - 1)) == ((unsigned long long)(nkc - 1) << (7 * xcc));
            if (!done) *flag = 2u;
            else if (!here) *flag = 1u;   // some tile of the slab ran on another XCD: its sums may be wrong
            if (!done || !here) __hip_atomic_store(poison, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *word = 0ull;   // every other tile of the slab has counted its part: free for the next product
            s_ok = done ? 1u : 0u;
        }
    }
    __syncthreads();
    if (!s_ok) return;

    // The other parts (slices 0 .. nkc - 2), read with agent-scope loads (sc1: past the vector L1, from the XCD's L2)
    // and added in part order to the tile's own sums. A thread serves POS 16-byte positions (POS = 1 up to 256
    // positions, M < 8; else 3) and takes the parts in groups of G (8, or 4 with 3 positions, which keeps the
    // registers of the whole kernel within three waves a SIMD): every load of a group is issued before any is used, so
    // a group costs one round trip. Reads past the parts return zero.
    const int32_t *pq = parts + (int64_t)q * nkc * pstride;
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void *)pq, (short)0, (nkc - 1) * (int32_t)pstride * 4, 0x00020000);
    constexpr int GX_SC1 = 16;   // cache policy: sc1
    static_assert(GX_COLS / 4 == 32 && 17 * 32 <= 3 * GX_THREADS, "position it: row it / 32, columns 4 (it % 32) ..");
    const int npos = R * (GX_COLS / 4);
    auto add_parts = [&](auto pos_tag, auto group_tag) {
        constexpr int POS = decltype(pos_tag)::value, G = decltype(group_tag)::value;
        v4i tot[POS];
        uint32_t at[POS];
#pragma unroll
        for (int u = 0; u < POS; u++) {
            const int it = tid + GX_THREADS * u;
            at[u] = (uint32_t)((it >> 5) * GX_COLS + 4 * (it & 31)) * 4u;
            tot[u] = it < npos ? *reinterpret_cast<const v4i *>(reinterpret_cast<const uint8_t *>(smem) + at[u])
                               : (v4i){0, 0, 0, 0};
        }
        for (int p0 = 0; p0 < nkc - 1; p0 += G) {
            v4i t[POS][G];
#pragma unroll
            for (int u = 0; u < POS; u++)
#pragma unroll
                for (int e = 0; e < G; e++) {
                    const bool in = tid + GX_THREADS * u < npos && p0 + e < nkc - 1;
                    t[u][e] = __builtin_amdgcn_raw_buffer_load_b128(
                        rp, in ? (uint32_t)(p0 + e) * (uint32_t)pstride * 4u + at[u] : 0x80000000u, 0, GX_SC1);
                }
#pragma unroll
            for (int u = 0; u < POS; u++)
#pragma unroll
                for (int e = 0; e < G; e++) tot[u] += t[u][e];
        }
#pragma unroll
        for (int u = 0; u < POS; u++)
            if (tid + GX_THREADS * u < npos)
                *reinterpret_cast<v4i *>(reinterpret_cast<uint8_t *>(smem) + at[u]) = tot[u];
    };
    if (npos <= GX_THREADS) add_parts(std::integral_constant<int, 1>{}, std::integral_constant<int, 8>{});
    else add_parts(std::integral_constant<int, 3>{}, std::integral_constant<int, 4>{});
    if (SUM_A && tid < 16) {
        uint32_t rs = (uint32_t)smem[R * GX_COLS + tid];
        for (int p0 = 0; p0 < nkc - 1; p0 += 8) {
            uint32_t t[8];
#pragma unroll
            for (int e = 0; e < 8; e++)
                t[e] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                    rp, p0 + e < nkc - 1 ? ((uint32_t)(p0 + e) * (uint32_t)pstride + (uint32_t)(R * GX_COLS + tid)) * 4u : 0x80000000u,
                    0, GX_SC1);
#pragma unroll
            for (int e = 0; e < 8; e++) rs += t[e];
        }
        smem[R * GX_COLS + tid] = (int32_t)rs;
    }
    __syncthreads();

    // A ranged float product: the NaN-ignoring range of the values this thread stores, then the slab's in slot q.
    float rmn = __int_as_float(0x7F800000), rmx = __int_as_float(0xFF800000);
    if (en < N) {
        const uint32_t cs = SUM_B ? (uint32_t)smem[M * GX_COLS + ecol] : 0u;
#pragma unroll
        for (int j = 0; j < 16 / GX_EROWS; j++) {
            const int m = erow0 + GX_EROWS * j;
            if (m >= M) break;
            const uint32_t v = (uint32_t)smem[m * GX_COLS + ecol];
            const uint32_t rs = SUM_A ? (uint32_t)smem[R * GX_COLS + m] : 0u;
            const uint32_t res = v - wz * rs - zz[j] * (cs - (uint32_t)K * wz) + ib;
            const int64_t ci = (int64_t)b * g.strideC + (int64_t)m * N + en;
            if (epi & EPI_REQUANT) {
                store_requantized_col(g, ci, res, esc, 0.0f);
            } else if (g.ranges) {
                float f = __fmul_rn((float)(int32_t)res, esc);
                if (epi & OG_EPI_FLOAT_BIAS) f = __fadd_rn(f, efb);
                static_cast<float *>(g.C)[ci] = f;
                rmn = fminf(rmn, f);
                rmx = fmaxf(rmx, f);
            } else {
                store_sum_col(g, ci, res, esc, efb);
            }
        }
    }
    if (g.ranges) {
        __syncthreads();   // every thread done reading the sums in LDS
        store_workgroup_range<GX_THREADS>(rmn, rmx, reinterpret_cast<float *>(smem), g.ranges, (uint32_t)q);
    }
}

// Records each workgroup's XCD: out[x] = HW_REG_XCC_ID of workgroup x.
__global__ void k_xcc_probe(uint32_t *out)
{
    if (threadIdx.x == 0) out[blockIdx.x] = gx_xcc_id();
}

hipError_t launch_xcc_probe(uint32_t *out, uint32_t groups, hipStream_t s)
{
    hipLaunchKernelGGL(k_xcc_probe, dim3(groups), dim3(64), 0, s, out);
    return hipGetLastError();
}

// The streaming floor of k_gemv_xcd's shapes (a benchmark utility): the same grid, tile mapping and loads of B (all
// 16 issued at once, nontemporal), with nothing done with the bytes but a checksum that is stored only if it equals
// an unlikely constant (so the loads stay live and nothing else touches memory).
__global__ __launch_bounds__(GX_THREADS) void k_stream_tiles(const uint8_t *B, int32_t K, int32_t N, int32_t slabs,
                                                             int32_t nkc, uint32_t *sink)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t x8 = (int32_t)(blockIdx.x & 7u), jx = (int32_t)(blockIdx.x >> 3);
    const int32_t q0 = (int32_t)((int64_t)x8 * slabs / 8), q1 = (int32_t)((int64_t)(x8 + 1) * slabs / 8);
    const int32_t nq = q1 - q0;
    if (jx >= nq * nkc) return;
    const int32_t slab = q0 + jx % nq, kc = jx / nq;
    const int32_t n0 = slab * GX_COLS, k0 = kc * GX_KT, rows = min(GX_KT, K - k0);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(B + (int64_t)k0 * N + n0), (short)0, (rows - 1) * N + min(GX_COLS, N - n0), 0x00020000);
    const uint32_t r0 = (uint32_t)(8 * wave + (lane >> 3)) * (uint32_t)N + 16u * (uint32_t)(lane & 7);
    v4i bv[GX_LOADS];
#pragma unroll
    for (int i = 0; i < GX_LOADS; i++) bv[i] = gx_load(rb, r0 + (uint32_t)(GX_ROWS_PER_LOAD * i) * (uint32_t)N);
    v4i x = bv[0];
#pragma unroll
    for (int i = 1; i < GX_LOADS; i++) x ^= bv[i];
    const uint32_t c = (uint32_t)(x.x ^ x.y ^ x.z ^ x.w);
    if (c == 0x9E3779B9u) sink[0] = c;
}

hipError_t launch_stream_tiles(const uint8_t *B, int32_t K, int32_t N, uint32_t *sink, hipStream_t s)
{
    const int32_t slabs = (N + GX_COLS - 1) / GX_COLS, nkc = (K + GX_KT - 1) / GX_KT;
    hipLaunchKernelGGL(k_stream_tiles, dim3((uint32_t)(8 * ((slabs + 7) / 8) * nkc)), dim3(GX_THREADS), 0, s, B, K, N,
                       slabs, nkc, sink);
    return hipGetLastError();
}

// The one-launch few-rows kernel's conditions: those of the two-launch tile kernel (B stored K x N; 16-byte aligned
// rows; K and N multiples of 16), at least 16 column slabs (two an XCD) and at most 127 row bands (a 7-bit field of
// the slab's word counts them).
bool gemv_xcd_ok(const GemmArgs &g)
{
    if (!gemv_tiles_ok(g)) return false;
    const int64_t q = (int64_t)g.batch * ((g.N + GX_COLS - 1) / GX_COLS), nkc = (g.K + GX_KT - 1) / GX_KT;
    if (q < 16 || nkc > 127) return false;
    if ((int64_t)GX_KT * g.ldb + GX_COLS > 0x7FFFFFFFll || (int64_t)16 * g.lda + GX_KT > 0x7FFFFFFFll) return false;
    return 8 * ((q + 7) / 8) * nkc <= 0x7FFFFFFFll && q <= 0x7FFFFFFFll / 8;
}

uint64_t gemv_xcd_workspace_bytes(const GemmArgs &g)
{
    const int64_t q = (int64_t)g.batch * ((g.N + GX_COLS - 1) / GX_COLS), nkc = (g.K + GX_KT - 1) / GX_KT;
    return (uint64_t)(q * nkc * gemv_xcd_part(g.M) * 4);
}

uint32_t gemv_xcd_range_groups(const GemmArgs &g)
{
    return (uint32_t)((int64_t)g.batch * ((g.N + GX_COLS - 1) / GX_COLS));   // one a column slab (its finishing tile)
}

uint64_t gemv_xcd_words(const GemmArgs &g)
{
    return 1 + (uint64_t)g.batch * ((g.N + GX_COLS - 1) / GX_COLS);   // the poison word, then one a slab
}

hipError_t launch_gemv_xcd(const GemmArgs &g, int32_t *parts, unsigned long long *words, uint32_t *flag,
                           uint32_t spin_limit, hipStream_t s, const char **kernel)
{
    const int32_t slabs = (g.N + GX_COLS - 1) / GX_COLS, nkc = (g.K + GX_KT - 1) / GX_KT;
    const int32_t q = g.batch * slabs;
    const bool fa = !(g.flags & OG_GEMM_A_INT8), fb = !(g.flags & OG_GEMM_B_INT8);
    const bool sa = (g.flags & OG_GEMM_ZB) || fb, sb = (g.flags & OG_GEMM_ZA) || fa;
    const dim3 block(GX_THREADS), grid((uint32_t)(8 * ((q + 7) / 8) * nkc));
    *kernel = "mfma-i8-rows16-xcd";
#define OG_GX(SA, SB, FA, FB)                                                                                     \
    do {                                                                                                          \
        if (SB && g.M == 16)                                                                                      \
            hipLaunchKernelGGL((k_gemv_xcd<SA, SB, FA, FB, true>), grid, block, 0, s, g, slabs, nkc, q,           \
                               parts, words, flag, spin_limit);                                                               \
        else                                                                                                      \
            hipLaunchKernelGGL((k_gemv_xcd<SA, SB, FA, FB, false>), grid, block, 0, s, g, slabs, nkc, q,          \
                               parts, words, flag, spin_limit);                                                               \
    } while (0)
    if (fa && fb) OG_GX(true, true, true, true);
    else if (fa) { if (sa) OG_GX(true, true, true, false); else OG_GX(false, true, true, false); }
    else if (fb) { if (sb) OG_GX(true, true, false, true); else OG_GX(true, false, false, true); }
    else if (sa && sb) OG_GX(true, true, false, false);
    else if (sa) OG_GX(true, false, false, false);
    else if (sb) OG_GX(false, true, false, false);
    else OG_GX(false, false, false, false);
#undef OG_GX
    return hipGetLastError();
}

}  // namespace og
