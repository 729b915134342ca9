// Few-rows int8 products (M <= 16, B stored K x N), streamed: the decode-step shape, bound by reading B once from HBM.
//
//  - Work units are (column slab of 256, 64 rows of K) pairs, dealt out evenly to one workgroup per CU: a workgroup
//    takes a contiguous run of units, which covers one slab or a few (every CU streams the same number of bytes).
//  - Each unit's B tile (64 x 256) and A tile (the <= 16 activation rows x 64) go from HBM to a ring of LDS stages by
//    DMA (buffer_load ... lds), seven units ahead; B is read back with the gfx950 transpose read ds_read_b64_tr_b8 and
//    each wave runs four v_mfma_i32_16x16x64_i8 (its 64 columns) per unit.
//  - Where a workgroup's run leaves a slab it writes that slab's part: the raw sums sum s t, and the byte sums of its
//    rows of A and columns of B over its k-range. The last workgroup to finish a slab (a counter per slab, reset by
//    that workgroup) adds the parts and applies the zero points and the epilogue once, with the whole K. Parts are
//    written as agent-scope atomic stores (written through, so no L2 write-back of a release fence is needed) and are
//    acknowledged (vmcnt 0) before their workgroup counts in; the finishing workgroup reads them after an acquire.
//        sum (s - z')(t - w') = sum s t - w' sum s - z' sum t + K z' w'   (mod 2^32; Int8GemmDot.hlsl:1-11)
//    Integer sums are exact in any order, so the result does not depend on how the units were dealt out.
#include <type_traits>

#include "og_internal.hpp"

namespace og {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u4w __attribute__((ext_vector_type(4)));

constexpr int GS_COLS = 256, GS_K = 64, GS_THREADS = 256;
constexpr int GS_B = GS_K * GS_COLS;     // bytes of B per unit
constexpr int GS_A = 16 * GS_K;          // bytes of A per unit (16 rows)
constexpr int GS_STG = GS_B + GS_A;
constexpr int GS_NS = 8;                 // LDS stages: one being read, seven in flight
constexpr int GS_LOADS = 5;              // loads per wave per unit: four of B (16 bytes a lane), one of A (4 bytes)
constexpr int GS_PART = 16 * GS_COLS + GS_COLS + 16;   // int32s of one part: sums s t, column sums, row sums

__device__ __forceinline__ u4w rsrc_of(const uint8_t *base, int32_t bytes)
{
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return (u4w){(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, (uint32_t)max(bytes, 0), 0x00020000u};
}

// LDS DMA of 16 (resp. 4) bytes a lane: lane l's bytes at rsrc + voff land at LDS address lds + 16 l (resp. 4 l).
// From inline assembly, so that the compiler adds no waits of its own; the loop waits for exactly what it needs.
// Nothing else in the kernel uses M0.
__device__ __forceinline__ void dma16(u4w rsrc, uint32_t lds, uint32_t voff)
{
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(lds), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void dma4(u4w rsrc, uint32_t lds, uint32_t voff)
{
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" : : "s"(lds), "v"(voff), "s"(rsrc) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm_lgkm_barrier()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}
__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); }

__device__ __forceinline__ int b_pos(int k, int c) { return c ^ ((k & 7) | (((k >> 4) & 1) << 3)); }

__device__ __forceinline__ uint32_t sad16(v4i v, uint32_t acc)
{
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.x, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.y, 0u, acc);
    acc = __builtin_amdgcn_sad_u8((uint32_t)v.z, 0u, acc);
    return __builtin_amdgcn_sad_u8((uint32_t)v.w, 0u, acc);
}

// Keeps the first n bytes (clamped to 0..16) of a 16-byte fragment, zeroing the rest.
__device__ __forceinline__ v4i keep16(v4i v, int32_t n)
{
    auto m = [](int32_t b) { return b >= 4 ? 0xFFFFFFFFu : (b <= 0 ? 0u : ((1u << (8 * b)) - 1u)); };
    return (v4i){(int32_t)((uint32_t)v.x & m(n)), (int32_t)((uint32_t)v.y & m(n - 4)), (int32_t)((uint32_t)v.z & m(n - 8)),
                 (int32_t)((uint32_t)v.w & m(n - 12))};
}

}  // namespace

// The split of a product into units and workgroups (computed on the host, read by every workgroup).
struct GemvPlan {
    int64_t units;      // batch * slabs * ns
    int32_t slabs, ns;  // column slabs of 256, units of 64 rows of K per slab
    int32_t groups;     // workgroups (one per CU, at most one per unit)
    int32_t maxp;       // parts per slab at most
};

// The workgroup whose run contains unit x (runs are [w U / G, (w + 1) U / G), in integer division).
__host__ __device__ inline int64_t gemv_wg_of(int64_t x, int64_t U, int64_t G) { return ((x + 1) * G - 1) / U; }

template <bool SUM_A, bool SUM_B, bool FLIP_A, bool FLIP_B>
__global__ __launch_bounds__(GS_THREADS) void k_gemv_stream(GemmArgs g, GemvPlan pl, int32_t *parts, uint32_t *counters)
{
    __shared__ __attribute__((aligned(1024))) uint8_t smem[GS_NS * GS_STG];
    __shared__ bool last_flag;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g4 = lane >> 4;
    const int64_t U = pl.units, G = pl.groups, w = blockIdx.x;
    const int64_t u_begin = w * U / G, u_end = (w + 1) * U / G;
    const int32_t cnt = (int32_t)(u_end - u_begin);
    const int32_t M = g.M, N = g.N, K = g.K, lda = g.lda, ldb = g.ldb, ns = pl.ns, slabs = pl.slabs;

    // Loop-invariant DMA offsets. B: load i of this wave fills 1 KB at i * 4 KB + wave * 1 KB of the tile, rows of 256
    // bytes with chunk c of row k at position b_pos(k, c). A: this wave's load fills rows 4 wave .. 4 wave + 3.
    uint32_t off_b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int s = (i * 4 + wave) * 64 + lane, k = s >> 4, p = s & 15;
        off_b[i] = (uint32_t)k * (uint32_t)ldb + 16u * (uint32_t)b_pos(k, p);
    }
    const uint32_t off_a = (uint32_t)(4 * wave + (lane >> 4)) * (uint32_t)lda + 4u * (uint32_t)(lane & 15);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)smem;

    // A position in the run: unit (batch b, slab, stage st), stepped without dividing.
    struct Cursor {
        int32_t b, slab, st;
    };
    Cursor first;
    {
        const int64_t q = u_begin / ns;
        first.st = (int32_t)(u_begin - q * ns);
        first.b = (int32_t)(q / slabs);
        first.slab = (int32_t)(q - (int64_t)first.b * slabs);
    }
    auto step = [&](Cursor &c) {
        if (++c.st == ns) {
            c.st = 0;
            if (++c.slab == slabs) {
                c.slab = 0;
                c.b++;
            }
        }
    };

    // Issues unit j of this workgroup's run (at cursor c) into ring buffer j % GS_NS; j >= cnt loads over empty
    // ranges, so that every wave issues the same count.
    auto issue = [&](int32_t j, const Cursor &c) {
        const uint32_t buf = lds0 + (uint32_t)(j % GS_NS) * GS_STG;
        u4w rb = rsrc_of(g.B, 0), ra = rsrc_of(g.A, 0);
        if (j < cnt) {
            const int32_t k0 = c.st * GS_K, n0 = c.slab * GS_COLS;
            rb = rsrc_of(g.B + c.b * g.strideB + (int64_t)k0 * ldb + n0, (K - 1 - k0) * ldb + min(N - n0, GS_COLS));
            ra = rsrc_of(g.A + c.b * g.strideA + k0, (M - 1) * lda + (K - k0));
        }
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(rb, buf + (uint32_t)(i * 4 + wave) * 1024u, off_b[i]);
        dma4(ra, buf + GS_B + (uint32_t)wave * 256u, off_a);
    };

    // A segment: this workgroup's units of one slab. Sums s t (MFMA layout), this lane's biased byte sums of its
    // columns of B and of its row of A, the units and the rows of K below K it covered.
    struct Seg {
        v4i acc[4];
        uint32_t cs[4], rs;
        int32_t units, kvalid, b, slab;
    };
    auto clear = [](Seg &sg) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sg.acc[j] = (v4i){0, 0, 0, 0};
            sg.cs[j] = 0;
        }
        sg.rs = 0;
        sg.units = 0;
        sg.kvalid = 0;
    };
    Seg cur, held;   // the running segment; a finished one kept in registers until the stream ends
    clear(cur);
    clear(held);
    bool have_held = false;

    // Finishes the slab (b, slab): adds its parts and applies the zero points and the epilogue (the last workgroup).
    // The parts were stored as agent-scope atomics (written through); an acquire fence drops this CU's stale copies
    // (the workspace is reused from call to call), after which plain loads, issued together, see them.
    auto finalize = [&](int32_t b, int32_t slab) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        const int64_t qs = (int64_t)b * slabs + slab;
        const int64_t wf = gemv_wg_of(qs * ns, U, G), wl = gemv_wg_of((qs + 1) * ns - 1, U, G);
        const int32_t np = (int32_t)(wl - wf + 1);
        const int32_t *pp = parts + qs * pl.maxp * GS_PART;
        const int32_t n = slab * GS_COLS + tid, nz = min(n, N - 1);
        // Branch-free, so that the loads issue together: all 16 rows of up to 4 parts at a time (rows past M and parts
        // past the last are read, inside the workspace, and masked off).
        uint32_t v[16], ss[16], st = 0;
#pragma unroll
        for (int m = 0; m < 16; m++) { v[m] = 0; ss[m] = 0; }
        for (int32_t p0 = 0; p0 < np; p0 += 4) {
            uint32_t lv[4][16], ls[4][16], lt[4];
#pragma unroll
            for (int pi = 0; pi < 4; pi++) {
                const int32_t *q = pp + min(p0 + pi, np - 1) * GS_PART;
                lt[pi] = SUM_B ? (uint32_t)q[16 * GS_COLS + tid] : 0u;
#pragma unroll
                for (int m = 0; m < 16; m++) {
                    lv[pi][m] = (uint32_t)q[m * GS_COLS + tid];
                    ls[pi][m] = SUM_A ? (uint32_t)q[16 * GS_COLS + GS_COLS + m] : 0u;
                }
            }
#pragma unroll
            for (int pi = 0; pi < 4; pi++) {
                const uint32_t keep = p0 + pi < np ? 0xFFFFFFFFu : 0u;
                st += lt[pi] & keep;
#pragma unroll
                for (int m = 0; m < 16; m++) {
                    v[m] += lv[pi][m] & keep;
                    ss[m] += ls[pi][m] & keep;
                }
            }
        }
        // Zero points in the signed domain (an absent one's raw byte reads as 0): all rows' loaded together too.
        uint32_t zraw[16], wraw = 0;
#pragma unroll
        for (int m = 0; m < 16; m++) zraw[m] = 0;
        if (SUM_B && g.ZA) {
            const bool per = g.flags & OG_GEMM_ZA_PER_ROW;
#pragma unroll
            for (int m = 0; m < 16; m++) zraw[m] = g.ZA[per ? min(m, M - 1) : 0];
        }
        if (SUM_A && g.ZB) wraw = g.ZB[(g.flags & OG_GEMM_ZB_PER_COL) ? nz : 0];
        const uint32_t wz = !SUM_A ? 0u : (FLIP_B ? wraw - 128u : (uint32_t)sext8(wraw));
        if (n < N) {
#pragma unroll
            for (int m = 0; m < 16; m++) {
                if (m < M) {
                    const uint32_t zz = !SUM_B ? 0u : (FLIP_A ? zraw[m] - 128u : (uint32_t)sext8(zraw[m]));
                    const uint32_t r = v[m] - wz * ss[m] - zz * st + (uint32_t)K * zz * wz;
                    store_value(g, b * g.strideC + (int64_t)m * N + n, n, r);
                }
            }
        }
        if (tid == 0) __hip_atomic_store(&counters[qs], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // Slabs whose parts this workgroup wrote and has not yet counted in (kept until the stream ends, so that the fences
    // of counting in do not drain the loads in flight).
    constexpr int PENDING = 8;
    __shared__ int32_t pend_b[PENDING], pend_slab[PENDING];
    int32_t npend = 0;
    // Counts this workgroup in for every pending slab; the last workgroup of a slab finishes it.
    auto settle = [&]() {
        wait_vm0();   // this wave's part stores acknowledged (and its loads landed)
        __syncthreads();
        for (int32_t e = 0; e < npend; e++) {
            const int32_t b = pend_b[e], slab = pend_slab[e];
            const int64_t qs = (int64_t)b * slabs + slab;
            const int64_t wf = gemv_wg_of(qs * ns, U, G), wl = gemv_wg_of((qs + 1) * ns - 1, U, G);
            if (tid == 0) {
                const uint32_t prev = __hip_atomic_fetch_add(&counters[qs], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_flag = prev == (uint32_t)(wl - wf);
            }
            __syncthreads();
            if (last_flag) finalize(b, slab);
            __syncthreads();
        }
        npend = 0;
    };

    // Writes a finished segment's part (counted in by settle()). Part stores wait in vmcnt in issue order behind the
    // DMA loads and hold up the waits of the stream, so they are left until the stream ends where possible.
    auto put = [](int32_t *p, int32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto write_part = [&](const Seg &sg) {
        const int64_t qs = (int64_t)sg.b * slabs + sg.slab;
        const int64_t wf = gemv_wg_of(qs * ns, U, G);
        int32_t *pp = parts + (qs * pl.maxp + (w - wf)) * GS_PART;
        // Byte sums: the four k-groups of a row / column sit in lanes l, l + 16, l + 32, l + 48. Biased bytes
        // (signed-domain value + 128) were summed; rows of B past K were read as zero, which an unsigned B's biased
        // sum does not count and a signed B's counts as 128.
        const uint32_t nbytes = (uint32_t)sg.units * GS_K;
        if (SUM_B) {
            const uint32_t nb_b = FLIP_B ? (uint32_t)sg.kvalid : nbytes;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t v = sg.cs[j] + (uint32_t)__shfl_xor((int32_t)sg.cs[j], 16);
                v += (uint32_t)__shfl_xor((int32_t)v, 32);
                if (g4 == 0) put(&pp[16 * GS_COLS + wave * 64 + 16 * j + i16], (int32_t)(v - 128u * nb_b));
            }
        }
        if (SUM_A && wave == 0) {
            uint32_t v = sg.rs + (uint32_t)__shfl_xor((int32_t)sg.rs, 16);
            v += (uint32_t)__shfl_xor((int32_t)v, 32);
            if (g4 == 0) put(&pp[16 * GS_COLS + GS_COLS + i16], (int32_t)(v - 128u * nbytes));
        }
        // Sums s t: MFMA 16 x 16 layout, lane l holds rows 4 (l / 16) + r of column l % 16.
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (4 * g4 + r < M) put(&pp[(4 * g4 + r) * GS_COLS + wave * 64 + 16 * j + i16], sg.acc[j][r]);
        if (tid == 0) {
            pend_b[npend] = sg.b;
            pend_slab[npend] = sg.slab;
        }
        npend++;
    };

    // Prologue: units 0 .. GS_NS - 2 in flight.
    Cursor ic = first, cc = first;   // next unit to issue, unit being computed
    for (int32_t j = 0; j < GS_NS - 1; j++) {
        issue(j, ic);
        step(ic);
    }

    for (int32_t j = 0; j < cnt; j++) {
        // Unit j landed (this wave's loads, then everyone's); nobody reads unit j - 1's buffer any more.
        wait_vm_lgkm_barrier<GS_LOADS * (GS_NS - 2)>();
        issue(j + GS_NS - 1, ic);
        step(ic);
        const int32_t st = cc.st, slab = cc.slab, b = cc.b;
        step(cc);
        const int32_t k0 = st * GS_K;
        const uint8_t *tile = smem + (j % GS_NS) * GS_STG;

        // A fragment: row i16, k-group g4; bytes at or past K zeroed in the signed domain.
        v4i a = *reinterpret_cast<const v4i *>(tile + GS_B + i16 * GS_K + 16 * g4);
        if constexpr (FLIP_A) a ^= (int32_t)0x80808080;
        a = keep16(a, K - (k0 + 16 * g4));
        v4i bf[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const int c = wave * 4 + jj;   // 16-byte chunk of the block's columns
            v2i h[2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int k = 16 * g4 + 8 * hh + (i16 >> 1);
                h[hh] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (__attribute__((address_space(3))) v2i *)(tile + k * GS_COLS + 16 * b_pos(k, c) + 8 * (i16 & 1)));
            }
            bf[jj] = (v4i){h[0].x, h[0].y, h[1].x, h[1].y};
            if constexpr (FLIP_B) bf[jj] ^= (int32_t)0x80808080;
        }
#pragma unroll
        for (int jj = 0; jj < 4; jj++) cur.acc[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bf[jj], cur.acc[jj], 0, 0, 0);
        if (SUM_A) cur.rs = sad16(a ^ (int32_t)0x80808080, cur.rs);
        if (SUM_B) {
#pragma unroll
            for (int jj = 0; jj < 4; jj++) cur.cs[jj] = sad16(bf[jj] ^ (int32_t)0x80808080, cur.cs[jj]);
        }
        cur.units++;
        cur.kvalid += min(GS_K, K - k0);
        cur.b = b;
        cur.slab = slab;
        // Last unit of a slab before the end of the run: keep the segment (the first) or write it (later ones).
        if (j < cnt - 1 && st == ns - 1) {
            if (!have_held) {
                held = cur;
                have_held = true;
            } else {
                write_part(cur);
                if (npend == PENDING - 2) settle();   // many short segments: count in now (room stays for two more)
            }
            clear(cur);
        }
    }
    if (have_held) write_part(held);
    if (cnt > 0) write_part(cur);
    settle();   // also waits for every DMA, before the workgroup (and its LDS) goes
}

// The streamed kernel's conditions: B stored K x N with 16-byte aligned rows and N a multiple of 16, A with 4-byte
// aligned rows and K a multiple of 4 (no load straddles the end of a row), each batch's operands under 2^31 bytes, at
// most kGemvMaxSlabs slabs (one counter each).
bool gemv_stream_ok(const GemmArgs &g)
{
    if (g.flags & OG_GEMM_TRANSPOSE_B) return false;
    if (g.M < 1 || g.M > 16 || g.K < 1 || g.N < 1) return false;
    if ((g.N & 15) != 0 || (g.K & 3) != 0) return false;
    if (((g.ldb | g.strideB | (int64_t)(uintptr_t)g.B) & 15) != 0) return false;
    if (((g.lda | g.strideA | (int64_t)(uintptr_t)g.A) & 3) != 0) return false;
    const int64_t lim = 0x7FFFFFFFll;
    if ((int64_t)g.K * g.ldb + GS_COLS > lim || (int64_t)16 * g.lda > lim) return false;
    const int64_t slabs = ((int64_t)g.N + GS_COLS - 1) / GS_COLS;
    return slabs * g.batch <= kGemvMaxSlabs;
}

static GemvPlan gemv_plan(const GemmArgs &g, int32_t cus)
{
    GemvPlan pl{};
    pl.slabs = (g.N + GS_COLS - 1) / GS_COLS;
    pl.ns = (g.K + GS_K - 1) / GS_K;
    pl.units = (int64_t)g.batch * pl.slabs * pl.ns;
    pl.groups = (int32_t)std::min<int64_t>(std::max(cus, 1), pl.units);
    int64_t maxp = 1;
    const int64_t nq = (int64_t)g.batch * pl.slabs;
    for (int64_t q = 0; q < nq; q++) {
        int64_t c = gemv_wg_of((q + 1) * pl.ns - 1, pl.units, pl.groups) - gemv_wg_of(q * pl.ns, pl.units, pl.groups) + 1;
        maxp = c > maxp ? c : maxp;
    }
    pl.maxp = (int32_t)maxp;
    return pl;
}

uint64_t gemv_stream_workspace_bytes(const GemmArgs &g, int32_t cus)
{
    const GemvPlan pl = gemv_plan(g, cus);
    return (uint64_t)g.batch * pl.slabs * pl.maxp * GS_PART * 4;
}

hipError_t launch_gemv_stream(const GemmArgs &g, const Workspace &ws, int32_t cus, hipStream_t s, const char **kernel)
{
    *kernel = "mfma-i8-rows16-stream";
    const GemvPlan pl = gemv_plan(g, cus);
    const bool fa = !(g.flags & OG_GEMM_A_INT8), fb = !(g.flags & OG_GEMM_B_INT8);
    const bool sa = (g.flags & OG_GEMM_ZB) || fb, sb = (g.flags & OG_GEMM_ZA) || fa;
    dim3 grid((uint32_t)pl.groups), block(GS_THREADS);
#define OG_GS(SA, SB, FA, FB) \
    hipLaunchKernelGGL((k_gemv_stream<SA, SB, FA, FB>), grid, block, 0, s, g, pl, ws.partials, ws.gemv_counters)
    if (fa && fb) OG_GS(true, true, true, true);
    else if (fa) { if (sa) OG_GS(true, true, true, false); else OG_GS(false, true, true, false); }
    else if (fb) { if (sb) OG_GS(true, true, false, true); else OG_GS(true, false, false, true); }
    else if (sa && sb) OG_GS(true, true, false, false);
    else if (sa) OG_GS(true, false, false, false);
    else if (sb) OG_GS(false, true, false, false);
    else OG_GS(false, false, false, false);
#undef OG_GS
    return hipGetLastError();
}

}  // namespace og
