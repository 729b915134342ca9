"""Batched products whose later batch entries start past 2^31 and 2^32 bytes into A and B, through the C ABI (the
host layer's buffers hold at most 2^31 - 1 elements, as the reference's GpuBuffer<T> does, so only the ABI reaches
these sizes): every product kernel must form each batch entry's operand addresses in 64 bits. The bytes between the
entries hold a fill pattern, so an address that wrapped would read it and give wrong sums. Checked against the oracle
entry by entry, bit for bit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from gpu_rig import abi, check, device, say

pytestmark = pytest.mark.gpu

STRIDE = 3 << 29   # 1.5 GiB between batch entries: entry 2 starts 3 GiB in, entry 3 4.5 GiB in
BATCH = 4
REGION = 4 << 20   # room for the largest entry below
A_INT8, B_INT8, TRANS_B, ZA, ZA_ROW, ZB, ZB_COL = 0x1, 0x2, 0x4, 0x8, 0x10, 0x20, 0x40
PORTABLE, NO_SKINNY, LARGE_TILE, TWO_PASS = 0x400, 0x800, 0x2000, 0x8000

# (label, m, n, k, flags, the kernel the product takes)
CASES = [
    ("direct 128", 128, 256, 256, B_INT8 | ZA | ZA_ROW, "mfma-i8-direct128x128x64"),
    ("direct 128 split along K", 128, 128, 2048, B_INT8 | ZA, "mfma-i8-direct128x128x64-splitk"),
    ("direct 256, both zero points", 256, 256, 256, ZA | ZB | ZB_COL | NO_SKINNY | LARGE_TILE,
     "mfma-i8-direct256x256x64"),
    ("direct 256 ping-pong", 256, 256, 256, B_INT8 | ZA | ZA_ROW | NO_SKINNY | LARGE_TILE, "mfma-i8-direct256x256x64"),
    ("direct 256, B stored N x K", 256, 256, 256, B_INT8 | TRANS_B | ZA | NO_SKINNY | LARGE_TILE,
     "mfma-i8-direct256x256x64"),
    ("register-staged tile", 64, 64, 208, A_INT8 | ZA | ZB, "mfma-i8-tile128x128x128"),
    ("generic, unaligned rows", 64, 64, 200, ZA | ZB | ZB_COL, "mfma-i8-generic128x128x64"),
    ("few rows, one launch", 2, 2048, 1024, B_INT8 | ZA, "mfma-i8-rows16-xcd"),
    ("few rows, two launches", 2, 2048, 1024, B_INT8 | ZA | TWO_PASS, "mfma-i8-rows16-tiles"),
    ("few rows split k", 3, 1000, 2000, B_INT8 | ZA | ZB, "mfma-i8-rows16-splitk"),
    ("few rows, one k slice", 2, 1000, 64, B_INT8 | ZA | ZB, "mfma-i8-rows16-direct"),
    ("portable", 64, 64, 256, A_INT8 | ZA | ZB | ZB_COL | PORTABLE, "portable-tile64x64x16"),
]


class _Big:
    """Two device buffers of 3 x STRIDE + REGION bytes (A and B), filled with 0xC3, held for the module."""

    def __init__(self, d):
        L = abi()
        L.og_alloc.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p)]
        L.og_free.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.og_memcpy_h2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
        L.og_memcpy_d2h.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
        L.og_fill_bytes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint8, ctypes.c_uint64]
        self.L, self.d = L, d
        self.bytes = (BATCH - 1) * STRIDE + REGION
        self.ptrs = []
        for _ in range(2):
            p = ctypes.c_void_p()
            check(L.og_alloc(d.Context, self.bytes, ctypes.byref(p)), d)
            self.ptrs.append(p.value)
            check(L.og_fill_bytes(d.Context, p.value, 0xC3, self.bytes), d)

    def put(self, which: int, offset: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data.view(np.uint8))
        assert offset + data.size <= self.bytes
        check(self.L.og_memcpy_h2d(self.d.Context, self.ptrs[which] + offset, data.ctypes.data, data.size), self.d)

    def free(self) -> None:
        for p in self.ptrs:
            self.L.og_free(self.d.Context, p)
        self.ptrs = []


@pytest.fixture(scope="module")
def big():
    b = _Big(device())
    yield b
    b.free()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_batch_entries_past_4_gib(big, case):
    label, m, n, k, flags, want_kernel = case
    d = device()
    L = big.L
    trans = bool(flags & TRANS_B)
    lda, ldb = k, (k if trans else n)
    rows_b = n if trans else k
    assert m * lda <= REGION and rows_b * ldb <= REGION
    rng = np.random.default_rng(7000 + m + n + k)
    a_dt = np.int8 if flags & A_INT8 else np.uint8
    b_dt = np.int8 if flags & B_INT8 else np.uint8
    za = rng.integers(0, 256, max(m, 4), dtype=np.uint8)
    zb = rng.integers(0, 256, max(n, 4), dtype=np.uint8)
    say(f"offsets past 4 GiB: {label} {BATCH} x {m}x{n}x{k} flags {flags:#x}")
    want = []
    for bt in range(BATCH):
        a = rng.integers(0, 256, m * lda, dtype=np.uint8)
        b = rng.integers(0, 256, rows_b * ldb, dtype=np.uint8)
        big.put(0, bt * STRIDE, a)
        big.put(1, bt * STRIDE, b)
        p = oracle.Gemm(m, n, k, TransposeB=trans)
        p.Lda, p.Ldb = lda, ldb
        zpa = (za, bool(flags & ZA_ROW), 0) if flags & ZA else None
        zpb = (zb, bool(flags & ZB_COL), 0) if flags & ZB else None
        want.append(oracle.int8_gemm(p, a.view(a_dt), bool(flags & A_INT8), b.view(b_dt), bool(flags & B_INT8), zpa,
                                     zpb))
    want = np.concatenate(want)
    c = d.CreateBuffer(np.full(BATCH * m * n + 2, 0x5A5A5A5A, np.int32))
    bza, bzb = d.CreateBuffer(za), d.CreateBuffer(zb)
    prm = L.GemmParams(M=m, N=n, K=k, Lda=lda, Ldb=ldb, Flags=flags, StrideA=STRIDE, StrideB=STRIDE, StrideC=m * n)
    none = L.Buf(None, 0)
    check(L.og_int8_gemm(d.Context, ctypes.byref(prm), BATCH, L.Buf(big.ptrs[0], big.bytes),
                         L.Buf(big.ptrs[1], big.bytes), L.Buf(c.DevicePointer, c.Size),
                         L.Buf(bza.DevicePointer, bza.Size) if flags & ZA else none,
                         L.Buf(bzb.DevicePointer, bzb.Size) if flags & ZB else none, none, none, none), d)
    d.WaitIdle()   # also reports a one-launch few-rows product whose parts never arrived
    kernel = L.og_last_kernel(d.Context).decode()
    got = c.Read()
    bad = int(np.count_nonzero(got[:BATCH * m * n] != want)) + int(np.count_nonzero(got[BATCH * m * n:] != 0x5A5A5A5A))
    say(f"ROW offsets past 4 GiB | {label} | {kernel} | mismatches {bad}")
    assert kernel == want_kernel, kernel
    assert bad == 0
