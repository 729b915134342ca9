"""og_int8_gemm_noalloc (the allocation-free entry point) against og_int8_gemm, through the C ABI: the same products
on the same inputs give the same bits, on two calls in a row with the second smaller, on every kernel that takes
scratch (the one-launch and two-launch few-rows kernels, the split-k few-rows kernel, the split-k direct kernel) and
on one that takes none; a product whose scratch exceeds the fixed array is refused before anything runs."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import onegpu_hip as og
from gpu_rig import abi, binding, check, device, say

pytestmark = pytest.mark.gpu

UNSUPPORTED = 2


def _lib():
    L = abi()
    if not getattr(L, "_noalloc_ready", False):
        L.og_int8_gemm_noalloc.argtypes = [ctypes.c_void_p, ctypes.POINTER(L.GemmParams), ctypes.c_uint32] + [L.Buf] * 8
        L.og_int8_gemm_noalloc.restype = ctypes.c_int
        L.og_int8_gemm.restype = ctypes.c_int
        L.og_last_error_argument.argtypes = [ctypes.c_void_p]
        L.og_last_error_argument.restype = ctypes.c_char_p
        L._noalloc_ready = True
    return L


# (label, m, n, k, batch, flags, epi, kernel the product takes)
CASES = [
    ("decode one launch", 4, 11008, 4096, 1, 0x0A, 0x5, "mfma-i8-rows16-xcd"),
    ("decode one launch, smaller", 1, 4096, 2048, 1, 0x0A, 0x5, "mfma-i8-rows16-xcd"),
    ("decode two launches", 16, 4096, 1024, 1, 0x0A | 0x8000, 0x0, "mfma-i8-rows16-tiles"),
    ("decode two launches, smaller", 3, 2048, 512, 1, 0x0A | 0x8000 | 0x20, 0x0, "mfma-i8-rows16-tiles"),
    ("few rows split k", 5, 1000, 2000, 1, 0x0A | 0x20 | 0x40, 0x0, "mfma-i8-rows16-splitk"),
    ("few rows split k, smaller", 2, 500, 1000, 1, 0x0A, 0x0, "mfma-i8-rows16-splitk"),
    ("split k direct", 256, 256, 2304, 1, 0x0A | 0x10, 0x0, "mfma-i8-direct128x128x64-splitk"),
    ("split k direct, smaller", 200, 128, 1536, 1, 0x0A, 0x0, "mfma-i8-direct128x128x64-splitk"),
    ("no scratch", 512, 512, 512, 2, 0x0A, 0x1, "mfma-i8-direct128x128x64"),
    ("no scratch, smaller", 256, 256, 256, 1, 0x0A, 0x0, "mfma-i8-direct128x128x64"),
]


def _run_pair(d, m, n, k, batch, flags, epi, seed):
    """One product through og_int8_gemm and og_int8_gemm_noalloc; returns (reference bits, no-alloc bits, kernel)."""
    L = _lib()
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, batch * m * k, dtype=np.uint8)
    b = rng.integers(-128, 128, batch * k * n, dtype=np.int8)
    za = rng.integers(0, 256, max(m, 4), dtype=np.uint8)
    zb = rng.integers(-8, 9, max(n, 4), dtype=np.int8)
    scale = (rng.random(n, dtype=np.float32) * 1e-3).astype(np.float32)
    ba, bb = d.CreateBuffer(a), d.CreateBuffer(b)
    bza, bzb, bsc = d.CreateBuffer(za), d.CreateBuffer(zb), d.CreateBuffer(scale)
    ety = og.ElementType.Float32 if epi & 1 else og.ElementType.Int32
    c1, c2 = d.CreateBufferOf(ety, batch * m * n), d.CreateBufferOf(ety, batch * m * n)
    prm = L.GemmParams(M=m, N=n, K=k, Lda=k, Ldb=n, Flags=flags, Epi=epi, StrideA=m * k, StrideB=k * n,
                       StrideC=m * n)
    none = L.Buf(None, 0)
    args = [binding(ba), binding(bb), None, binding(bza), binding(bzb), none, binding(bsc) if epi & 1 else none, none]
    check(L.og_int8_gemm(d.Context, ctypes.byref(prm), batch, args[0], args[1], binding(c1), *args[3:]), d)
    d.WaitIdle()
    kernel_ref = L.og_last_kernel(d.Context).decode()
    check(L.og_int8_gemm_noalloc(d.Context, ctypes.byref(prm), batch, args[0], args[1], binding(c2), *args[3:]), d)
    d.WaitIdle()
    kernel = L.og_last_kernel(d.Context).decode()
    assert kernel == kernel_ref, (kernel, kernel_ref)
    return c1.Read().view(np.uint32), c2.Read().view(np.uint32), kernel


@pytest.mark.parametrize("first, second", [(0, 1), (2, 3), (4, 5), (6, 7), (8, 9)])
def test_noalloc_matches_the_allocating_entry_point(first, second):
    d = device()
    for i in (first, second):
        label, m, n, k, batch, flags, epi, want_kernel = CASES[i]
        say(f"noalloc {label}: {batch} x {m}x{n}x{k} flags {flags:#x} epi {epi:#x}")
        ref, got, kernel = _run_pair(d, m, n, k, batch, flags, epi, 40 + i)
        say(f"  {kernel}: {int(np.count_nonzero(ref != got))} differ")
        assert kernel == want_kernel, kernel
        assert np.array_equal(ref, got)


# (label, m, n, k, batch, strideB): products that take the one-launch few-rows kernel ("mfma-i8-rows16-xcd") and need
# more of the fixed array than it holds. Its parts: 86 column slabs x 24 row bands of 17 x 128 + 32 ints (8,832
# bytes) = 18.2 MB, past the 16 MiB array. Its count words: one a column slab and the poison word, 1 + 96 x 86 = 8,257,
# past the 8,192 the array holds (the 96 batch entries share one B, strideB = 0; their parts take 9.5 MB).
REFUSED = [
    ("parts past the array", 16, 11008, 12288, 1, 11008 * 12288),
    ("count words past the array", 1, 11008, 512, 96, 0),
]


@pytest.mark.parametrize("label, m, n, k, batch, stride_b", REFUSED)
def test_noalloc_refuses_a_product_past_its_scratch(label, m, n, k, batch, stride_b):
    # Refused with OG_ERR_UNSUPPORTED (argument "scratch") before any kernel runs.
    d = device()
    L = _lib()
    L.og_int8_gemm_kernel_name.argtypes = [ctypes.POINTER(L.GemmParams), ctypes.c_uint32, ctypes.c_char_p,
                                           ctypes.c_size_t]
    prm = L.GemmParams(M=m, N=n, K=k, Lda=k, Ldb=n, Flags=0x0A, StrideA=m * k, StrideB=stride_b, StrideC=m * n)
    name = ctypes.create_string_buffer(64)
    assert L.og_int8_gemm_kernel_name(ctypes.byref(prm), batch, name, 64) == 0
    assert name.value.decode() == "mfma-i8-rows16-xcd", name.value
    say(f"noalloc refusal, {label}: {batch} x {m}x{n}x{k}")
    ba = d.CreateBuffer(np.zeros(batch * m * k, np.uint8))
    bb = d.CreateBufferOf(og.ElementType.Int8, k * n)
    bc = d.CreateBufferOf(og.ElementType.Int32, batch * m * n)
    bz = d.CreateBuffer(np.full(4, 128, np.uint8))
    none = L.Buf(None, 0)
    st = L.og_int8_gemm_noalloc(d.Context, ctypes.byref(prm), batch, binding(ba), binding(bb), binding(bc),
                                binding(bz), none, none, none, none)
    assert st == UNSUPPORTED
    assert L.og_last_error_argument(d.Context).decode() == "scratch"
    d.WaitIdle()
