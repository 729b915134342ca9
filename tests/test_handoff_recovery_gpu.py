"""The one-launch few-rows product ("mfma-i8-rows16-xcd") when its hand-off fails, driven from the host.

og_test_set_spin_limit(ctx, 0) makes each column slab's finishing tile give up at once instead of waiting for the
other parts (every kernel still ends normally; that slab's columns of C are left unwritten). The library must then:
  - report the failure at og_sync (OG_ERR_LAUNCH_FAILED), for the context whose product failed;
  - not let a later one-launch product on the same count words read stale counts: the failed launch poisons the words,
    and a later launch on them (here another context's og_int8_gemm_noalloc on the device's fixed words) reports a
    failure instead of producing sums;
  - clear every count word at og_sync, and run later products in the two-launch form, bit-exact against the oracle.
Each test opens contexts of its own, so the shared device of the other GPU tests keeps its one-launch path."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
import onegpu_hip as og
from gpu_rig import abi, binding, say

pytestmark = pytest.mark.gpu

LAUNCH_FAILED = 5
M, N, K = 1, 11008, 4096           # configuration 3's shape at M = 1: 86 column slabs of 8 k-slices
FLAGS = 0x0A                       # B int8 | OG_GEMM_ZA (a scalar zero point of A); A uint8


def _lib():
    L = abi()
    if not getattr(L, "_recovery_ready", False):
        L.og_int8_gemm_noalloc.argtypes = [ctypes.c_void_p, ctypes.POINTER(L.GemmParams), ctypes.c_uint32] + [L.Buf] * 8
        L.og_int8_gemm_noalloc.restype = ctypes.c_int
        L.og_int8_gemm.restype = ctypes.c_int
        L.og_sync.argtypes = [ctypes.c_void_p]
        L.og_sync.restype = ctypes.c_int
        L.og_test_set_spin_limit.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.og_test_set_spin_limit.restype = ctypes.c_int
        L.og_test_nonzero_words.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_uint64)]
        L.og_test_nonzero_words.restype = ctypes.c_int
        L._recovery_ready = True
    return L


class _Product:
    """Configuration 3's product at M = 1 on one context: operands, the oracle's sums, and the two entry points."""

    def __init__(self, d, seed):
        rng = np.random.default_rng(seed)
        self.d = d
        self.a = rng.integers(0, 256, M * K, dtype=np.uint8)
        self.b = rng.integers(-127, 128, K * N, dtype=np.int8)
        self.za = np.array([rng.integers(0, 256)] * 4, np.uint8)
        self.want = oracle.int8_gemm(oracle.Gemm(M, N, K), self.a, False, self.b.view(np.uint8), True,
                                     (self.za[:1], False, 0))
        self.ba, self.bb, self.bza = d.CreateBuffer(self.a), d.CreateBuffer(self.b), d.CreateBuffer(self.za)
        self.bc = d.CreateBufferOf(og.ElementType.Int32, M * N)
        L = _lib()
        self.prm = L.GemmParams(M=M, N=N, K=K, Lda=K, Ldb=N, Flags=FLAGS)

    def launch(self, noalloc=False):
        """Records the product on the context's stream (no wait); returns the status and the kernel it took."""
        L = _lib()
        none = L.Buf(None, 0)
        fn = L.og_int8_gemm_noalloc if noalloc else L.og_int8_gemm
        st = fn(self.d.Context, ctypes.byref(self.prm), 1, binding(self.ba), binding(self.bb), binding(self.bc),
                binding(self.bza), none, none, none, none)
        return st, L.og_last_kernel(self.d.Context).decode()

    def sync(self):
        return _lib().og_sync(self.d.Context)

    def nonzero_words(self):
        ctx_words, fixed_words = ctypes.c_uint64(0), ctypes.c_uint64(0)
        assert _lib().og_test_nonzero_words(self.d.Context, ctypes.byref(ctx_words), ctypes.byref(fixed_words)) == 0
        return ctx_words.value, fixed_words.value

    def bit_exact(self):
        return np.array_equal(self.bc.Read(), self.want)


def test_give_up_reported_words_cleared_two_launch_form_after():
    L = _lib()
    d = og.GpuDevice.Create(0)
    pr = _Product(d, 71)
    say("recovery: one-launch product before any failure")
    assert pr.launch() == (0, "mfma-i8-rows16-xcd")
    assert pr.sync() == 0 and pr.bit_exact()
    assert pr.nonzero_words() == (0, 0)

    say("recovery: the finishing tiles give up at once (spin limit 0)")
    assert L.og_test_set_spin_limit(d.Context, 0) == 0
    assert pr.launch() == (0, "mfma-i8-rows16-xcd")
    assert pr.sync() == LAUNCH_FAILED
    assert L.og_test_set_spin_limit(d.Context, 1 << 22) == 0
    assert pr.nonzero_words() == (0, 0), "og_sync leaves every count word zero"

    say("recovery: later products on this context take the two-launch form, bit-exact")
    for _ in range(2):
        assert pr.launch() == (0, "mfma-i8-rows16-tiles")
        assert pr.sync() == 0 and pr.bit_exact()
    del pr, d


def test_poisoned_fixed_words_are_reported_by_another_context():
    L = _lib()
    dx, dy = og.GpuDevice.Create(0), og.GpuDevice.Create(0)
    px, py = _Product(dx, 72), _Product(dy, 73)
    say("poison: context X's allocation-free product gives up (spin limit 0)")
    assert L.og_test_set_spin_limit(dx.Context, 0) == 0
    assert px.launch(noalloc=True) == (0, "mfma-i8-rows16-xcd")
    # Waits for X's stream without og_sync (which would clear the words): the fixed words are poisoned now.
    ctx_words, fixed_words = px.nonzero_words()
    say(f"  X's words non-zero: own {ctx_words}, fixed {fixed_words}")
    assert fixed_words >= 1

    say("poison: context Y's allocation-free product finds the words poisoned and reports it at og_sync")
    assert py.launch(noalloc=True) == (0, "mfma-i8-rows16-xcd")
    assert py.sync() == LAUNCH_FAILED
    assert py.nonzero_words() == (0, 0)
    assert py.launch(noalloc=True) == (0, "mfma-i8-rows16-tiles")
    assert py.sync() == 0 and py.bit_exact()

    say("poison: X's own og_sync reports its give-up; X's later products are bit-exact")
    assert px.sync() == LAUNCH_FAILED
    assert L.og_test_set_spin_limit(dx.Context, 1 << 22) == 0
    assert px.nonzero_words() == (0, 0)
    for noalloc in (False, True):
        assert px.launch(noalloc=noalloc) == (0, "mfma-i8-rows16-tiles")
        assert px.sync() == 0 and px.bit_exact()

    say("poison: a fresh context takes the one-launch form again, bit-exact on the cleared words")
    dz = og.GpuDevice.Create(0)
    pz = _Product(dz, 74)
    for noalloc in (False, True):
        assert pz.launch(noalloc=noalloc) == (0, "mfma-i8-rows16-xcd")
        assert pz.sync() == 0 and pz.bit_exact()
    assert pz.nonzero_words() == (0, 0)
    del px, py, pz, dx, dy, dz
