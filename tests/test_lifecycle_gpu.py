"""The device lifecycle through the C ABI, after DeviceCycleTests.cs, ConcurrentDeviceTests.cs and MultiDeviceTests.cs
on one GPU: contexts created, used and destroyed many times in a row, by eight threads at once, and two contexts of
one thread used in turn; and four contexts running the one-launch few-rows product at once. Every use allocates its own buffers, runs the closed-form product of MultiDeviceTests.cs:30-55
([[1, 2], [3, 4]] x [[1, -1, 2], [-2, 3, -3]] = [[-3, 5, -4], [-5, 9, -6]]) and a larger seeded one on the MFMA
kernel, and checks both."""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest

import oracle
from gpu_rig import abi, say

pytestmark = pytest.mark.gpu

CLOSED_A = np.array([1, 2, 3, 4], np.uint8)
CLOSED_B = np.array([1, -1, 2, -2, 3, -3, 0, 0], np.int8)   # padded to a whole word
CLOSED_C = [-3, 5, -4, -5, 9, -6]
M, N, K = 96, 160, 256   # the 128 x 128 direct kernel


def _lib():
    L = abi()
    if not hasattr(L, "_lifecycle"):
        vp = ctypes.c_void_p
        L.og_init.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
        L.og_destroy.argtypes = [vp]
        L.og_alloc.argtypes = [vp, ctypes.c_uint64, ctypes.POINTER(vp)]
        L.og_free.argtypes = [vp, vp]
        L.og_memcpy_h2d.argtypes = [vp, vp, vp, ctypes.c_uint64]
        L.og_memcpy_d2h.argtypes = [vp, vp, vp, ctypes.c_uint64]
        L.og_sync.argtypes = [vp]
        L._lifecycle = True
    return L


def _use(L, ctx, seed: int) -> str:
    """One use of a context: the two products, checked; returns '' or what went wrong."""
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, M * K, dtype=np.uint8)
    b = rng.integers(-128, 128, K * N, dtype=np.int8)
    za = np.array([rng.integers(0, 256)], np.uint8)
    want = oracle.int8_gemm(oracle.Gemm(M, N, K), a, False, b, True, (za, False, 0))
    host = [CLOSED_A, CLOSED_B, np.zeros(6, np.int32), a, b, np.zeros(M * N, np.int32), np.zeros(4, np.uint8)]
    host[6][0] = za[0]
    ptrs = []
    try:
        for h in host:
            p = ctypes.c_void_p()
            if L.og_alloc(ctx, h.nbytes, ctypes.byref(p)) != 0:
                return f"og_alloc: {L.og_last_error(ctx).decode()}"
            ptrs.append(p)
            if L.og_memcpy_h2d(ctx, p, h.ctypes.data, h.nbytes) != 0:
                return f"og_memcpy_h2d: {L.og_last_error(ctx).decode()}"
        buf = [L.Buf(p.value, h.nbytes) for p, h in zip(ptrs, host)]
        none = L.Buf(None, 0)
        closed = L.GemmParams(M=2, N=3, K=2, Flags=0x002)
        if L.og_int8_gemm(ctx, ctypes.byref(closed), 1, buf[0], buf[1], buf[2], none, none, none, none, none) != 0:
            return f"closed form: {L.og_last_error(ctx).decode()}"
        big = L.GemmParams(M=M, N=N, K=K, Flags=0x002 | 0x008)   # B int8; A's zero point (scalar)
        if L.og_int8_gemm(ctx, ctypes.byref(big), 1, buf[3], buf[4], buf[5], buf[6], none, none, none, none) != 0:
            return f"product: {L.og_last_error(ctx).decode()}"
        got_c, got_big = np.zeros(6, np.int32), np.zeros(M * N, np.int32)
        if (L.og_memcpy_d2h(ctx, got_c.ctypes.data, ptrs[2], got_c.nbytes) != 0 or
                L.og_memcpy_d2h(ctx, got_big.ctypes.data, ptrs[5], got_big.nbytes) != 0 or L.og_sync(ctx) != 0):
            return f"read back: {L.og_last_error(ctx).decode()}"
        if got_c.tolist() != CLOSED_C:
            return f"closed form gave {got_c.tolist()}"
        bad = int(np.count_nonzero(got_big != want))
        return f"{bad} wrong sums" if bad else ""
    finally:
        for p in ptrs:
            L.og_free(ctx, p)


def _cycle(L, seed: int) -> str:
    ctx = ctypes.c_void_p()
    if L.og_init(0, ctypes.byref(ctx)) != 0:
        return "og_init failed"
    err = _use(L, ctx, seed)
    if L.og_destroy(ctx) != 0:
        return "og_destroy failed"
    return err


def test_contexts_created_used_and_destroyed_in_a_row():
    # DeviceCycleTests.cs: create, use, dispose, over and over (100 cycles here).
    L = _lib()
    for i in range(100):
        err = _cycle(L, 1000 + i)
        assert err == "", f"cycle {i}: {err}"
    say("ROW lifecycle: 100 create / use / destroy cycles, every product exact")


def test_contexts_on_eight_threads_at_once():
    # ConcurrentDeviceTests.cs: 8 threads, each creating, using and destroying its own contexts (20 cycles each).
    L = _lib()
    errors: list[str] = []
    lock = threading.Lock()

    def worker(t: int) -> None:
        for i in range(20):
            err = _cycle(L, 2000 + 100 * t + i)
            if err:
                with lock:
                    errors.append(f"thread {t}, cycle {i}: {err}")
                return

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=100)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert errors == [], errors
    say("ROW lifecycle: 8 threads x 20 cycles, every product exact")


def test_two_contexts_of_one_thread_in_turn():
    # MultiDeviceTests.cs on one GPU: two contexts open together, each with its own stream and workspaces, used
    # alternately; destroying one leaves the other working.
    L = _lib()
    c1, c2 = ctypes.c_void_p(), ctypes.c_void_p()
    assert L.og_init(0, ctypes.byref(c1)) == 0 and L.og_init(0, ctypes.byref(c2)) == 0
    try:
        for i in range(6):
            for ctx in (c1, c2):
                err = _use(L, ctx, 3000 + i)
                assert err == "", f"round {i}: {err}"
        assert L.og_destroy(c1) == 0
        c1 = None
        err = _use(L, c2, 3100)
        assert err == "", err
    finally:
        if c1 is not None:
            L.og_destroy(c1)
        L.og_destroy(c2)


def test_one_launch_few_row_products_on_four_contexts_at_once():
    # Four threads, each with its own context (stream, workspace and count words), run the one-launch few-rows product
    # (its column slabs' parts handed over inside one XCD) back to back while the others do the same: every product
    # exact, every og_sync clean, so no context's hand-off sees another's parts or words.
    L = _lib()
    m, n, k = 4, 4096, 4096
    L.og_last_kernel.restype = ctypes.c_char_p
    rng = np.random.default_rng(77)
    data = []
    for t in range(4):
        a = rng.integers(0, 256, m * k, dtype=np.uint8)
        b = rng.integers(-128, 128, k * n, dtype=np.int8)
        za = np.array([rng.integers(0, 256), 0, 0, 0], np.uint8)
        data.append((a, b, za, oracle.int8_gemm(oracle.Gemm(m, n, k), a, False, b, True, (za[:1], False, 0))))
    errors: list[str] = []
    lock = threading.Lock()

    def worker(t: int) -> None:
        a, b, za, want = data[t]
        ctx = ctypes.c_void_p()
        if L.og_init(0, ctypes.byref(ctx)) != 0:
            with lock:
                errors.append(f"thread {t}: og_init failed")
            return
        ptrs = []
        try:
            host = [a, b, za, np.zeros(m * n, np.int32)]
            for h in host:
                p = ctypes.c_void_p()
                assert L.og_alloc(ctx, h.nbytes, ctypes.byref(p)) == 0
                ptrs.append(p)
                assert L.og_memcpy_h2d(ctx, p, h.ctypes.data, h.nbytes) == 0
            buf = [L.Buf(p.value, h.nbytes) for p, h in zip(ptrs, host)]
            none = L.Buf(None, 0)
            prm = L.GemmParams(M=m, N=n, K=k, Flags=0x002 | 0x008)   # B int8; A's zero point (scalar)
            got = np.zeros(m * n, np.int32)
            for i in range(25):
                st = L.og_int8_gemm(ctx, ctypes.byref(prm), 1, buf[0], buf[1], buf[3], buf[2], none, none, none, none)
                kernel = L.og_last_kernel(ctx).decode()
                if st != 0 or kernel != "mfma-i8-rows16-xcd":
                    raise RuntimeError(f"status {st}, kernel {kernel}")
                if L.og_memcpy_d2h(ctx, got.ctypes.data, ptrs[3], got.nbytes) != 0 or L.og_sync(ctx) != 0:
                    raise RuntimeError(f"sync: {L.og_last_error(ctx).decode()}")
                bad = int(np.count_nonzero(got != want))
                if bad:
                    raise RuntimeError(f"iteration {i}: {bad} wrong sums")
        except Exception as ex:   # noqa: BLE001 - reported below with the thread
            with lock:
                errors.append(f"thread {t}: {ex}")
        finally:
            for p in ptrs:
                L.og_free(ctx, p)
            L.og_destroy(ctx)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=100)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert errors == [], errors
    say("ROW lifecycle: 4 contexts at once x 25 one-launch few-rows products, every product exact, every sync clean")
