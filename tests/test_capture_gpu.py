"""Graph capture of the library's stream (og_stream): a product whose workspace would have to grow is refused while
the stream is being captured (the allocation could not be part of the graph, and a replay must not find its memory
freed), with OG_ERR_INVALID_ARG naming "workspace"; once one product of that size has run, the same product captures,
and every replay of the graph, with the program's own work between replays, gives the eager result."""
import ctypes

import numpy as np
import pytest

import onegpu_hip as og
from gpu_rig import abi, binding, say

pytestmark = pytest.mark.gpu

OG_ERR_INVALID_ARG = 1
CAPTURE_RELAXED = 2


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_char_p, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    return hip


def test_workspace_growth_is_refused_during_capture_and_captured_products_replay():
    d = og.GpuDevice.Create(0)   # a context of its own: its workspace still has the initial size
    L, hip = abi(), _hip()
    L.og_stream.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    L.og_last_error_argument.argtypes = [ctypes.c_void_p]
    L.og_last_error_argument.restype = ctypes.c_char_p
    L.og_fill_bytes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint8, ctypes.c_uint64]
    ctx = ctypes.c_void_p(d.Context)
    stream = ctypes.c_void_p()
    assert L.og_stream(ctx, ctypes.byref(stream)) == 0
    # A few-rows product whose k-slices' parts need 36 MB of workspace (16 rows, 256 slabs x 16 k-slices of 8832
    # bytes) against the 32 MiB a context starts with.
    M, N, K = 16, 32768, 8192
    a = d.CreateBufferOf(og.ElementType.UInt8, M * K)
    b = d.CreateBufferOf(og.ElementType.Int8, K * N)
    c = d.CreateBufferOf(og.ElementType.Int32, M * N)
    for buf, t, lo, hi in ((a, 0, 0, 255), (b, 1, -127, 127)):
        assert L.og_util_synth(ctx, 0, 11, t, binding(buf), 0, buf.Size, lo, hi) == 0
    p = L.GemmParams(M=M, N=N, K=K, Lda=K, Ldb=N, Flags=0x2)   # u8 A, int8 B
    none = L.Buf(None, 0)
    args = (ctx, ctypes.byref(p), 1, binding(a), binding(b), binding(c), none, none, none, none, none)

    say("capture: a product that needs a larger workspace")
    assert hip.hipStreamBeginCapture(stream, CAPTURE_RELAXED) == 0
    st = L.og_int8_gemm(*args)
    graph = ctypes.c_void_p()
    assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
    if graph.value:
        hip.hipGraphDestroy(graph)
    assert st == OG_ERR_INVALID_ARG, L.og_last_error(ctx)
    assert L.og_last_error_argument(ctx) == b"workspace"
    assert b"captured" in L.og_last_error(ctx)

    say("eager: the workspace grows and the product runs")
    assert L.og_int8_gemm(*args) == 0
    d.WaitIdle()
    want = c.Read().copy()
    assert np.count_nonzero(want) > 0

    say("capture again: nothing grows, the product is recorded")
    assert hip.hipStreamBeginCapture(stream, CAPTURE_RELAXED) == 0
    st = L.og_int8_gemm(*args)
    graph = ctypes.c_void_p()
    assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
    assert st == 0, L.og_last_error(ctx)
    exe = ctypes.c_void_p()
    assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
    try:
        for rep in range(3):
            say(f"replay {rep}")
            assert L.og_fill_bytes(ctx, c.DevicePointer, 0, c.Size) == 0   # the program's own work between replays
            d.WaitIdle()
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            d.WaitIdle()   # og_sync also reports a one-launch product whose hand-off did not complete
            got = c.Read()
            assert np.array_equal(got, want), f"replay {rep}: {int(np.count_nonzero(got != want))} values differ"
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
