"""Shared helpers of the GPU parity tests: the device, uploads, and RunInt32 (Int8Tests.cs:108-172) through the host
layer. Every GPU step prints the case it runs (flushed) first, so a failing run names its case."""
from __future__ import annotations

import atexit
import ctypes
import gc
import sys

import numpy as np

import cases
import oracle
import onegpu_hip as og

_DEVICE = None


def device() -> og.GpuDevice:
    """The one HIP device of the box. Raises (never skips) when there is none: these tests must run the HIP path."""
    global _DEVICE
    if _DEVICE is None:
        _DEVICE = og.GpuDevice.Create(0)
        atexit.register(_release)
    return _DEVICE


def _release() -> None:
    """Waits for the device and drops it before the interpreter shuts down."""
    global _DEVICE
    if _DEVICE is not None:
        _DEVICE.WaitIdle()
        _DEVICE = None
        gc.collect()


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def run(d, record) -> None:
    """Rig.Run: record into a fresh encoder and submit it."""
    e = d.BeginCommands()
    record(e)
    d.Submit(e)


def as_i8(a: np.ndarray) -> np.ndarray:
    """The bytes of a uint8 array as int8, padded to a whole word (Int8Tests.Cast)."""
    pad = np.zeros((a.size + 3) & ~3, np.uint8)
    pad[:a.size] = a
    return pad.view(np.int8)


def as_u8(a: np.ndarray) -> np.ndarray:
    pad = np.zeros((a.size + 3) & ~3, np.uint8)
    pad[:a.size] = a.view(np.uint8)
    return pad


def to_problem(p: oracle.Gemm) -> og.Int8GemmProblem:
    q = og.Int8GemmProblem(p.M, p.N, p.K)
    q.Batch = p.Batch
    q.TransposeB = p.TransposeB
    q.Lda, q.Ldb = p.Lda, p.Ldb
    q.OffsetA, q.OffsetB, q.OffsetC = p.OffsetA, p.OffsetB, p.OffsetC
    q.StrideA, q.StrideB = p.StrideA, p.StrideB
    return q


SENTINEL = 0x5A5A5A5A


def run_int32(d, gemm, c: cases.Case, seed: int, want: np.ndarray | None = None) -> tuple[int, str]:
    """RunInt32: the case's sums through EncodeInt32, sentinel-guarded; returns (mismatches, kernel run)."""
    p = c.p
    data = cases.case_data(c, seed)
    if want is None:
        want = cases.reference_sums(c, data)
    count = want.size
    out = np.full(p.OffsetC + count + 2, SENTINEL, np.int32)
    bc = d.CreateBuffer(out)
    ba = d.CreateBuffer(as_i8(data["a"]) if c.a_signed else as_u8(data["a"]))
    bb = d.CreateBuffer(as_i8(data["b"]) if c.b_signed else as_u8(data["b"]))
    za = zb = None
    if data["za"] is not None:
        za = og.Int8Operand(d.CreateBuffer(as_i8(data["za"]) if c.a_signed else as_u8(data["za"])), 0, c.za_mode == 2)
    if data["zb"] is not None:
        zb = og.Int8Operand(d.CreateBuffer(as_i8(data["zb"]) if c.b_signed else as_u8(data["zb"])), 0, c.zb_mode == 2)
    run(d, lambda e: gemm.EncodeInt32(e, to_problem(p), ba, bb, bc, za, zb))
    got = bc.Read()
    kernel = d.LastKernel
    bad = int(np.count_nonzero(got[p.OffsetC:p.OffsetC + count] != want))
    bad += int(np.count_nonzero(got[:p.OffsetC] != SENTINEL)) + int(np.count_nonzero(got[p.OffsetC + count:] != SENTINEL))
    if bad:
        idx = np.nonzero(got[p.OffsetC:p.OffsetC + count] != want)[0][:6]
        for i in idx:
            say(f"  differs at row {i // max(p.N, 1)} col {i % max(p.N, 1)}: got {got[p.OffsetC + i]} want {want[i]} [{kernel}]")
    return bad, kernel


# The options of each configuration: as chosen, portable, and the test hooks that force each kernel.
CONFIG_OPTIONS = {"default": {}, "portable": {"AllowPackedDot": False}, "tiled only": {"Tile": 64},
                  "split k": {"Tile": 32}, "large tile": {"Tile": 256}}


def configs(d, all_: bool, **extra):
    """Int8Tests.Configs (Int8Tests.cs:23-34); `extra` adds options (FusedRequantize) to every configuration."""
    names = ["default", "portable"] + (["tiled only", "split k", "large tile"] if all_ else [])
    return [(n, og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[n], **extra))) for n in names]


_ABI = None


def abi():
    """The C ABI itself (ctypes), for the calls the host layer does not wrap (benchmark utilities)."""
    global _ABI
    if _ABI is None:
        L = ctypes.CDLL(og.LIB_PATH)

        class Buf(ctypes.Structure):
            _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_uint64)]

        L.Buf = Buf
        L.og_util_scale_product.argtypes = [ctypes.c_void_p, Buf, Buf, ctypes.c_uint32, Buf]
        L.og_util_synth.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32, Buf,
                                    ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double]
        L.og_util_col_absmax_scale.argtypes = [ctypes.c_void_p, Buf, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float, Buf]
        L.og_last_error.argtypes = [ctypes.c_void_p]
        L.og_last_error.restype = ctypes.c_char_p
        L.og_last_kernel.argtypes = [ctypes.c_void_p]
        L.og_last_kernel.restype = ctypes.c_char_p

        class GemmParams(ctypes.Structure):
            _fields_ = [(n, ctypes.c_uint32) for n in (
                "M", "N", "K", "OffA", "OffB", "OffC", "StrideA", "StrideB", "StrideC", "Lda", "Ldb", "Flags", "OffZA",
                "OffZB", "Epi", "OffBias", "OffScale", "OffFBias", "GridX")]

        L.GemmParams = GemmParams
        L.og_int8_gemm.argtypes = [ctypes.c_void_p, ctypes.POINTER(GemmParams), ctypes.c_uint32] + [Buf] * 8
        _ABI = L
    return _ABI


def binding(b: og.GpuBuffer):
    return abi().Buf(b.DevicePointer, b.Size)


def check(status: int, d) -> None:
    if status != 0:
        raise RuntimeError(f"C ABI status {status}: {abi().og_last_error(d.Context).decode()}")
