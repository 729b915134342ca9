"""numpy front end of the CPU oracle (oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as the checker:
the product (the HIP library and its host layer) never loads it.

Each wrapper keeps the name and argument meaning of the C function it calls; oracle.c cites the reference file:line
each one restates. The gather (byte and element copies, no arithmetic) is restated here in numpy.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> str:
    """Compiles oracle.c with its Makefile (gcc, -ffp-contract=off) and returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F = ctypes.c_float


class Problem(ctypes.Structure):
    """ora_problem: Int8GemmProblem's fields (src/RecursiveAI.OneGpu.Kernels/Int8Gemm.cs:43-95)."""

    _fields_ = [(n, ctypes.c_int32) for n in
                ("M", "N", "K", "Batch", "TransposeB", "Lda", "Ldb", "OffsetA", "OffsetB", "OffsetC", "StrideA", "StrideB")]


def _declare(L):
    L.ora_bytes.argtypes = [_P, _I64, _I32]
    L.ora_rig_random.argtypes = [_P, _I64, _I32, _F, _F]
    L.ora_dq_input.argtypes = [_P, _I64, _I32, _I32]
    L.ora_dequant_input_i32.argtypes = [_P, _I64, _I32]
    L.ora_dequant_input_bytes.argtypes = [_P, _I64, _I32]
    L.ora_quantize_input.argtypes = [_P, _I64, _I32, _I32]
    L.ora_splitmix64.argtypes = [_U64]
    L.ora_splitmix64.restype = _U64
    L.ora_synth_uniform_i32.argtypes = [_P, _I64, _U64, ctypes.c_uint32, _I32, _I32]
    L.ora_synth_normal_f32.argtypes = [_P, _I64, _U64, ctypes.c_uint32, _F, _F]
    gemm_args = [ctypes.POINTER(Problem), _P, _I32, _P, _I32, _P, _I32, _I32, _P, _I32, _I32]
    L.ora_int8_gemm.argtypes = gemm_args + [_P, _I32]
    L.ora_int8_gemm_identity.argtypes = gemm_args + [_P]
    L.ora_int8_gemm_rows.argtypes = gemm_args + [_P, _I64, _P, _I32]
    L.ora_float_epilogue.argtypes = [_P, _I64, _I32, _P, _P, _I32, _P, _P]
    L.ora_conv_integer.argtypes = [_P, _P, _I32, _P, _I32, _P, _P, _I32, _P, _I32]
    L.ora_requant.argtypes = [_I32, _F, _I32, _I32]
    L.ora_requant.restype = _I32
    L.ora_requant_array.argtypes = [_P, _I64, _I32, _P, _P, _I32, _I32, _I32, _P]
    L.ora_dynamic_quantize.argtypes = [_P, _I64, _P, _P, _P]
    L.ora_div_exact.argtypes = [_F, _F]
    L.ora_div_exact.restype = _F
    L.ora_f2h.argtypes = [_F]
    L.ora_f2h.restype = ctypes.c_uint16
    L.ora_h2f.argtypes = [ctypes.c_uint16]
    L.ora_h2f.restype = _F
    L.ora_dequantize.argtypes = [_I32, _P, _I64, _I32, _I64, _I64, _P, _P, _I32, _P, _P]
    L.ora_quantize_one.argtypes = [_F, _F, _I32, _I32, _I32]
    L.ora_quantize_one.restype = _I32
    L.ora_quantize.argtypes = [_P, _I64, _I32, _I64, _I64, _P, _P, _I32, _P]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ generators

def bytes_(length: int, seed: int) -> np.ndarray:
    """Int8Tests.Bytes (tests/RecursiveAI.OneGpu.Kernels.Tests/Int8Tests.cs:36-47)."""
    out = np.empty(max(length, 0), np.uint8)
    lib().ora_bytes(_ptr(out), length, seed)
    return out


def rig_random(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    """Rig.Random (tests/RecursiveAI.OneGpu.Kernels.Tests/Rig.cs:8-19)."""
    out = np.empty(n, np.float32)
    lib().ora_rig_random(_ptr(out), n, seed, lo, hi)
    return out


def dq_input(count: int, seed: int, kind: int) -> np.ndarray:
    """The DynamicQuantizeLinear test inputs (Int8Tests.cs:633-647)."""
    out = np.empty(count, np.float32)
    lib().ora_dq_input(_ptr(out), count, seed, kind)
    return out


def dequant_input_i32(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().ora_dequant_input_i32(_ptr(out), n, seed)
    return out


def dequant_input_bytes(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().ora_dequant_input_bytes(_ptr(out), n, seed)
    return out


def quantize_input(n: int, seed: int, special: bool) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ora_quantize_input(_ptr(out), n, seed, int(special))
    return out


def synth_uniform_i32(n: int, seed: int, tensor: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().ora_synth_uniform_i32(_ptr(out), n, seed, tensor, lo, hi)
    return out


def synth_normal_f32(n: int, seed: int, tensor: int, mean: float, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ora_synth_normal_f32(_ptr(out), n, seed, tensor, mean, std)
    return out


# ------------------------------------------------------------------ the product

@dataclass
class Gemm:
    """One int8 product with its operands as numpy byte arrays (the raw bytes of the buffers)."""

    M: int
    N: int
    K: int
    Batch: int = 1
    TransposeB: bool = False
    Lda: int = 0
    Ldb: int = 0
    OffsetA: int = 0
    OffsetB: int = 0
    OffsetC: int = 0
    StrideA: int = 0
    StrideB: int = 0

    def c_problem(self) -> Problem:
        return Problem(self.M, self.N, self.K, self.Batch, int(self.TransposeB), self.Lda, self.Ldb, self.OffsetA,
                       self.OffsetB, self.OffsetC, self.StrideA, self.StrideB)


def _zp(z):
    """(bytes, is_vector, offset) or None -> the C argument triple."""
    if z is None:
        return None, 0, 0
    buf, vec, off = z
    return _c(buf.view(np.uint8) if buf.dtype != np.uint8 else buf, np.uint8), int(vec), int(off)


def int8_gemm(p: Gemm, a, a_signed, b, b_signed, za=None, zb=None, threads: int = 8) -> np.ndarray:
    """Definition form (Int8Tests.cs:52-82): dense int32 [Batch*M*N]. za/zb are (bytes, is_vector, offset)."""
    a = _c(a.view(np.uint8), np.uint8)
    b = _c(b.view(np.uint8), np.uint8)
    zab, zav, zao = _zp(za)
    zbb, zbv, zbo = _zp(zb)
    c = np.zeros(max(p.Batch * p.M * p.N, 0), np.int32)
    pr = p.c_problem()
    lib().ora_int8_gemm(ctypes.byref(pr), _ptr(a), int(a_signed), _ptr(b), int(b_signed), _ptr(zab), zav, zao,
                        _ptr(zbb), zbv, zbo, _ptr(c), threads)
    return c


def int8_gemm_identity(p: Gemm, a, a_signed, b, b_signed, za=None, zb=None) -> np.ndarray:
    """Signed-domain identity form (Int8GemmDot.hlsl:1-11, 134-140)."""
    a = _c(a.view(np.uint8), np.uint8)
    b = _c(b.view(np.uint8), np.uint8)
    zab, zav, zao = _zp(za)
    zbb, zbv, zbo = _zp(zb)
    c = np.zeros(max(p.Batch * p.M * p.N, 0), np.int32)
    pr = p.c_problem()
    lib().ora_int8_gemm_identity(ctypes.byref(pr), _ptr(a), int(a_signed), _ptr(b), int(b_signed), _ptr(zab), zav,
                                 zao, _ptr(zbb), zbv, zbo, _ptr(c))
    return c


def int8_gemm_rows(p: Gemm, a, a_signed, b, b_signed, rows, za=None, zb=None, threads: int = 8) -> np.ndarray:
    """The definition-form sums of the given rows (indices over Batch*M): int32 [len(rows), N]."""
    a = _c(a.view(np.uint8), np.uint8)
    b = _c(b.view(np.uint8), np.uint8)
    zab, zav, zao = _zp(za)
    zbb, zbv, zbo = _zp(zb)
    rows = _c(rows, np.int64)
    c = np.zeros((len(rows), p.N), np.int32)
    pr = p.c_problem()
    lib().ora_int8_gemm_rows(ctypes.byref(pr), _ptr(a), int(a_signed), _ptr(b), int(b_signed), _ptr(zab), zav, zao,
                             _ptr(zbb), zbv, zbo, _ptr(rows), len(rows), _ptr(c), threads)
    return c


def float_epilogue(sums, n, scale, scale_vec, ibias=None, fbias=None) -> np.ndarray:
    """MatMulIntegerToFloat's float steps (Int8Tests.cs:356-373)."""
    sums = _c(sums, np.int32)
    scale = _c(scale, np.float32)
    ibias = _c(ibias, np.int32)
    fbias = _c(fbias, np.float32)
    out = np.empty(sums.size, np.float32)
    lib().ora_float_epilogue(_ptr(sums), sums.size, n, _ptr(ibias), _ptr(scale), int(scale_vec), _ptr(fbias), _ptr(out))
    return out


def requant(acc: int, mult: float, zero: int, unsigned: bool) -> int:
    """Int8Tests.Requant (Int8Tests.cs:84-97)."""
    return lib().ora_requant(acc, mult, zero, int(unsigned))


def requant_array(sums, n, mult, mult_vec, zero, unsigned, ibias=None) -> np.ndarray:
    sums = _c(sums, np.int32)
    mult = _c(mult, np.float32)
    ibias = _c(ibias, np.int32)
    out = np.empty(sums.size, np.uint8)
    lib().ora_requant_array(_ptr(sums), sums.size, n, _ptr(ibias), _ptr(mult), int(mult_vec), zero, int(unsigned),
                            _ptr(out))
    return out


# ------------------------------------------------------------------ quantizers

def dynamic_quantize(x) -> tuple[np.ndarray, np.float32, int]:
    """DynamicReference (Int8Tests.cs:576-615): (y, scale, zero point)."""
    x = _c(x, np.float32)
    y = np.empty(x.size, np.uint8)
    s = np.zeros(1, np.float32)
    z = np.zeros(1, np.uint8)
    lib().ora_dynamic_quantize(_ptr(x), x.size, _ptr(y), _ptr(s), _ptr(z))
    return y, s[0], int(z[0])


def div_exact(x: float, s: float) -> np.float32:
    return np.float32(lib().ora_div_exact(x, s))


def f2h(f: float) -> int:
    return lib().ora_f2h(f)


def h2f(h: int) -> np.float32:
    return np.float32(lib().ora_h2f(h))


_KIND = {np.dtype(np.uint8): 0, np.dtype(np.int8): 1, np.dtype(np.int32): 2}


def dequantize(x, scale, per_axis=False, axis_len=1, inner=1, zero=None, f16_out=False) -> np.ndarray:
    """DequantizeLinear (DequantizeTests.cs:67-74). x is u8, i8 or i32; returns float32, or binary16 bits as uint16."""
    kind = _KIND[np.dtype(x.dtype)]
    x = np.ascontiguousarray(x)
    zero = None if zero is None else np.ascontiguousarray(zero, dtype=x.dtype)
    scale = _c(scale, np.float32)
    count = x.size
    out32 = None if f16_out else np.empty(count, np.float32)
    out16 = np.empty(count, np.uint16) if f16_out else None
    lib().ora_dequantize(kind, _ptr(x), count, int(per_axis), axis_len, inner, _ptr(scale), _ptr(zero), int(f16_out),
                         _ptr(out32), _ptr(out16))
    return out16 if f16_out else out32


def quantize_one(x: float, scale: float, zero: int, lo: int, hi: int) -> int:
    return lib().ora_quantize_one(x, scale, zero, lo, hi)


def quantize(x, scale, is_signed, per_axis=False, axis_len=1, inner=1, zero=None) -> np.ndarray:
    """QuantizeLinear (DequantizeTests.cs:147-157): returns the output bytes (int8 values as their uint8 bits)."""
    x = _c(x, np.float32)
    scale = _c(scale, np.float32)
    zero = None if zero is None else np.ascontiguousarray(zero).view(np.uint8)
    out = np.empty(x.size, np.uint8)
    lib().ora_quantize(_ptr(x), x.size, int(per_axis), axis_len, inner, _ptr(scale), _ptr(zero), int(is_signed),
                       _ptr(out))
    return out


# ------------------------------------------------------------------ gather

def gather(data, shape, axis, indices, wide=False):
    """ONNX Gather along one axis as Gather.hlsl:25-43 with IndexCommon.hlsli:12-43 computes it and GatherTests.cs:8-68
    checks it. The data (any element dtype, dense row-major) is [outer, axisLen, inner] around `axis`;
    out[o, i, n] = data[o, idx[i], n], a negative index counting from the end of the axis. An index outside
    [-axisLen, axisLen), or, with int64 indices (`wide`), one that does not fit an int32, reads nothing: its output
    elements are zero. Returns (the flat output [outer * count * inner], the smallest invalid position or None)."""
    shape = [int(x) for x in shape]
    rank = len(shape)
    ax = axis + rank if axis < 0 else axis
    outer = int(np.prod(shape[:ax], dtype=np.int64))
    inner = int(np.prod(shape[ax + 1:], dtype=np.int64))
    n_axis = shape[ax]
    v = np.asarray(indices).astype(np.int64).ravel()
    valid = (v >= -n_axis) & (v < n_axis)
    if wide:
        valid &= (v >= -(1 << 31)) & (v < (1 << 31))
    norm = np.where(v < 0, v + n_axis, v)
    d3 = np.asarray(data).reshape(outer, n_axis, inner)
    out = np.zeros((outer, v.size, inner), d3.dtype)
    if valid.any():
        out[:, valid, :] = d3[:, norm[valid], :]
    bad = np.flatnonzero(~valid)
    return out.reshape(-1), (int(bad[0]) if bad.size else None)


# ------------------------------------------------------------------ ConvInteger

class _Conv(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("Batch", "InChannels", "Height", "Width", "OutChannels", "KernelHeight", "KernelWidth", "StrideHeight",
                 "StrideWidth", "DilationHeight", "DilationWidth", "PadTop", "PadLeft", "Groups", "OutHeight",
                 "OutWidth")]


def conv_out_extent(inp: int, kernel: int, stride: int, dilation: int, pad_begin: int, pad_end: int) -> int:
    """GpuWindow.OutputExtent without auto padding or ceil mode (ConvProblem.cs:36-73): floor of the padded span
    over the stride, plus one; 0 when the dilated kernel does not fit."""
    effective = dilation * (kernel - 1) + 1
    span = inp + pad_begin + pad_end - effective
    return 0 if span < 0 else span // stride + 1


def conv_integer(conv: dict, x, x_signed, w, w_signed, xz=None, wz=None, wz_vec=False, threads: int = 8) -> np.ndarray:
    """ConvIntegerTests.Reference (ConvIntegerTests.cs:42-89): int32 [Batch, OutChannels, OutHeight, OutWidth], flat.
    `conv` holds the ConvProblem fields (PadBottom / PadRight only enter the output extent); x and w start at their
    first element (the caller applies OffsetX / OffsetW)."""
    c = dict(StrideHeight=1, StrideWidth=1, DilationHeight=1, DilationWidth=1, PadTop=0, PadLeft=0, PadBottom=0,
             PadRight=0, Groups=1)
    c.update(conv)
    oh = conv_out_extent(c["Height"], c["KernelHeight"], c["StrideHeight"], c["DilationHeight"], c["PadTop"], c["PadBottom"])
    ow = conv_out_extent(c["Width"], c["KernelWidth"], c["StrideWidth"], c["DilationWidth"], c["PadLeft"], c["PadRight"])
    fields = [f for f, _ in _Conv._fields_ if f not in ("OutHeight", "OutWidth")]
    pr = _Conv(**{f: int(c[f]) for f in fields}, OutHeight=oh, OutWidth=ow)
    x = _c(np.asarray(x).view(np.uint8), np.uint8)
    w = _c(np.asarray(w).view(np.uint8), np.uint8)
    xzb = None if xz is None else _c(np.asarray(xz).view(np.uint8), np.uint8)
    wzb = None if wz is None else _c(np.asarray(wz).view(np.uint8), np.uint8)
    y = np.zeros(c["Batch"] * c["OutChannels"] * oh * ow, np.int32)
    lib().ora_conv_integer(ctypes.byref(pr), _ptr(x), int(x_signed), _ptr(w), int(w_signed), _ptr(xzb), _ptr(wzb),
                           int(wz_vec), _ptr(y), threads)
    return y
