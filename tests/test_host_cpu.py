"""CPU tests of the boundary: the host layer rejects what the reference rejects (with the same exception and argument),
and the C-ABI library loads, exports every entry point include/onegpu_hip.h declares, and re-validates arguments
itself. No kernel runs here: the host-only device records work but cannot submit it."""
import ctypes
import os
import re

import numpy as np
import pytest

import onegpu_hip as og

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def d():
    return og.GpuDevice.CreateHostOnly()


def buf(d, t, n):
    return d.CreateBufferOf(t, n)


def shape_error(fn, argument=None):
    with pytest.raises(og.GpuKernelShapeException) as ex:
        fn()
    if argument is not None:
        assert ex.value.Argument == argument, str(ex.value)
    return ex.value


def test_int8_gemm_bad_arguments_are_rejected(d):
    # BadArgumentsAreRejected (Int8Tests.cs:549-574), with the argument each rejection names.
    gemm = og.Int8Gemm(d)
    a, b = buf(d, og.ElementType.UInt8, 64), buf(d, og.ElementType.Int8, 64)
    c, f, fl = buf(d, og.ElementType.Int32, 64), buf(d, og.ElementType.Float32, 64), buf(d, og.ElementType.Float32, 1)
    enc = d.BeginCommands()
    P = og.Int8GemmProblem

    def prob(m, n, k, **kw):
        p = P(m, n, k)
        for key, v in kw.items():
            setattr(p, key, v)
        return p

    shape_error(lambda: gemm.EncodeInt32(enc, P(9, 9, 9), a, b, c), "OffsetA")
    shape_error(lambda: gemm.EncodeInt32(enc, P(-1, 2, 2), a, b, c), "M")
    shape_error(lambda: gemm.EncodeInt32(enc, prob(2, 2, 2, Batch=0), a, b, c), "Batch")
    shape_error(lambda: gemm.EncodeInt32(enc, prob(2, 2, 2, Lda=1), a, b, c), "Lda")
    shape_error(lambda: gemm.EncodeInt32(enc, prob(2, 2, 2, OffsetC=62), a, b, c), "c")
    shape_error(lambda: gemm.EncodeInt32(enc, prob(8, 8, 8, OffsetA=1), a, b, c), "OffsetA")
    shape_error(lambda: gemm.EncodeInt32(enc, P(2, 2, 2), a, b, c, og.Int8Operand(a, 63, True)), "zpA")
    shape_error(lambda: gemm.EncodeInt32(enc, P(2, 2, 2), f, b, c), "a")
    shape_error(lambda: gemm.EncodeFloat(enc, P(2, 8, 2), a, b, f, og.Int8Operand(fl, 0, True)), "scale")
    # EncodeFloatScaled (this library's one-launch MatMulIntegerToFloat): EncodeFloat's checks plus a float32
    # activation scale of one element.
    shape_error(lambda: gemm.EncodeFloatScaled(enc, P(2, 8, 2), a, b, f, og.Int8Operand(fl, 0), og.Int8Operand(fl, 0, True)),
                "scale")
    shape_error(lambda: gemm.EncodeFloatScaled(enc, P(2, 8, 2), a, b, f, og.Int8Operand(fl, 1), og.Int8Operand(fl, 0)),
                "activationScale")
    shape_error(lambda: gemm.EncodeFloatScaled(enc, P(2, 8, 2), a, b, f, og.Int8Operand(c, 0), og.Int8Operand(fl, 0)),
                "activationScale")
    ok_enc = d.BeginCommands()
    gemm.EncodeFloatScaled(ok_enc, P(2, 8, 2), a, b, f, og.Int8Operand(fl, 0), og.Int8Operand(f, 0, True))
    assert ok_enc.DispatchCount == 1
    shape_error(lambda: gemm.EncodeRequantized(enc, P(2, 2, 2), a, b, a, og.Int8Operand(fl, 0), 300), "zeroPointY")
    shape_error(lambda: gemm.EncodeRequantized(enc, P(2, 2, 2), a, b, b, og.Int8Operand(fl, 0), 128), "zeroPointY")
    # Further checks of Prepare (Int8Gemm.cs:419-484).
    shape_error(lambda: gemm.EncodeInt32(enc, prob(2, 2, 2, Ldb=1), a, b, c), "Ldb")
    shape_error(lambda: gemm.EncodeInt32(enc, prob(2, 2, 2, StrideA=-1), a, b, c), "StrideA")
    shape_error(lambda: gemm.EncodeInt32(enc, P(2, 2, 2), a, c, c), "b")
    shape_error(lambda: gemm.EncodeInt32(enc, P(2, 2, 2), a, b, f), "c")
    shape_error(lambda: gemm.EncodeInt32(enc, prob(70000, 70000, 1), a, b, c), "Batch")
    assert enc.DispatchCount == 0
    # A valid call records one dispatch; M = 0 records nothing (Int8Gemm.cs:247-250).
    gemm.EncodeInt32(enc, P(2, 2, 2), a, b, c)
    gemm.EncodeInt32(enc, P(0, 2, 2), a, b, c)
    assert enc.DispatchCount == 1
    with pytest.raises(og.GpuUnsupportedException):
        d.Submit(enc)
    # An empty ranged product records a host step (its count reads 0 from there on), not a dispatch: a host-only
    # device runs it.
    ranges = og.Int8Ranges(buf(d, og.ElementType.Float32, 2 * og.OG_RANGES_MAX))
    enc = d.BeginCommands()
    gemm.EncodeFloatRanged(enc, P(0, 8, 2), a, b, f, og.Int8Operand(fl, 0), ranges)
    assert enc.DispatchCount == 0
    d.Submit(enc)
    assert ranges.Groups == 0


def test_scratch_that_is_too_small_is_refused(d):
    # Int8ScratchTests.cs:68-89
    gemm = og.Int8Gemm(d)
    a = d.CreateBuffer(np.zeros(64 * 8 + 4, np.uint8))
    b = d.CreateBuffer(np.zeros(64 * 8 + 4, np.int8))
    y = buf(d, og.ElementType.UInt8, 64 * 64 + 4)
    mult = d.CreateBuffer(np.array([0.001], np.float32))
    small = buf(d, og.ElementType.Int32, 100)
    e = shape_error(lambda: gemm.EncodeRequantized(d.BeginCommands(), og.Int8GemmProblem(64, 64, 8), a, b, y,
                                                   og.Int8Operand(mult, 0), 0, scratch=og.Int8Scratch(small)), "scratch")
    assert e.Operation == "Int8Gemm"
    assert og.Int8Gemm.ScratchElements(og.Int8GemmProblem(160, 96, 64)) == 160 * 96
    assert og.Int8Gemm.ScratchElements(og.Int8GemmProblem(0, 96, 64)) == 0


def test_operands_beyond_one_binding_are_unsupported():
    # CheckBindable (Int8Gemm.cs:402-409), with a device that caps a binding as llvmpipe does (128 MB here 1 KB).
    d = og.GpuDevice.CreateHostOnly(max_binding_bytes=1024)
    gemm = og.Int8Gemm(d)
    a, b = buf(d, og.ElementType.UInt8, 4096), buf(d, og.ElementType.Int8, 64)
    c = buf(d, og.ElementType.Int32, 64)
    with pytest.raises(og.GpuUnsupportedException) as ex:
        gemm.EncodeInt32(d.BeginCommands(), og.Int8GemmProblem(2, 2, 2), a, b, c)
    assert ex.value.Capability == "MaxStorageBufferBindingBytes"


def test_variants(d):
    assert og.Int8Gemm(d, og.Int8GemmOptions(AllowPackedDot=False)).Variant == "portable-tile64x64x16"
    assert og.Int8Gemm(d).Variant == "mfma-i8-gfx950"
    assert og.Int8Gemm(d).BindGroupsCreated == 0


def test_argument_blocks_follow_the_binding_cache_contract(d):
    # BindingCacheTests.cs:141-197 on this backend's argument blocks: a family's first call with a buffer set adds
    # blocks, the same call again adds none, and after ReleaseBindings the same call adds them again (the count is kept);
    # a cache size below 1 is refused. Recording is enough: the count changes when work is recorded, not when it runs.
    f, f2 = buf(d, og.ElementType.Float32, 4096), buf(d, og.ElementType.Float32, 4096)
    u8, i8 = buf(d, og.ElementType.UInt8, 4096), buf(d, og.ElementType.Int8, 4096)
    i32 = buf(d, og.ElementType.Int32, 4096)
    zero = buf(d, og.ElementType.UInt8, 8)
    int8, dq = og.Int8Gemm(d, None, 8), og.DynamicQuantizeKernels(d, 8)
    dequantize, quantizer, gather = og.DequantizeKernels(d, 8), og.DequantizeKernels(d, 8), og.GatherKernels(d, 8)
    conv = og.ConvIntegerKernels(d, None, 8)
    families = [
        ("int8 gemm", lambda e: int8.EncodeInt32(e, og.Int8GemmProblem(16, 16, 16), u8, i8, i32), int8),
        ("dynamic quantize", lambda e: dq.Encode(e, f, 0, 1000, u8, 0, f2, 0, zero, 0), dq),
        ("dequantize", lambda e: dequantize.Encode(e, u8, 0, [16, 16], 0, False, f, 0, None, 0, f2, 0), dequantize),
        ("quantize", lambda e: quantizer.EncodeQuantize(e, f, 0, [16, 16], 0, False, f2, 0, None, 0, u8, 0), quantizer),
        ("gather", lambda e: gather.EncodeGather(e, f, 0, [64, 8], 0, i32, 0, 20, f2, 0), gather),
        ("conv", lambda e: conv.Encode(e, og.ConvProblem(1, 1, 8, 8, 4, 3, 3), u8, i8, i32), conv),
    ]
    for name, record, family in families:
        record(d.BeginCommands())
        first = family.BindGroupsCreated
        record(d.BeginCommands())
        second = family.BindGroupsCreated
        family.ReleaseBindings()
        record(d.BeginCommands())
        third = family.BindGroupsCreated
        assert first > 0 and second == first and third == 2 * first, (name, first, second, third)
    # A new buffer set adds blocks; the cache keeps at most maxCachedBindGroups of them, the least recent dropped.
    small = og.DequantizeKernels(d, 2)
    outs = [buf(d, og.ElementType.Float32, 256) for _ in range(3)]
    rec = lambda o: small.Encode(d.BeginCommands(), u8, 0, [256], 0, False, f, 0, None, 0, o, 0)  # noqa: E731
    for o in outs:
        rec(o)
    assert small.BindGroupsCreated == 3
    rec(outs[2])
    rec(outs[1])
    assert small.BindGroupsCreated == 3
    rec(outs[0])   # dropped when the third set came in
    assert small.BindGroupsCreated == 4
    for make in (lambda: og.Int8Gemm(d, None, 0), lambda: og.DynamicQuantizeKernels(d, 0),
                 lambda: og.DequantizeKernels(d, 0), lambda: og.GatherKernels(d, 0)):
        with pytest.raises((IndexError, ValueError, OverflowError)):
            make()


def test_dynamic_quantize_bad_arguments(d):
    k = og.DynamicQuantizeKernels(d)
    x, y = buf(d, og.ElementType.Float32, 16), buf(d, og.ElementType.UInt8, 16)
    s, z = buf(d, og.ElementType.Float32, 1), buf(d, og.ElementType.UInt8, 4)
    enc = d.BeginCommands()
    shape_error(lambda: k.Encode(enc, x, 0, 0, y, 0, s, 0, z, 0), "count")
    shape_error(lambda: k.Encode(enc, x, 1, 16, y, 0, s, 0, z, 0), "x")
    shape_error(lambda: k.Encode(enc, x, 0, 16, y, 1, s, 0, z, 0), "y")
    shape_error(lambda: k.Encode(enc, x, 0, 16, y, 0, s, 1, z, 0), "scale")
    shape_error(lambda: k.Encode(enc, x, 0, 16, y, 0, s, 0, z, 4), "zeroPoint")
    shape_error(lambda: k.Encode(enc, x, -1, 4, y, 0, s, 0, z, 0), "xOffset")
    k.Encode(enc, x, 0, 16, y, 0, s, 0, z, 3)
    assert enc.DispatchCount == 1


def test_dequantize_bad_arguments(d):
    # DequantizeTests.BadArgumentsAreRejected (DequantizeTests.cs:126-145)
    k = og.DequantizeKernels(d)
    x, s = buf(d, og.ElementType.UInt8, 16), buf(d, og.ElementType.Float32, 4)
    o, big = buf(d, og.ElementType.Float32, 16), buf(d, og.ElementType.UInt32, 16)
    ox = buf(d, og.ElementType.UInt16, 16)
    enc = d.BeginCommands()
    shape_error(lambda: k.Encode(enc, x, 0, [4, 4], 1, True, s, 1, None, 0, o, 0), "scale")
    shape_error(lambda: k.Encode(enc, x, 0, [4, 4], 5, True, s, 0, None, 0, o, 0), "axis")
    shape_error(lambda: k.Encode(enc, x, 8, [4, 4], 0, False, s, 0, None, 0, o, 0), "x")
    shape_error(lambda: k.Encode(enc, big, 0, [4], 0, False, s, 0, None, 0, o, 0), "TIn")
    shape_error(lambda: k.Encode(enc, x, 0, [4], 0, False, s, 0, None, 0, ox, 0), "T")
    shape_error(lambda: k.Encode(enc, x, 0, [-1, 4], 0, False, s, 0, None, 0, o, 0), "shape[0]")


def test_quantize_bad_arguments(d):
    # DequantizeTests.QuantizeRejectsBadArguments (DequantizeTests.cs:291-311)
    k = og.DequantizeKernels(d)
    x, s = buf(d, og.ElementType.Float32, 16), buf(d, og.ElementType.Float32, 4)
    o, o16 = buf(d, og.ElementType.UInt8, 16), buf(d, og.ElementType.Int16, 16)
    xi = buf(d, og.ElementType.Int32, 16)
    enc = d.BeginCommands()
    shape_error(lambda: k.EncodeQuantize(enc, x, 0, [4, 4], 1, True, s, 1, None, 0, o, 0), "scale")
    shape_error(lambda: k.EncodeQuantize(enc, x, 0, [4, 4], 5, True, s, 0, None, 0, o, 0), "axis")
    shape_error(lambda: k.EncodeQuantize(enc, x, 8, [4, 4], 0, False, s, 0, None, 0, o, 0), "x")
    shape_error(lambda: k.EncodeQuantize(enc, x, 0, [4, 4], 0, False, s, 0, None, 0, o, 3), "output")
    shape_error(lambda: k.EncodeQuantize(enc, x, 0, [4], 0, False, s, 0, None, 0, o16, 0), "TOut")
    shape_error(lambda: k.EncodeQuantize(enc, xi, 0, [4], 0, False, s, 0, None, 0, o, 0), "T")


def test_gather_bad_arguments_are_rejected(d):
    # GatherTests.cs:228-258: the rejections EncodeGather makes before recording, with the argument each names.
    k = og.GatherKernels(d)
    data, idx = buf(d, og.ElementType.Float32, 12), buf(d, og.ElementType.Int32, 4)
    outp = buf(d, og.ElementType.Float32, 12)
    enc = d.BeginCommands()
    k.EncodeGather(enc, data, 0, [3, 4], 0, idx, 0, 0, outp, 0)       # no indices: nothing to record
    k.EncodeGather(enc, data, 0, [0, 4], 0, idx, 0, 2, outp, 0)       # an empty axis: valid, every index fails
    assert enc.DispatchCount == 1
    shape_error(lambda: k.EncodeGather(enc, data, 0, [3, 4], 2, idx, 0, 2, outp, 0), "axis")
    shape_error(lambda: k.EncodeGather(enc, data, 0, [3, 4], 0, idx, 3, 2, outp, 0), "indices")
    shape_error(lambda: k.EncodeGather(enc, data, 0, [3, 4], 0, idx, 0, 4, outp, 1), "output")
    shape_error(lambda: k.EncodeGather(enc, data, 0, [3, 4], 0, idx, 0, -1, outp, 0), "indexCount")
    shape_error(lambda: k.EncodeGather(enc, data, 0, [], 0, idx, 0, 1, outp, 0), "dataShape")
    shape_error(lambda: k.EncodeGather(enc, data, 0, [3, 5], 0, idx, 0, 1, outp, 0), "data")
    shape_error(lambda: k.EncodeGather(enc, data, 0, [2147483647, 2], 0, idx, 0, 1, outp, 0))
    shorts = buf(d, og.ElementType.UInt16, 16)
    shape_error(lambda: k.EncodeGather(enc, shorts, 0, [16], 0, idx, 0, 1, shorts, 0), "T")
    # Byte payloads are packed four to a word: a buffer that ends inside a word is refused.
    b18, b20 = buf(d, og.ElementType.UInt8, 18), buf(d, og.ElementType.UInt8, 20)
    assert b18.Size == 20   # CreateBuffer pads bytes to a whole word, but the element count is what is checked
    shape_error(lambda: k.EncodeGather(enc, b18, 0, [1, 18], 0, idx, 0, 1, b20, 0), "data")
    shape_error(lambda: k.EncodeGather(enc, b20, 0, [1, 18], 0, idx, 0, 1, b18, 0), "output")
    floats = buf(d, og.ElementType.Float32, 4)
    shape_error(lambda: k.EncodeGather(enc, data, 0, [3, 4], 0, floats, 0, 1, outp, 0), "TIndex")
    i8 = buf(d, og.ElementType.Int8, 20)
    shape_error(lambda: k.EncodeGather(enc, b20, 0, [20], 0, idx, 0, 1, i8, 0), "output")   # element types differ
    assert enc.DispatchCount == 1


def _conv(batch, cin, h, w, cout, kh, kw, groups=1):
    p = og.ConvProblem(batch, cin, h, w, cout, kh, kw)
    p.Groups = groups
    return p


def test_conv_integer_bad_shapes_throw_typed_errors(d):
    # BadShapesThrowTypedErrors (ConvIntegerTests.cs:309-329), with the argument each names, and the scratch rules of
    # Encode (ConvIntegerKernels.cs:158-185).
    conv = og.ConvIntegerKernels(d)
    x, w = buf(d, og.ElementType.UInt8, 64), buf(d, og.ElementType.Int8, 64)
    y, f = buf(d, og.ElementType.Int32, 64), buf(d, og.ElementType.Float32, 64)
    enc = d.BeginCommands()
    shape_error(lambda: conv.Encode(enc, _conv(1, 3, 4, 4, 4, 3, 3, groups=2), x, w, y), "Groups")
    shape_error(lambda: conv.Encode(enc, _conv(1, 3, 2, 2, 4, 3, 3), x, w, y), "height")
    shape_error(lambda: conv.Encode(enc, _conv(1, 3, 8, 8, 4, 3, 3), x, w, y), "x")          # 192 bytes of x
    shape_error(lambda: conv.Encode(enc, _conv(1, 1, 4, 4, 1, 1, 1), x, w, y, None, og.Int8Operand(w, 64, True)),
                "wZeroPoint")
    shape_error(lambda: conv.Encode(enc, _conv(1, 1, 4, 4, 1, 1, 1), f, w, y), "x")
    shape_error(lambda: conv.Encode(enc, _conv(1, 1, 4, 4, 1, 1, 1), x, w, y, None, None, x, 2), "scratchOffset")
    shape_error(lambda: conv.Encode(enc, _conv(1, 1, 4, 4, 1, 1, 1), x, w, y, None, None, x, 60), "scratch")
    shape_error(lambda: conv.Encode(enc, _conv(1, 1, 4, 4, 1, 1, 1), x, w, y, og.Int8Operand(x, 0, True)), "xZeroPoint")
    shape_error(lambda: conv.Encode(enc, _conv(0, 1, 4, 4, 1, 1, 1), x, w, y), "Batch")
    p = _conv(1, 1, 4, 4, 1, 1, 1)
    p.StrideHeight = 0
    shape_error(lambda: conv.Encode(enc, p, x, w, y), "height stride")
    p = _conv(1, 1, 4, 4, 1, 1, 1)
    p.PadLeft = -1
    shape_error(lambda: conv.Encode(enc, p, x, w, y), "width padding")
    p = _conv(1, 1, 4, 4, 1, 1, 1)
    p.Activation = 1
    shape_error(lambda: conv.Encode(enc, p, x, w, y), "Activation")
    assert enc.DispatchCount == 0
    conv.Encode(enc, _conv(1, 1, 4, 4, 1, 1, 1), x, w, y)
    assert enc.DispatchCount == 1


def test_conv_integer_geometry():
    # ConvProblem.OutHeight / OutWidth (ConvProblem.cs:36-73, 190-206) and the column scratch per image: Groups * K *
    # round16(OutHeight * OutWidth) here (the reference rounds to 4).
    p = og.ConvProblem(2, 4, 9, 11, 5, 3, 3)
    p.StrideHeight = p.StrideWidth = 2
    p.PadTop = p.PadBottom = p.PadLeft = p.PadRight = 1
    assert (p.OutHeight, p.OutWidth) == (5, 6)
    assert og.ConvIntegerKernels.ScratchBytesPerImage(p) == 4 * 9 * 32
    q = og.ConvProblem.Conv1D(1, 80, 3000, 768, 3, padBegin=1, padEnd=1)
    assert (q.Height, q.OutHeight, q.OutWidth) == (1, 1, 3000)
    # K = 240 is padded to 256, with the weights (768 x 256) in rows of 256 ahead of the columns.
    assert og.ConvIntegerKernels.ScratchBytesPerImage(q) == 256 * 3008 + 16 + 768 * 256
    stem = og.ConvProblem(1, 3, 224, 224, 64, 7, 7)
    stem.StrideHeight = stem.StrideWidth = 2
    stem.PadTop = stem.PadBottom = stem.PadLeft = stem.PadRight = 3
    assert (stem.OutHeight, stem.OutWidth) == (112, 112)
    assert og.ConvIntegerKernels.ScratchBytesPerImage(stem) == 192 * 12544 + 16 + 12288   # K = 147 padded to 192
    r = og.ConvProblem(1, 2, 14, 15, 3, 5, 5)
    r.DilationHeight = r.DilationWidth = 2
    r.PadTop = r.PadBottom = r.PadLeft = r.PadRight = 4
    assert (r.OutHeight, r.OutWidth) == (14, 15)
    g = og.ConvProblem(2, 6, 9, 10, 6, 3, 3)
    g.Groups = 6
    assert og.ConvIntegerKernels.ScratchBytesPerImage(g) == 6 * 9 * 64


# ------------------------------------------------------------------ the C ABI


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "onegpu_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(og_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(og.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 25, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


class Buf(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_uint64)]


class GemmParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("M", "N", "K", "OffA", "OffB", "OffC", "StrideA", "StrideB", "StrideC",
                                               "Lda", "Ldb", "Flags", "OffZA", "OffZB", "Epi", "OffBias", "OffScale",
                                               "OffFBias", "GridX")]


class DequantParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("Count", "OffX", "OffO", "OffS", "OffZ", "GridX", "Flags", "AxisLen",
                                               "Inner")]


def test_dequantize_batch_validates_before_touching_a_device():
    # og_dequantize_batch: every pass checked as og_dequantize checks one; the passes must share count, flags and axis,
    # and no pass's output may meet another pass's operands (they run together). Host addresses stand in for device
    # ones: nothing is dereferenced.
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_dequantize_batch.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_uint32,
                                        ctypes.POINTER(DequantParams)] + [ctypes.POINTER(Buf)] * 4
    lib.og_last_error_argument.restype = ctypes.c_char_p
    lib.og_last_error_argument.argtypes = [ctypes.c_void_p]
    host = (ctypes.c_uint8 * 65536)()
    addr = ctypes.addressof(host)
    n, cols = 3, 16

    def call(params, outs=None, xs=None):
        k = len(params)
        P = (DequantParams * k)(*params)
        X = (Buf * k)(*(xs or [Buf(addr + 1024 * i, 256) for i in range(k)]))
        S = (Buf * k)(*[Buf(addr + 8192 + 256 * i, 64) for i in range(k)])
        Z = (Buf * k)(*[Buf(None, 0)] * k)
        O = (Buf * k)(*(outs or [Buf(addr + 16384 + 1024 * i, 256) for i in range(k)]))
        st = lib.og_dequantize_batch(None, 2, 0, k, P, X, S, Z, O)   # int32 -> float32
        return st, lib.og_last_error_argument(None).decode()

    good = DequantParams(Count=64, Flags=1, AxisLen=cols, Inner=1)
    assert call([good] * n) == (6, "ctx")                                                    # valid: no device
    assert call([good, DequantParams(Count=60, Flags=1, AxisLen=cols, Inner=1), good])[1] == "params"
    assert call([good, DequantParams(Count=64, Flags=0), good])[1] == "params"
    assert call([good] * n, outs=[Buf(addr + 16384, 256)] * n)[1] == "output"                # one output for all
    assert call([good] * 2, outs=[Buf(addr + 16384, 256), Buf(addr, 256)])[1] == "output"   # pass 1 writes pass 0's x
    assert call([good] * 2, outs=[Buf(addr + 16384, 256), Buf(addr + 1024, 256)]) == (6, "ctx")   # in place: its own
    assert call([good] * n, xs=[Buf(addr, 255)] + [Buf(addr + 1024, 256)] * 2)[1] == "x"     # x one byte short
    assert call([good] * 300)[1] == "n"


def test_abi_validates_before_touching_a_device():
    # The C ABI re-checks ranges itself: with no context it reports the bad argument, or, when every argument is
    # valid, that there is no device. Host addresses stand in for device ones: nothing is dereferenced.
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_int8_gemm.argtypes = [ctypes.c_void_p, ctypes.POINTER(GemmParams), ctypes.c_uint32] + [Buf] * 8
    lib.og_last_error_argument.restype = ctypes.c_char_p
    lib.og_last_error_argument.argtypes = [ctypes.c_void_p]
    lib.og_last_error.restype = ctypes.c_char_p
    lib.og_last_error.argtypes = [ctypes.c_void_p]
    host = (ctypes.c_uint8 * 4096)()
    addr = ctypes.addressof(host)
    none = Buf(None, 0)

    def call(p, a=64, b=64, c=256, batch=1, **kw):
        bufs = dict(A=Buf(addr, a), B=Buf(addr, b), C=Buf(addr, c), ZA=none, ZB=none, bias=none, scale=none, fbias=none)
        bufs.update(kw)
        st = lib.og_int8_gemm(None, ctypes.byref(p), batch, *bufs.values())
        return st, lib.og_last_error_argument(None).decode()

    p = GemmParams(M=4, N=4, K=4, Lda=4, Ldb=4, StrideC=16)
    assert call(p) == (6, "ctx")                                  # valid: no device
    assert call(p, a=15) == (1, "OffsetA")                        # A one byte short
    assert call(p, b=15) == (1, "OffsetB")
    assert call(p, c=63) == (1, "c")
    assert call(GemmParams(M=4, N=4, K=4, Lda=3, Ldb=4))[1] == "Lda"
    assert call(GemmParams(M=4, N=4, K=4, Flags=0x08))[1] == "zpA"  # zero point flagged but absent
    assert call(GemmParams(M=4, N=4, K=4, Epi=0x1))[1] == "scale"
    assert call(GemmParams(M=4, N=4, K=4, Epi=0x4))[1] == "Epi"
    assert call(GemmParams(M=4, N=4, K=4, Flags=0x10000))[1] == "Flags"
    assert call(p, batch=0)[1] == "Batch"
    assert call(GemmParams(M=0x80000000, N=1, K=1))[1] == "M"
    st, _ = call(GemmParams(M=4, N=4, K=4, Flags=0x08 | 0x10), ZA=Buf(addr, 3))
    assert lib.og_last_error_argument(None).decode() == "zpA"

    # The one-launch requantized product: Y counts bytes (no alignment), the multiplier is required, the output zero
    # point lies in the output type's range, and Epi holds only the int bias and per-column bits.
    lib.og_int8_gemm_requantized.argtypes = ([ctypes.c_void_p, ctypes.POINTER(GemmParams), ctypes.c_uint32] + [Buf] * 7
                                             + [ctypes.c_int32, ctypes.c_uint32])

    def rq(p, y=16, mult=4, zero=0, signed=0, **kw):
        bufs = dict(A=Buf(addr, 64), B=Buf(addr, 64), Y=Buf(addr + 1, y), ZA=none, ZB=none, bias=none,
                    mult=Buf(addr, mult))
        bufs.update(kw)
        st = lib.og_int8_gemm_requantized(None, ctypes.byref(p), 1, *bufs.values(), zero, signed)
        return st, lib.og_last_error_argument(None).decode()

    assert rq(p) == (6, "ctx")                                    # 16 bytes at an odd address: valid
    assert rq(p, y=15) == (1, "y")
    assert rq(GemmParams(M=4, N=4, K=4, OffC=1)) == (1, "y")      # 16 bytes from byte 1 of a 16-byte buffer
    assert rq(p, mult=0) == (1, "multiplier")
    assert rq(GemmParams(M=4, N=4, K=4, Epi=0x4), mult=12) == (1, "multiplier")   # per column: 4 floats
    assert rq(GemmParams(M=4, N=4, K=4, Epi=0x4), mult=16) == (6, "ctx")
    assert rq(GemmParams(M=4, N=4, K=4, Epi=0x1)) == (1, "Epi")   # a float result is not a requantized one
    assert rq(p, zero=256) == (1, "zeroPointY")
    assert rq(p, zero=-1) == (1, "zeroPointY")
    assert rq(p, zero=-128, signed=1) == (6, "ctx")
    assert rq(p, zero=128, signed=1) == (1, "zeroPointY")
    assert rq(GemmParams(M=4, N=4, K=4, Epi=0x2))[1] == "bias"

    # The one-launch MatMulIntegerToFloat: a float result whose column scale takes the activation scale.
    lib.og_int8_gemm_float_scaled.argtypes = ([ctypes.c_void_p, ctypes.POINTER(GemmParams), ctypes.c_uint32] + [Buf] * 7
                                              + [ctypes.c_uint32, Buf, Buf])

    def fs(p, act=4, act_off=0, **kw):
        bufs = dict(A=Buf(addr, 64), B=Buf(addr, 64), C=Buf(addr, 64), ZA=none, ZB=none, bias=none)
        st = lib.og_int8_gemm_float_scaled(None, ctypes.byref(p), 1, *bufs.values(), Buf(addr, act), act_off,
                                           kw.get("scale", Buf(addr, 16)), none)
        return st, lib.og_last_error_argument(None).decode()

    pf = GemmParams(M=4, N=4, K=4, Epi=0x1 | 0x4)
    assert fs(pf) == (6, "ctx")
    assert fs(GemmParams(M=4, N=4, K=4)) == (1, "Epi")           # an int32 result has no scale
    assert fs(pf, act=0) == (1, "activationScale")
    assert fs(pf, act=8, act_off=2) == (1, "activationScale")
    assert fs(pf, act=8, act_off=1) == (6, "ctx")
    assert fs(pf, scale=Buf(addr, 12)) == (1, "scale")


class GatherParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("Count", "OffData", "OffOut", "OffIdx", "GridX", "Flags", "Inner",
                                               "IdxCount", "AxisLen")]


def test_gather_abi_validates_before_touching_a_device():
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_gather.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(GatherParams), Buf, Buf, Buf, Buf]
    lib.og_last_error_argument.restype = ctypes.c_char_p
    lib.og_last_error_argument.argtypes = [ctypes.c_void_p]
    host = (ctypes.c_uint8 * 4096)()
    addr = ctypes.addressof(host)

    def call(p, eb=1, data=64, idx=64, out=64, status=Buf(None, 0)):
        st = lib.og_gather(None, eb, ctypes.byref(p), Buf(addr, data), Buf(addr, idx), Buf(addr, out), status)
        return st, lib.og_last_error_argument(None).decode()

    # data [2, 8, 3] bytes gathered on axis 1 with 4 int32 indices: output [2, 4, 3] = 24 bytes.
    p = GatherParams(Count=24, Inner=3, IdxCount=4, AxisLen=8)
    assert call(p) == (6, "ctx")
    assert call(p, data=47) == (1, "data")          # 2 * 8 * 3 = 48 bytes
    assert call(p, idx=15) == (1, "indices")
    assert call(p, out=23) == (1, "output")
    assert call(p, eb=4, data=192, out=95) == (1, "output")
    assert call(p, eb=3) == (1, "T")
    assert call(GatherParams(Count=25, Inner=3, IdxCount=4, AxisLen=8)) == (1, "Count")
    assert call(GatherParams(Count=24, Inner=3, IdxCount=4, AxisLen=8, Flags=1), idx=31) == (1, "indices")
    assert call(GatherParams(Count=24, Inner=3, IdxCount=4, AxisLen=8, Flags=2)) == (1, "Flags")
    assert call(p, status=Buf(addr + 1, 4)) == (1, "status")
    assert call(GatherParams(Count=0, Inner=3, IdxCount=0, AxisLen=8), data=0, idx=0, out=0) == (6, "ctx")


class ConvParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "Batch", "InChannels", "Height", "Width", "OutChannels", "KernelHeight", "KernelWidth", "StrideHeight",
        "StrideWidth", "DilationHeight", "DilationWidth", "PadTop", "PadLeft", "PadBottom", "PadRight", "Groups",
        "OffsetX", "OffsetW", "OffsetY", "Flags", "OffXZero", "OffWZero", "GemmFlags")]


def test_conv_abi_validates_before_touching_a_device():
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_conv_integer.argtypes = [ctypes.c_void_p, ctypes.POINTER(ConvParams)] + [Buf] * 6 + [ctypes.c_uint64]
    lib.og_conv_integer_scratch_bytes.argtypes = [ctypes.POINTER(ConvParams)]
    lib.og_conv_integer_scratch_bytes.restype = ctypes.c_uint64
    lib.og_last_error_argument.restype = ctypes.c_char_p
    lib.og_last_error_argument.argtypes = [ctypes.c_void_p]
    host = (ctypes.c_uint8 * 65536)()
    addr = ctypes.addressof(host)
    none = Buf(None, 0)
    base = dict(Batch=2, InChannels=4, Height=6, Width=6, OutChannels=8, KernelHeight=3, KernelWidth=3, StrideHeight=1,
                StrideWidth=1, DilationHeight=1, DilationWidth=1, PadTop=1, PadLeft=1, PadBottom=1, PadRight=1, Groups=1)

    def call(x=288, w=288, y=2304, xz=none, wz=none, scratch=4 * 9 * 48, off=0, **kw):
        p = ConvParams(**{**base, **kw})
        st = lib.og_conv_integer(None, ctypes.byref(p), Buf(addr, x), Buf(addr, w), Buf(addr, y), xz, wz,
                                 Buf(addr, scratch) if scratch else none, off)
        return st, lib.og_last_error_argument(None).decode()

    assert lib.og_conv_integer_scratch_bytes(ctypes.byref(ConvParams(**base))) == 36 * 48   # K = 36, ldb = 48
    assert call() == (6, "ctx")
    assert call(x=287) == (1, "x")
    assert call(w=287) == (1, "w")
    assert call(y=2303) == (1, "y")
    assert call(scratch=36 * 48 - 1) == (1, "scratch")
    assert call(off=2, scratch=4096) == (1, "scratchOffset")
    assert call(Groups=3) == (1, "Groups")
    assert call(KernelHeight=9) == (1, "height")
    assert call(Flags=0x4) == (1, "xZeroPoint")
    assert call(Flags=0x8 | 0x10, wz=Buf(addr, 7)) == (1, "wZeroPoint")
    assert call(Flags=0x10) == (1, "Flags")
    assert call(GemmFlags=0x1) == (1, "GemmFlags")
    # One input channel a group (depthwise): no scratch needed; through the column matrix it is.
    assert call(InChannels=8, Groups=8, x=576, w=72, scratch=0) == (6, "ctx")
    assert call(InChannels=8, Groups=8, x=576, w=72, scratch=0, Flags=0x20) == (1, "scratch")
    # A 1 x 1 window with unit strides and no padding over rows of 16-byte multiples multiplies x as it lies: no
    # scratch either (6 x 6 = 36-byte rows are packed; 8 x 8 = 64-byte rows are not).
    pw = dict(KernelHeight=1, KernelWidth=1, PadTop=0, PadLeft=0, PadBottom=0, PadRight=0)
    aligned = (addr + 15) & ~15
    st = lib.og_conv_integer(None, ctypes.byref(ConvParams(**{**base, **pw, "Height": 8, "Width": 8})),
                             Buf(aligned, 512), Buf(addr, 288), Buf(addr, 4096), none, none, none, 0)
    assert (st, lib.og_last_error_argument(None).decode()) == (6, "ctx")
    assert call(scratch=0, **pw)[1] == "scratch"


def test_kernel_choice_is_reported():
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_int8_gemm_kernel_name.argtypes = [ctypes.POINTER(GemmParams), ctypes.c_uint32, ctypes.c_char_p, ctypes.c_size_t]
    out = ctypes.create_string_buffer(64)

    def name(**kw):
        lib.og_int8_gemm_kernel_name(ctypes.byref(GemmParams(**kw)), 1, out, 64)
        return out.value.decode()

    assert name(M=4096, N=4096, K=4096) == "mfma-i8-direct256x256x64"
    assert name(M=256, N=256, K=64) == "mfma-i8-direct128x128x64"
    assert name(M=256, N=256, K=96) == "mfma-i8-tile128x128x128"          # K % 64 != 0: register-staged
    assert name(M=256, N=256, K=64, Ldb=260) == "mfma-i8-tile128x128x128"   # rows of B 4-byte aligned only
    assert name(M=256, N=256, K=64, Lda=72) == "mfma-i8-generic128x128x64"  # rows of A 8-byte aligned only
    assert name(M=256, N=256, K=64, Flags=0x2000) == "mfma-i8-direct256x256x64"
    assert name(M=1, N=11008, K=4096) == "mfma-i8-rows16-xcd"             # 43 slabs: one launch
    assert name(M=1, N=11008, K=4096, Flags=0x8000) == "mfma-i8-rows16-tiles"   # OG_GEMM_TWO_PASS
    assert name(M=1, N=1536, K=768) == "mfma-i8-rows16-tiles"             # 12 slabs of 128: under two an XCD
    assert name(M=16, N=4096, K=4096) == "mfma-i8-rows16-xcd"
    assert name(M=1, N=11008, K=4100) == "mfma-i8-rows16-splitk"          # K % 16 != 0: not tiled
    assert name(M=1, N=11008, K=4096, Flags=0x4000) == "mfma-i8-rows16-splitk"
    assert name(M=1, N=11000, K=4096) == "mfma-i8-rows16-splitk"          # N % 16 != 0: not tiled
    assert name(M=16, N=11008, K=4096).startswith("mfma-i8-rows16")
    # Transposed B takes the tiled kernels; 86 tiles of 128 over 64 stages of K split into 3 slices.
    assert name(M=1, N=11008, K=4096, Flags=0x4) == "mfma-i8-direct128x128x64-splitk"
    assert name(M=256, N=256, K=2304) == "mfma-i8-direct128x128x64-splitk"   # 4 tiles, 36 stages
    assert name(M=1024, N=3072, K=768) == "mfma-i8-direct128x128x64"          # 192 tiles: no split
    assert name(M=2048, N=3072, K=768) == "mfma-i8-direct128x128x64"          # 384 tiles: two workgroups a CU
    assert name(M=256, N=256, K=448) == "mfma-i8-direct128x128x64"            # 7 stages: too short to split
    assert name(M=1, N=11008, K=4096, Flags=0x400) == "portable-tile64x64x16"


class DqParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("Count", "OffX", "OffY", "GridX", "Groups", "OffScale", "OffZero")]


def test_ranged_entry_points_validate_before_touching_a_device():
    # og_int8_gemm_float_ranged and og_dynamic_quantize_ranged (the quantize pass over a ranged product's output):
    # the float result bit, a ranges buffer of OG_RANGES_MAX pairs, a dense C, a groups count in range. With no context
    # a valid call reports that there is no device. Host addresses stand in for device ones: nothing is dereferenced.
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_int8_gemm_float_ranged.argtypes = ([ctypes.c_void_p, ctypes.POINTER(GemmParams), ctypes.c_uint32] +
                                              [Buf] * 7 + [ctypes.c_uint32, Buf, Buf, Buf,
                                                           ctypes.POINTER(ctypes.c_uint32)])
    lib.og_dynamic_quantize_ranged.argtypes = [ctypes.c_void_p, ctypes.POINTER(DqParams)] + [Buf] * 5 + [ctypes.c_uint32]
    lib.og_last_error_argument.restype = ctypes.c_char_p
    lib.og_last_error_argument.argtypes = [ctypes.c_void_p]
    host = (ctypes.c_uint8 * 65536)()
    addr = ctypes.addressof(host)
    none = Buf(None, 0)
    assert og.OG_RANGES_MAX == 1024
    ranges_ok = Buf(addr + 32768, 8 * og.OG_RANGES_MAX)
    groups = ctypes.c_uint32(7)

    def gemm(epi=0x1 | 0x4, batch=1, stride_c=0, ranges=ranges_ok, act=none, g=ctypes.byref(groups)):
        # 4 x 8 x 16 product, A u8, B i8, float result with a per-column scale
        p = GemmParams(M=4, N=8, K=16, Flags=0x2, Epi=epi, StrideA=64, StrideB=128, StrideC=stride_c)
        st = lib.og_int8_gemm_float_ranged(None, ctypes.byref(p), batch, Buf(addr, 256), Buf(addr, 512),
                                           Buf(addr + 1024, 512), none, none, none, act, 0, Buf(addr + 2048, 64),
                                           none, ranges, g)
        return st, lib.og_last_error_argument(None).decode()

    assert gemm() == (6, "ctx")
    assert gemm(epi=0) == (1, "Epi")                                  # an int32 product has no range
    assert gemm(ranges=Buf(addr + 32768, 8 * og.OG_RANGES_MAX - 8)) == (1, "ranges")
    assert gemm(ranges=Buf(addr + 32772, 8 * og.OG_RANGES_MAX)) == (1, "ranges")   # not 8-byte aligned
    assert gemm(batch=2, stride_c=40) == (1, "StrideC")               # C must be dense
    assert gemm(batch=2, stride_c=32) == (6, "ctx")
    assert gemm(g=None) == (1, "groups")
    assert gemm(act=Buf(addr + 3072, 4)) == (6, "ctx")                # with the activation scale (scaled form)

    def quant(count=64, groups_=5, ranges=ranges_ok):
        p = DqParams(Count=count)
        st = lib.og_dynamic_quantize_ranged(None, ctypes.byref(p), Buf(addr, 4 * count), Buf(addr + 8192, count),
                                            Buf(addr + 12288, 4), Buf(addr + 12292, 4), ranges, groups_)
        return st, lib.og_last_error_argument(None).decode()

    assert quant() == (6, "ctx")
    assert quant(groups_=0) == (1, "groups")
    assert quant(groups_=og.OG_RANGES_MAX + 1) == (1, "groups")
    assert quant(groups_=og.OG_RANGES_MAX) == (6, "ctx")
    assert quant(ranges=Buf(addr + 32768, 64)) == (1, "ranges")
    assert quant(count=0) == (1, "count")


def test_stream_tiles_validates_before_touching_a_device():
    # og_util_stream_tiles (the streaming floor of the one-launch few-rows product): N a multiple of 16, B 16-byte
    # aligned and holding K x N bytes, a 4-byte sink. With no context a valid call reports that there is no device.
    lib = ctypes.CDLL(og.LIB_PATH)
    lib.og_util_stream_tiles.argtypes = [ctypes.c_void_p, Buf, ctypes.c_uint32, ctypes.c_uint32, Buf]
    lib.og_last_error_argument.restype = ctypes.c_char_p
    lib.og_last_error_argument.argtypes = [ctypes.c_void_p]
    host = (ctypes.c_uint8 * 8192)()
    addr = (ctypes.addressof(host) + 15) & ~15

    def stream(k=64, n=64, b=None, sink=None):
        b = Buf(addr, 4096) if b is None else b
        sink = Buf(addr + 4096, 4) if sink is None else sink
        st = lib.og_util_stream_tiles(None, b, k, n, sink)
        return st, lib.og_last_error_argument(None).decode()

    assert stream() == (6, "ctx")
    assert stream(n=72) == (1, "K")                        # N not a multiple of 16
    assert stream(k=0) == (1, "K")
    assert stream(k=65) == (1, "B")                        # 65 x 64 bytes reach past the 4 KB buffer
    assert stream(b=Buf(addr + 4, 4096)) == (1, "B")       # not 16-byte aligned
    assert stream(sink=Buf(addr + 4096, 2)) == (1, "sink")
