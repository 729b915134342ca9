"""GPU parity of DequantizeLinear and QuantizeLinear against the CPU oracle, bit for bit: the reference's
DequantizeTests (tests/RecursiveAI.OneGpu.Kernels.Tests/DequantizeTests.cs), case for case."""
import numpy as np
import pytest

import cases
import oracle
import onegpu_hip as og
from gpu_rig import device, run, say

pytestmark = pytest.mark.gpu

OffX, OffS, OffZ, OffO = 3, 1, 2, 5


def _quantized(dtype, n, seed):
    """DequantizeTests.Quantized<T> (DequantizeTests.cs:8-32)."""
    if dtype == np.int32:
        return oracle.dequant_input_i32(n, seed)
    return oracle.dequant_input_bytes(og.padded_bool_length(max(n, 1)), seed).view(dtype)


def _dequant_case(d, k, dtype, shape, axis, per_axis, with_zero, half, seed):
    """DequantizeTests.Case (DequantizeTests.cs:36-88)."""
    n, axis_len, inner = cases.axis_split(shape, axis, per_axis)
    x = _quantized(dtype, n + OffX, seed)
    scale = oracle.rig_random(axis_len + OffS, seed + 1, 0.001, 2.0)
    zeros = _quantized(dtype, axis_len + OffZ, seed + 2)
    want = oracle.dequantize(x[OffX:OffX + n], scale[OffS:], per_axis, axis_len, inner,
                             zeros[OffZ:OffZ + axis_len] if with_zero else None, f16_out=half)
    length = og.padded_half_length(n + OffO + 1) if half else n + OffO + 1
    sentinel = np.float16(-77) if half else np.float32(-77)
    out = np.full(length, sentinel, np.float16 if half else np.float32)
    bx, bs, bz, bo = d.CreateBuffer(x), d.CreateBuffer(scale), d.CreateBuffer(zeros), d.CreateBuffer(out)
    run(d, lambda e: k.Encode(e, bx, OffX, shape, axis, per_axis, bs, OffS, bz if with_zero else None, OffZ, bo, OffO))
    got = bo.Read()
    gbits = got.view(np.uint16 if half else np.uint32)
    wbits = want.view(np.uint16) if half else want.view(np.uint32)
    bad = int(np.count_nonzero(gbits[OffO:OffO + n] != wbits))
    sbits = np.array([sentinel]).view(np.uint16 if half else np.uint32)[0]
    bad += int(np.count_nonzero(gbits[:OffO] != sbits)) + int(np.count_nonzero(gbits[OffO + n:] != sbits))
    return bad


@pytest.mark.parametrize("dtype,seed0", [(np.uint8, 1), (np.int8, 100), (np.int32, 200)])
def test_dequantize_is_exact(dtype, seed0):
    # DequantizeIsExact (DequantizeTests.cs:113-124)
    d = device()
    k = og.DequantizeKernels(d)
    seed, bad = seed0, 0
    for shape, axis, per_axis in cases.DEQUANT_SHAPES:
        for with_zero in (True, False):
            for half in (False, True):
                say(f"dequantize {np.dtype(dtype).name} {shape} axis {axis} per {per_axis} zero {with_zero} f16 {half}")
                bad += _dequant_case(d, k, dtype, shape, axis, per_axis, with_zero, half, seed)
                seed += 1
    assert bad == 0


def _quant_case(d, k, signed, shape, axis, per_axis, with_zero, half_in, scales, seed):
    """DequantizeTests.QuantizeCase (DequantizeTests.cs:179-255)."""
    n, axis_len, inner = cases.axis_split(shape, axis, per_axis)
    x = oracle.quantize_input(n + OffX, seed, True)
    xh = x.astype(np.float16)
    if half_in:
        x = xh.astype(np.float32)
    scale = np.array([scales[i % len(scales)] for i in range(axis_len + OffS)], np.float32)
    zeros = oracle.dequant_input_bytes(og.padded_bool_length(max(axis_len + OffZ, 1)), seed + 2)
    if signed:
        zeros = zeros.view(np.int8)
    want = oracle.quantize(x[OffX:OffX + n], scale[OffS:], signed, per_axis, axis_len, inner,
                           zeros[OffZ:OffZ + axis_len] if with_zero else None)
    out = np.full(og.padded_bool_length(n + OffO + 3), 177, np.uint8)
    if signed:
        out = out.view(np.int8)
        out[:] = -77
    xin = np.zeros(og.padded_half_length(xh.size), np.float16)
    xin[:xh.size] = xh
    bx = d.CreateBuffer(xin if half_in else x)
    bs, bz, bo = d.CreateBuffer(scale), d.CreateBuffer(zeros), d.CreateBuffer(out)
    run(d, lambda e: k.EncodeQuantize(e, bx, OffX, shape, axis, per_axis, bs, OffS, bz if with_zero else None, OffZ, bo, OffO))
    got = bo.Read().view(np.uint8)
    init = out.view(np.uint8)
    bad = int(np.count_nonzero(got[OffO:OffO + n] != want))
    bad += int(np.count_nonzero(got[:OffO] != init[:OffO])) + int(np.count_nonzero(got[OffO + n:] != init[OffO + n:]))
    return bad


def test_quantize_is_exact():
    # QuantizeIsExact (DequantizeTests.cs:257-289)
    d = device()
    k = og.DequantizeKernels(d)
    bad = count = 0
    seed = 1
    for shape, axis, per_axis in cases.DEQUANT_SHAPES:
        for with_zero in (True, False):
            scales = cases.QUANT_SCALE_SETS[count % len(cases.QUANT_SCALE_SETS)]
            for signed, half_in in ((False, False), (True, False), (False, True), (True, True)):
                say(f"quantize {shape} axis {axis} per {per_axis} zero {with_zero} signed {signed} f16 {half_in}")
                bad += _quant_case(d, k, signed, shape, axis, per_axis, with_zero, half_in, scales, seed)
                seed += 1
                count += 1
    assert bad == 0


def test_dynamic_quantize_golden_fixture():
    # The committed DynamicQuantizeLinear fixture (tests/golden/dq_vectors.npz) on the GPU quantizer, bit for bit.
    import os
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dq_vectors.npz"), allow_pickle=False)
    d = device()
    k = og.DynamicQuantizeKernels(d)
    offs = f["offsets"]
    bad = 0
    for i in range(len(offs) - 1):
        x = f["x"][offs[i]:offs[i + 1]]
        bx, by = d.CreateBuffer(x), d.CreateBufferOf(og.ElementType.UInt8, x.size)
        bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
        run(d, lambda e: k.Encode(e, bx, 0, x.size, by, 0, bs, 0, bz, 0))
        here = int(np.count_nonzero(by.Read()[:x.size] != f["y"][offs[i]:offs[i + 1]]))
        here += int(bs.Read()[0].view(np.uint32) != f["scale"][i].view(np.uint32)) + int(bz.Read()[0] != f["zero"][i])
        if here:
            say(f"MISMATCH dq fixture vector {i}: {here}")
        bad += here
    assert bad == 0
