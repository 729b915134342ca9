"""GPU parity of DequantizeLinear and QuantizeLinear against the CPU oracle, bit for bit: the reference's
DequantizeTests (tests/RecursiveAI.OneGpu.Kernels.Tests/DequantizeTests.cs), case for case."""
import numpy as np
import pytest

import cases
import oracle
import onegpu_hip as og
from gpu_rig import device, run, say

pytestmark = pytest.mark.gpu

# Element offsets of x, scale, zero point and output: the reference's (every tensor unaligned, so each element moves on
# its own), and all zero (16-byte aligned starts: a thread's 16 elements move with vector loads and stores).
UNALIGNED, ALIGNED = (3, 1, 2, 5), (0, 0, 0, 0)


def run_named(d, record) -> list:
    """Records one pass with a timing pair around each dispatch and returns the dispatches' kernel names."""
    e = d.BeginCommands()
    e.BeginPassTiming(1)
    record(e)
    e.EndPassTiming()
    d.Submit(e)
    d.WaitIdle()
    return [k for _, k in d.ReadPassTimes()]


def _quantized(dtype, n, seed):
    """DequantizeTests.Quantized<T> (DequantizeTests.cs:8-32)."""
    if dtype == np.int32:
        return oracle.dequant_input_i32(n, seed)
    return oracle.dequant_input_bytes(og.padded_bool_length(max(n, 1)), seed).view(dtype)


def _dequant_case(d, k, dtype, shape, axis, per_axis, with_zero, half, seed, offs=UNALIGNED):
    """DequantizeTests.Case (DequantizeTests.cs:36-88)."""
    OffX, OffS, OffZ, OffO = offs
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
    names = run_named(d, lambda e: k.Encode(e, bx, OffX, shape, axis, per_axis, bs, OffS, bz if with_zero else None, OffZ,
                                             bo, OffO))
    want_kernel = ("dequantize4-" if offs == ALIGNED else "dequantize-") + ("f16" if half else "f32")
    assert names == [want_kernel], names
    got = bo.Read()
    gbits = got.view(np.uint16 if half else np.uint32)
    wbits = want.view(np.uint16) if half else want.view(np.uint32)
    bad = int(np.count_nonzero(gbits[OffO:OffO + n] != wbits))
    sbits = np.array([sentinel]).view(np.uint16 if half else np.uint32)[0]
    bad += int(np.count_nonzero(gbits[:OffO] != sbits)) + int(np.count_nonzero(gbits[OffO + n:] != sbits))
    return bad


@pytest.mark.parametrize("offs", [UNALIGNED, ALIGNED], ids=["unaligned", "aligned"])
@pytest.mark.parametrize("dtype,seed0", [(np.uint8, 1), (np.int8, 100), (np.int32, 200)])
def test_dequantize_is_exact(dtype, seed0, offs):
    # DequantizeIsExact (DequantizeTests.cs:113-124), at the reference's offsets and at aligned ones
    d = device()
    k = og.DequantizeKernels(d)
    seed, bad = seed0, 0
    for shape, axis, per_axis in cases.DEQUANT_SHAPES + cases.DEQUANT_SHAPES_BLOCKS:
        for with_zero in (True, False):
            for half in (False, True):
                say(f"dequantize {np.dtype(dtype).name} {shape} axis {axis} per {per_axis} zero {with_zero} f16 {half} "
                    f"offsets {offs}")
                bad += _dequant_case(d, k, dtype, shape, axis, per_axis, with_zero, half, seed, offs)
                seed += 1
    assert bad == 0


@pytest.mark.parametrize("offs", [UNALIGNED, ALIGNED], ids=["unaligned", "aligned"])
@pytest.mark.parametrize("dtype,seed0", [(np.uint8, 3001), (np.int8, 3100), (np.int32, 3200)])
def test_batched_dequantize_is_exact(dtype, seed0, offs):
    # The cases of DequantizeIsExact, each as three passes of one shape with their own buffers recorded together, so
    # that the recorder runs them as one batched launch: every input kind, zero points per tensor and per axis, both
    # output types, the vector and the scalar forms.
    OffX, OffS, OffZ, OffO = offs
    d = device()
    k = og.DequantizeKernels(d)
    seed, bad = seed0, 0
    for shape, axis, per_axis in cases.DEQUANT_SHAPES + cases.DEQUANT_SHAPES_BLOCKS:
        n, axis_len, inner = cases.axis_split(shape, axis, per_axis)
        for with_zero in (True, False):
            for half in (False, True):
                say(f"dequantize batch {np.dtype(dtype).name} {shape} axis {axis} per {per_axis} zero {with_zero} "
                    f"f16 {half} offsets {offs}")
                passes = []
                for q in range(3):
                    x = _quantized(dtype, n + OffX, seed)
                    scale = oracle.rig_random(axis_len + OffS, seed + 1, 0.001, 2.0)
                    zeros = _quantized(dtype, axis_len + OffZ, seed + 2)
                    seed += 3
                    want = oracle.dequantize(x[OffX:OffX + n], scale[OffS:], per_axis, axis_len, inner,
                                             zeros[OffZ:OffZ + axis_len] if with_zero else None, f16_out=half)
                    length = og.padded_half_length(n + OffO + 1) if half else n + OffO + 1
                    out = np.full(length, -77, np.float16 if half else np.float32)
                    passes.append((d.CreateBuffer(x), d.CreateBuffer(scale), d.CreateBuffer(zeros), d.CreateBuffer(out),
                                   want))
                names = run_named(d, lambda e: [k.Encode(e, bx, OffX, shape, axis, per_axis, bs,
                                                         OffS, bz if with_zero else None, OffZ, bo, OffO)
                                                for bx, bs, bz, bo, _ in passes])
                want_kernel = ("dequantize4-" if offs == ALIGNED else "dequantize-") + ("f16" if half else "f32")
                assert names == [want_kernel + "-batch"], names
                for _, _, _, bo, want in passes:
                    gbits = bo.Read().view(np.uint16 if half else np.uint32)
                    wbits = want.view(np.uint16) if half else want.view(np.uint32)
                    bad += int(np.count_nonzero(gbits[OffO:OffO + n] != wbits))
    assert bad == 0


def test_binary16_conversion_is_exact():
    # Every binary32 -> binary16 case the output conversion meets, through DequantizeLinear of int32 ones with one scale
    # per element (y = fl(1 * s) = s): ties to even at the normal/subnormal/zero boundaries, the largest finite value and
    # the first to overflow, infinities, signed zeros and NaNs with payloads and either sign (all become 0x7E00 of their
    # sign). Checked against numpy's float16 cast, with the NaNs canonicalised, and against the oracle's conversion.
    f = np.float32
    halfulp = lambda v: f(v) * f(1 + 2**-11)  # noqa: E731
    probes = [0.0, -0.0, 1.0, -1.0, 1.0 + 2**-11, 1.0 + 3 * 2**-11, 1.0 + 2**-11 + 2**-20, 65504.0, 65519.996,
              65520.0, -65520.0, 2**-14, 2**-14 * (1 - 2**-11), 2**-24, 2**-25, 2**-25 * (1 + 2**-20), -2**-25,
              3 * 2**-25, 2**-26, 1e-8, 6e-5, 6.1e-5, -3.14159, 0.1, 1e30, -1e-30, float(halfulp(2.0))]
    probes += [np.inf, -np.inf]
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFBFFFFF, 0x7FC0ABCD], np.uint32).view(np.float32)
    rng = np.random.default_rng(16)
    rand = np.concatenate([rng.uniform(-70000, 70000, 200), rng.uniform(-1e-4, 1e-4, 200),
                           rng.standard_normal(200) * 2.0 ** rng.integers(-30, 17, 200)]).astype(np.float32)
    s = np.concatenate([np.array(probes, np.float32), nans, rand]).astype(np.float32)
    n = s.size
    d = device()
    k = og.DequantizeKernels(d)
    out = np.zeros(og.padded_half_length(n), np.float16)
    bx, bs, bo = d.CreateBuffer(np.ones(n, np.int32)), d.CreateBuffer(s), d.CreateBuffer(out)
    run(d, lambda e: k.Encode(e, bx, 0, [n], 0, True, bs, 0, None, 0, bo, 0))
    got = bo.Read().view(np.uint16)[:n]
    with np.errstate(over="ignore"):
        want = s.astype(np.float16).view(np.uint16).copy()
    isnan = np.isnan(s)
    want[isnan] = (s.view(np.uint32)[isnan] >> 16).astype(np.uint16) & 0x8000 | 0x7E00
    assert np.array_equal(got, want), [(float(s[i]), hex(got[i]), hex(want[i])) for i in np.nonzero(got != want)[0][:8]]
    assert np.array_equal(want, np.array([oracle.f2h(float(v)) for v in s], np.uint16))


def _quant_case(d, k, signed, shape, axis, per_axis, with_zero, half_in, scales, seed, offs=UNALIGNED):
    """DequantizeTests.QuantizeCase (DequantizeTests.cs:179-255)."""
    OffX, OffS, OffZ, OffO = offs
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
    names = run_named(d, lambda e: k.EncodeQuantize(e, bx, OffX, shape, axis, per_axis, bs, OffS, bz if with_zero else None,
                                                     OffZ, bo, OffO))
    want_kernel = ("quantize4-" if offs == ALIGNED else "quantize-") + ("f16-" if half_in else "f32-") + \
        ("i8" if signed else "u8")
    assert names == [want_kernel], names
    got = bo.Read().view(np.uint8)
    init = out.view(np.uint8)
    bad = int(np.count_nonzero(got[OffO:OffO + n] != want))
    bad += int(np.count_nonzero(got[:OffO] != init[:OffO])) + int(np.count_nonzero(got[OffO + n:] != init[OffO + n:]))
    return bad


@pytest.mark.parametrize("offs", [UNALIGNED, ALIGNED], ids=["unaligned", "aligned"])
def test_quantize_is_exact(offs):
    # QuantizeIsExact (DequantizeTests.cs:257-289), at the reference's offsets and at aligned ones
    d = device()
    k = og.DequantizeKernels(d)
    bad = count = 0
    seed = 1
    for shape, axis, per_axis in cases.DEQUANT_SHAPES + cases.DEQUANT_SHAPES_BLOCKS:
        for with_zero in (True, False):
            scales = cases.QUANT_SCALE_SETS[count % len(cases.QUANT_SCALE_SETS)]
            for signed, half_in in ((False, False), (True, False), (False, True), (True, True)):
                say(f"quantize {shape} axis {axis} per {per_axis} zero {with_zero} signed {signed} f16 {half_in} "
                    f"offsets {offs}")
                bad += _quant_case(d, k, signed, shape, axis, per_axis, with_zero, half_in, scales, seed, offs)
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


def _batch_passes(d, k, n_pass, rows, cols, seed, half=False, aligned=True):
    """n_pass DequantizeLinear passes of int32 [rows x cols] with per-column scales, each its own input, scale and
    output (the per-batch rescale after a batched product whose batches have their own column scales), recorded in
    one encoder. Returns (mismatching elements against the oracle, the dispatches' kernel names)."""
    n = rows * cols
    xs = [oracle.dequant_input_i32(n, seed + 3 * p) for p in range(n_pass)]
    ss = [oracle.rig_random(cols, seed + 3 * p + 1, 0.001, 2.0) for p in range(n_pass)]
    off = 0 if aligned else 1
    length = og.padded_half_length(n + off) if half else n + off
    outs = [np.full(length, -77, np.float16 if half else np.float32) for _ in range(n_pass)]
    bx = [d.CreateBuffer(x) for x in xs]
    bs = [d.CreateBuffer(s) for s in ss]
    bo = [d.CreateBuffer(o) for o in outs]
    names = run_named(d, lambda e: [k.Encode(e, bx[p], 0, [rows, cols], 1, True, bs[p], 0, None, 0, bo[p], off)
                                    for p in range(n_pass)])
    bad = 0
    for p in range(n_pass):
        want = oracle.dequantize(xs[p], ss[p], True, cols, 1, None, f16_out=half)
        got = bo[p].Read()
        bits = np.uint16 if half else np.uint32
        bad += int(np.count_nonzero(got[off:off + n].view(bits) != want.view(bits)))
    return bad, names


@pytest.mark.parametrize("half", [False, True])
def test_consecutive_dequantize_passes_run_as_one_launch(half):
    # 40 passes of one shape: one batch of 40 (the recorder batches up to 256, a launch takes up to 64), bit-exact, and
    # the same bits with batching off (a launch a pass).
    d = device()
    k = og.DequantizeKernels(d)
    say(f"dequantize batch: 40 passes of 64 x 256, f16 {half}")
    bad, names = _batch_passes(d, k, 40, 64, 256, 500, half)
    assert bad == 0
    assert names == ["dequantize4-" + ("f16" if half else "f32") + "-batch"], names
    d1 = og.GpuDevice.Create(0, 0, BatchDispatches=False)
    bad1, names1 = _batch_passes(d1, og.DequantizeKernels(d1), 40, 64, 256, 500, half)
    assert bad1 == 0 and len(names1) == 40, names1
    say("  unaligned outputs (the scalar form, batched)")
    bad, names = _batch_passes(d, k, 5, 33, 100, 900, half, aligned=False)
    assert bad == 0 and names == ["dequantize-" + ("f16" if half else "f32") + "-batch"], names


def test_long_runs_of_dequantize_passes_split_into_batches():
    # 300 passes of one shape: the recorder takes at most 256 passes a call (OG_DEQUANT_BATCH_MAX), so two calls (256 +
    # 44), and a call launches at most 64 passes at once (four launches for the first); every pass bit-exact.
    d = device()
    k = og.DequantizeKernels(d)
    say("dequantize batch: 300 passes of 4 x 64")
    bad, names = _batch_passes(d, k, 300, 4, 64, 1300)
    assert bad == 0
    assert names == ["dequantize4-f32-batch"] * 2, names


def test_dependent_dequantize_passes_stay_in_order():
    # Passes whose buffers meet are not batched: the second of two passes into the same output wins, as in order; a
    # pass of another shape ends a batch.
    d = device()
    k = og.DequantizeKernels(d)
    rows, cols = 16, 64
    n = rows * cols
    x1, x2 = oracle.dequant_input_i32(n, 7), oracle.dequant_input_i32(n, 8)
    s1, s2 = oracle.rig_random(cols, 9, 0.001, 2.0), oracle.rig_random(cols, 10, 0.001, 2.0)
    b1, b2, c1, c2 = d.CreateBuffer(x1), d.CreateBuffer(x2), d.CreateBuffer(s1), d.CreateBuffer(s2)
    out = d.CreateBuffer(np.zeros(n, np.float32))
    other = d.CreateBuffer(np.zeros(n, np.float32))
    say("dequantize batch: two passes into one output, then a pass of another shape")
    names = run_named(d, lambda e: [k.Encode(e, b1, 0, [rows, cols], 1, True, c1, 0, None, 0, out, 0),
                                    k.Encode(e, b2, 0, [rows, cols], 1, True, c2, 0, None, 0, out, 0),
                                    k.Encode(e, b1, 0, [rows * cols], 0, False, c1, 0, None, 0, other, 0)])
    assert names == ["dequantize4-f32"] * 3, names
    want = oracle.dequantize(x2, s2, True, cols, 1, None)
    assert np.array_equal(out.Read().view(np.uint32), want.view(np.uint32))
    want_other = oracle.dequantize(x1, s1, False, 1, 1, None)
    assert np.array_equal(other.Read().view(np.uint32), want_other.view(np.uint32))
