"""Pins the CPU oracle before anything is compared with it (CPU only).

The reference ships no golden vectors for this path (its tests compute their expectations on the fly in C#), so the
oracle is pinned by: the reference's closed forms, brute force / library routines that compute the same mathematics
independently (numpy int64 matmul, IEEE float32 arithmetic, numpy's float16 cast, np.rint), the signed-domain identity
agreeing with the definition form, the reference kernel's own integer division agreeing with IEEE division, and the
worked examples of the ONNX specifications (DynamicQuantizeLinear, Gather, ConvInteger). tests/test_oracle_mutants.py
runs the same pins against deliberately broken implementations and shows that each one fails them.
"""
import numpy as np
import pytest

import cases
import oracle


# ------------------------------------------------------------------ int32 sums

def numpy_sums(p, a, a_signed, b, b_signed, za=None, zb=None):
    """C[b, m, n] = sum_k (A - za)(B - zb) by numpy int64 matmul, wrapped to int32."""
    lda = p.Lda or p.K
    ldb = p.Ldb or (p.K if p.TransposeB else p.N)
    av = a.view(np.int8).astype(np.int64) if a_signed else a.astype(np.int64)
    bv = b.view(np.int8).astype(np.int64) if b_signed else b.astype(np.int64)
    out = np.zeros((p.Batch, p.M, p.N), np.int64)
    for bt in range(p.Batch):
        ia = p.OffsetA + bt * p.StrideA + np.arange(p.M)[:, None] * lda + np.arange(p.K)[None, :]
        A = av[ia] if p.K else np.zeros((p.M, 0), np.int64)
        if p.TransposeB:
            ib = p.OffsetB + bt * p.StrideB + np.arange(p.N)[:, None] * ldb + np.arange(p.K)[None, :]
            B = bv[ib].T if p.K else np.zeros((0, p.N), np.int64)
        else:
            ib = p.OffsetB + bt * p.StrideB + np.arange(p.K)[:, None] * ldb + np.arange(p.N)[None, :]
            B = bv[ib] if p.K else np.zeros((0, p.N), np.int64)
        if za is not None:
            zbuf, zvec, zoff = za
            zv = zbuf.view(np.int8).astype(np.int64) if a_signed else zbuf.astype(np.int64)
            A = A - (zv[zoff:zoff + p.M][:, None] if zvec else zv[zoff])
        if zb is not None:
            zbuf, zvec, zoff = zb
            zv = zbuf.view(np.int8).astype(np.int64) if b_signed else zbuf.astype(np.int64)
            B = B - (zv[zoff:zoff + p.N][None, :] if zvec else zv[zoff])
        out[bt] = A @ B
    return ((out + 2**31) % 2**32 - 2**31).astype(np.int32).ravel()


def test_closed_form_matches_the_reference():
    # MultiDeviceTests.cs:30-31, 53-55: [[1 2], [3 4]] x [[1 -1 2], [-2 3 -3]] = [[-3 5 -4], [-5 9 -6]]
    p = oracle.Gemm(2, 3, 2)
    a = np.array([1, 2, 3, 4], np.uint8)
    b = np.array([1, -1, 2, -2, 3, -3], np.int8).view(np.uint8)
    want = [-3, 5, -4, -5, 9, -6]
    assert oracle.int8_gemm(p, a, False, b, True).tolist() == want
    assert oracle.int8_gemm_identity(p, a, False, b, True).tolist() == want


def test_edge_cases_definition_equals_numpy_and_identity():
    # Every EdgeShapesAreBitExact case (Int8Tests.cs:214-270), with its own data.
    for i, c in enumerate(cases.edge_cases()):
        d = cases.case_data(c, i + 1)
        za = None if d["za"] is None else (d["za"], c.za_mode == 2, 0)
        zb = None if d["zb"] is None else (d["zb"], c.zb_mode == 2, 0)
        got = oracle.int8_gemm(c.p, d["a"], c.a_signed, d["b"], c.b_signed, za, zb)
        np.testing.assert_array_equal(got, numpy_sums(c.p, d["a"], c.a_signed, d["b"], c.b_signed, za, zb), err_msg=c.name)
        np.testing.assert_array_equal(got, oracle.int8_gemm_identity(c.p, d["a"], c.a_signed, d["b"], c.b_signed, za, zb),
                                      err_msg=c.name)


def test_sums_wrap_modulo_2_32():
    # K = 40000 at the extremes: |sum| reaches 2.6e9 > 2^31, so the int32 result must wrap like two's complement.
    k = 40000
    p = oracle.Gemm(2, 3, k)
    a = np.full(2 * k, 0x00, np.uint8)
    b = np.full(k * 3, 0xFF, np.uint8)
    za = (np.array([255], np.uint8), False, 0)
    got = oracle.int8_gemm(p, a, False, b, False, za)
    want = numpy_sums(p, a, False, b, False, za)
    assert abs(-255 * 255 * k) > 2**31
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got, oracle.int8_gemm_identity(p, a, False, b, False, za))


def test_sampled_rows_equal_full_product():
    c = cases.model_case("minilm qkv/proj b1x128", 128, 384, 384)
    d = cases.case_data(c, 3)
    full = cases.reference_sums(c, d).reshape(128, 384)
    rows = np.array([0, 5, 77, 127])
    got = oracle.int8_gemm_rows(c.p, d["a"], False, d["b"], True, rows, (d["za"], False, 0))
    np.testing.assert_array_equal(got, full[rows])


# ------------------------------------------------------------------ float and requantized forms

def test_float_epilogue_is_two_float32_roundings():
    rng = np.random.default_rng(0)
    sums = rng.integers(-2**31, 2**31, 5000, dtype=np.int64).astype(np.int32)
    n = 50
    scale = rng.uniform(1e-5, 1e-2, n).astype(np.float32)
    ib = rng.integers(-10000, 10000, n).astype(np.int32)
    fb = rng.uniform(-2, 2, n).astype(np.float32)
    got = oracle.float_epilogue(sums, n, scale, True, ib, fb)
    cols = np.arange(sums.size) % n
    acc = ((sums.astype(np.int64) + ib[cols] + 2**31) % 2**32 - 2**31).astype(np.int32)
    want = (acc.astype(np.float32) * scale[cols]).astype(np.float32) + fb[cols]
    np.testing.assert_array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    # One rounding instead of two (a multiply-add contracted to an FMA) gives different bits on these inputs.
    fused = (acc.astype(np.float64) * scale[cols].astype(np.float64) + fb[cols]).astype(np.float32)
    assert np.any(fused.view(np.uint32) != got.view(np.uint32))
    # Without biases, scalar scale.
    got = oracle.float_epilogue(sums, n, scale[:1], False)
    np.testing.assert_array_equal(got.view(np.uint32), (sums.astype(np.float32) * scale[0]).view(np.uint32))


def _requant_numpy(acc, mult, zero, unsigned):
    lo, hi = (0, 255) if unsigned else (-128, 127)
    v = np.float32(acc) * np.float32(mult)
    if np.isnan(v):
        return lo
    r = np.rint(v)
    r = min(max(r, np.float32(lo - zero)), np.float32(hi - zero))
    return int(r) + zero


def test_requant_ties_and_saturation():
    # RequantizationRoundsHalfToEvenAndSaturates (Int8Tests.cs:503-547), plus explicit tie expectations.
    for mult, zero, unsigned in cases.REQUANT_TIES:
        for av in range(-9, 10):
            with np.errstate(invalid="ignore", over="ignore"):
                assert oracle.requant(av, mult, zero, unsigned) == _requant_numpy(av, mult, zero, unsigned)
    assert oracle.requant(5, 0.5, 0, True) == 2      # 2.5 -> 2 (half to even)
    assert oracle.requant(7, 0.5, 0, True) == 4      # 3.5 -> 4
    assert oracle.requant(-5, 0.5, 0, False) == -2   # -2.5 -> -2
    assert oracle.requant(1, 1e9, 3, True) == 255
    assert oracle.requant(1, float("nan"), 5, False) == -128


# ------------------------------------------------------------------ DynamicQuantizeLinear

def dq_numpy(x):
    """DynamicQuantizeLinear from numpy float32 arithmetic (IEEE division, np.rint half-to-even)."""
    x = np.asarray(x, np.float32)
    ok = ~np.isnan(x)
    mn = x[ok].min() if ok.any() else np.float32(np.inf)
    mx = x[ok].max() if ok.any() else np.float32(-np.inf)
    lo = mn if mn <= 0 else np.float32(0)
    hi = mx if mx > 0 else np.float32(0)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        scale = np.float32(hi - lo) / np.float32(255)
        zp = 0
        if scale != 0 and np.isfinite(scale):
            z = np.rint(np.float32(0) - np.float32(lo / scale))
            zp = 0 if z < 0 else (255 if z > 255 else int(z))
        if scale == 0:
            return np.zeros(x.size, np.uint8), np.float32(1), 0
        v = np.rint(x / scale).astype(np.float32) + np.float32(zp)
        y = np.where(np.isnan(v), 0, np.clip(v, 0, 255)).astype(np.uint8)
    return y, scale, zp


def test_dynamic_quantize_matches_numpy_on_reference_cases():
    # All 105 tensors of DynamicQuantizeIsBitExact (Int8Tests.cs:617-703).
    for count, kind, seed in cases.dq_cases():
        x = oracle.dq_input(count, seed, kind)
        y, s, z = oracle.dynamic_quantize(x)
        wy, ws, wz = dq_numpy(x)
        assert np.float32(s).view(np.uint32) == np.float32(ws).view(np.uint32), (count, kind)
        assert z == wz, (count, kind)
        np.testing.assert_array_equal(y, wy, err_msg=f"{count} {kind}")


def test_dynamic_quantize_special_inputs():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    for x in ([0.0], [-0.0, 0.0], [nan, nan], [1.0, nan, -1.0], [inf, 1.0], [-inf, 2.0], [1e-42, 3e-42], [-1e-42],
              [1e30, -1e30], [255.0, 0.0], [-3.0, -2.0]):
        x = np.array(x, np.float32)
        y, s, z = oracle.dynamic_quantize(x)
        wy, ws, wz = dq_numpy(x)
        assert (np.isnan(s) and np.isnan(ws)) or np.float32(s).view(np.uint32) == np.float32(ws).view(np.uint32), x
        assert z == wz, x
        np.testing.assert_array_equal(y, wy, err_msg=str(x))
    # Closed forms: [0, 255] -> scale 1, zp 0, y = x; all zero -> (1, 0).
    y, s, z = oracle.dynamic_quantize(np.array([0, 255, 17], np.float32))
    assert (s, z, y.tolist()) == (1.0, 0, [0, 255, 17])
    assert oracle.dynamic_quantize(np.zeros(5, np.float32))[1:] == (1.0, 0)


def test_dynamic_quantize_onnx_examples():
    # The ONNX DynamicQuantizeLinear specification's worked examples: published outputs, so they pin the formula
    # (range adjusted to include 0, scale = range / 255, zero point = rne(-lo / scale) clamped) and its float32
    # rounding (-2.5 / scale is -127.49999... in float32, hence 26, not 25).
    for x, want_y, want_z in cases.DQ_ONNX_EXAMPLES:
        y, s, z = oracle.dynamic_quantize(np.array(x, np.float32))
        assert y.tolist() == want_y and z == want_z, x
        lo, hi = min(0.0, min(x)), max(0.0, max(x))
        assert np.float32(s) == np.float32(np.float32(hi) - np.float32(lo)) / np.float32(255)


def test_dynamic_quantize_hand_vectors():
    # Ties, a clamped output and a zero point that is itself a tie (cases.DQ_HAND_VECTORS, derived by hand).
    for x, want_y, want_s, want_z in cases.DQ_HAND_VECTORS:
        y, s, z = oracle.dynamic_quantize(np.array(x, np.float32))
        assert (y.tolist(), float(s), z) == (want_y, want_s, want_z), x


def test_div_exact_equals_ieee_division():
    # The reference kernel's integer long division (DivExact.hlsli) equals IEEE float32 division on the quantizer's
    # operands: the scale computations and every x / scale of the DQ cases, plus random and edge operands.
    rng = np.random.default_rng(1)
    xs = [rng.standard_normal(20000).astype(np.float32) * np.float32(10) ** rng.integers(-40, 38, 20000).astype(np.float32),
          oracle.quantize_input(5000, 3, True), oracle.dq_input(5000, 7, 3)]
    ss = [np.float32(1 / 255), np.float32(0.0137), np.float32(3.3), np.float32(1e-6), np.float32(1e3),
          np.float32(4.7 * 2 / 255), np.float32(1e-44), np.float32(7e37)]
    count = 0
    with np.errstate(all="ignore"):
        for x in np.concatenate(xs):
            for s in ss:
                got = oracle.div_exact(float(x), float(s))
                want = np.float32(x) / s
                assert (np.isnan(got) and np.isnan(want)) or got.view(np.uint32) == np.float32(want).view(np.uint32), (x, s)
                count += 1
    assert count > 200000


# ------------------------------------------------------------------ (de)quantize

def test_f2h_equals_numpy_float16_rounding():
    rng = np.random.default_rng(2)
    # Every half value and its float32 neighbours (ties in between), random bit patterns, the overflow edge.
    halves = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    halves = halves[np.isfinite(halves)]
    bits = halves.view(np.uint32)
    probes = np.concatenate([bits, bits + 1, bits - 1, bits + 0x1000, bits + 0xFFF, bits + 0x1001,
                             rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32),
                             np.array([0x477FEFFF, 0x477FF000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x33000000, 0x33000001],
                                      np.uint32)]).view(np.float32)
    lib = oracle.lib()
    got = np.array([lib.ora_f2h(float(f)) for f in probes], np.uint16)
    want = probes.astype(np.float16).view(np.uint16)
    nan = np.isnan(probes)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_h2f_equals_numpy_for_every_half():
    lib = oracle.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([lib.ora_h2f(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))


@pytest.mark.parametrize("kind", [np.uint8, np.int8, np.int32])
def test_dequantize_equals_numpy(kind):
    seed = 7
    for shape, axis, per_axis in cases.DEQUANT_SHAPES:
        count, axis_len, inner = cases.axis_split(shape, axis, per_axis)
        if kind == np.int32:
            x = oracle.dequant_input_i32(count, seed)
            z = oracle.dequant_input_i32(axis_len, seed + 2)
        else:
            x = oracle.dequant_input_bytes(count, seed).view(kind)
            z = oracle.dequant_input_bytes(axis_len, seed + 2).view(kind)
        scale = oracle.rig_random(axis_len, seed + 1, 0.001, 2.0)
        for zero in (z, None):
            got = oracle.dequantize(x, scale, per_axis, axis_len, inner, zero)
            a = (np.arange(count) // inner) % axis_len if per_axis else np.zeros(count, np.int64)
            zp = zero[a].astype(np.int64) if zero is not None else 0
            d = ((x.astype(np.int64) - zp + 2**31) % 2**32 - 2**31).astype(np.int32)
            want = d.astype(np.float32) * scale[a]
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
            got16 = oracle.dequantize(x, scale, per_axis, axis_len, inner, zero, f16_out=True)
            np.testing.assert_array_equal(got16, want.astype(np.float16).view(np.uint16))
        seed += 3


def test_quantize_equals_numpy():
    seed = 1
    for shape, axis, per_axis in cases.DEQUANT_SHAPES:
        count, axis_len, inner = cases.axis_split(shape, axis, per_axis)
        for scales in cases.QUANT_SCALE_SETS:
            x = oracle.quantize_input(count, seed, True)
            scale = np.array([scales[i % len(scales)] for i in range(axis_len)], np.float32)
            for signed in (False, True):
                zero = oracle.dequant_input_bytes(axis_len, seed + 2)
                for zp in (zero, None):
                    got = oracle.quantize(x, scale, signed, per_axis, axis_len, inner, zp)
                    a = (np.arange(count) // inner) % axis_len if per_axis else np.zeros(count, np.int64)
                    z = 0 if zp is None else (zp.view(np.int8) if signed else zp).astype(np.float32)[a]
                    with np.errstate(all="ignore"):
                        v = np.rint(x / scale[a]).astype(np.float32) + np.float32(z) if zp is None else \
                            np.rint(x / scale[a]).astype(np.float32) + z
                    lo, hi = (-128, 127) if signed else (0, 255)
                    want = np.where(np.isnan(v), lo, np.clip(v, lo, hi)).astype(np.int64).astype(np.uint8)
                    np.testing.assert_array_equal(got, want, err_msg=f"{shape} {axis} {scales} {signed}")
            seed += 1


def test_generators_are_deterministic_and_in_range():
    a = oracle.bytes_(1000, 5)
    assert np.array_equal(a, oracle.bytes_(1000, 5)) and not np.array_equal(a, oracle.bytes_(1000, 6))
    r = oracle.rig_random(1000, 3, -3.0, 5.0)
    assert r.min() >= -3.0 and r.max() < 5.0
    u = oracle.synth_uniform_i32(100000, 4, 1, 100, 156)
    assert u.min() == 100 and u.max() == 156
    g = oracle.synth_normal_f32(200000, 1, 0, 0.0, 1.0)
    assert abs(float(g.mean())) < 0.01 and abs(float(g.std()) - 1.0) < 0.01


# ------------------------------------------------------------------ gather

def _gather_loops(data, shape, axis, idx, wide):
    """The index map GatherTests.cs:45-57 walks, in plain loops (tiny shapes only)."""
    rank = len(shape)
    ax = axis + rank if axis < 0 else axis
    outer = int(np.prod(shape[:ax])) if ax else 1
    inner = int(np.prod(shape[ax + 1:])) if ax + 1 < rank else 1
    n_axis = shape[ax]
    out, bad = [], None
    for o in range(outer):
        for i, v in enumerate(idx):
            ok = -n_axis <= v < n_axis and (not wide or -(1 << 31) <= v < (1 << 31))
            if not ok and bad is None:
                bad = i
            for m in range(inner):
                out.append(data[(o * n_axis + (v + n_axis if v < 0 else v)) * inner + m] if ok else 0)
    return np.array(out, dtype=np.asarray(data).dtype), bad


def test_gather_onnx_examples():
    # The two examples of the ONNX Gather operator's specification (axis 0 and axis 1).
    d0 = np.array([[1.0, 1.2], [2.3, 3.4], [4.5, 5.7]], np.float32)
    out, bad = oracle.gather(d0, d0.shape, 0, [0, 1, 1, 2])
    assert bad is None and out.reshape(2, 2, 2).tolist() == np.array(
        [[[1.0, 1.2], [2.3, 3.4]], [[2.3, 3.4], [4.5, 5.7]]], np.float32).tolist()
    d1 = np.array([[1.0, 1.2, 1.9], [2.3, 3.4, 3.9], [4.5, 5.7, 5.9]], np.float32)
    out, bad = oracle.gather(d1, d1.shape, 1, [0, 2])
    assert bad is None and out.reshape(3, 1, 2).tolist() == np.array(
        [[[1.0, 1.9]], [[2.3, 3.9]], [[4.5, 5.9]]], np.float32).tolist()


def test_gather_against_loops_and_numpy_take():
    rng = np.random.default_rng(5)
    for shape, axis in (([10], 0), ([5, 6], 1), ([5, 6], -1), ([2, 3, 4, 5], 2), ([4, 1, 9], 0), ([3, 0, 2], 1)):
        data = rng.integers(-128, 128, int(np.prod(shape)), dtype=np.int8)
        n_axis = shape[axis]
        for wide in (False, True):
            idx = [int(x) for x in rng.integers(-2 * n_axis - 1, 2 * n_axis + 2, 7)]
            if wide:
                idx += [(1 << 31) + 1, -(1 << 31) - 3]
            got, bad = oracle.gather(data, shape, axis, idx, wide)
            want, want_bad = _gather_loops(data, shape, axis, idx, wide)
            assert np.array_equal(got, want) and bad == want_bad, (shape, axis, idx)
            ok = [v for v in idx if -n_axis <= v < n_axis]
            if ok:   # valid indices only: numpy's take along the axis
                got, bad = oracle.gather(data, shape, axis, ok, wide)
                assert bad is None
                assert np.array_equal(got, np.take(data.reshape(shape), ok, axis=axis).ravel())
    # A plausible slip (a negative index taken modulo the axis twice, or positions counted from 1) changes these.
    out, bad = oracle.gather(np.arange(4, dtype=np.uint8), [4], 0, [-1, -4, 4, 0, -5])
    assert out.tolist() == [3, 0, 0, 0, 0] and bad == 2


# ------------------------------------------------------------------ ConvInteger

def test_conv_integer_onnx_examples():
    # The ONNX ConvInteger specification's two examples (without and with padding 1).
    x = np.array([2, 3, 4, 5, 6, 7, 8, 9, 10], np.uint8)
    c = dict(Batch=1, InChannels=1, Height=3, Width=3, OutChannels=1, KernelHeight=2, KernelWidth=2)
    assert oracle.conv_integer(c, x, False, np.ones(4, np.uint8), False, np.array([1], np.uint8)).tolist() == \
        [12, 16, 24, 28]
    c.update(PadTop=1, PadLeft=1, PadBottom=1, PadRight=1)
    assert oracle.conv_integer(c, x, False, np.ones(4, np.uint8), False, np.array([1], np.uint8)).tolist() == \
        [1, 3, 5, 3, 5, 12, 16, 9, 11, 24, 28, 15, 7, 15, 17, 9]


def _conv_loops(c, x, xs, w, ws, xz, wz, wz_vec):
    """The ONNX definition in plain loops (tiny shapes): int64 sums wrapped to int32 at the end."""
    B, C, H, W, M = c["Batch"], c["InChannels"], c["Height"], c["Width"], c["OutChannels"]
    KH, KW, G = c["KernelHeight"], c["KernelWidth"], c.get("Groups", 1)
    SH, SW, DH, DW = c.get("StrideHeight", 1), c.get("StrideWidth", 1), c.get("DilationHeight", 1), c.get("DilationWidth", 1)
    PT, PL, PB, PR = c.get("PadTop", 0), c.get("PadLeft", 0), c.get("PadBottom", 0), c.get("PadRight", 0)
    oh = (H + PT + PB - DH * (KH - 1) - 1) // SH + 1
    ow = (W + PL + PR - DW * (KW - 1) - 1) // SW + 1
    xv = (x.view(np.int8) if xs else x).astype(np.int64).reshape(B, C, H, W)
    wv = (w.view(np.int8) if ws else w).astype(np.int64).reshape(M, C // G, KH, KW)
    xzv = 0 if xz is None else int((xz.view(np.int8) if xs else xz)[0])
    wzv = np.zeros(M, np.int64) if wz is None else (wz.view(np.int8) if ws else wz).astype(np.int64)
    if wz is not None and not wz_vec:
        wzv = np.full(M, wzv[0])
    y = np.zeros((B, M, oh, ow), np.int64)
    for n in range(B):
        for m in range(M):
            g = m // (M // G)
            for i in range(oh):
                for j in range(ow):
                    acc = 0
                    for cc in range(C // G):
                        for kh in range(KH):
                            for kw in range(KW):
                                ih, iw = i * SH + kh * DH - PT, j * SW + kw * DW - PL
                                if 0 <= ih < H and 0 <= iw < W:
                                    acc += (xv[n, g * (C // G) + cc, ih, iw] - xzv) * (wv[m, cc, kh, kw] - wzv[m])
                    y[n, m, i, j] = acc
    return ((y & 0xFFFFFFFF).astype(np.uint32).view(np.int32)).ravel()


def _conv_im2col(c, x, xs, w, ws, xz, wz, wz_vec):
    """An independent lowering: padded input filled with the zero point, windows unfolded with numpy slicing, one
    int64 matrix product per group (numpy), wrapped to int32."""
    B, C, H, W, M = c["Batch"], c["InChannels"], c["Height"], c["Width"], c["OutChannels"]
    KH, KW, G = c["KernelHeight"], c["KernelWidth"], c.get("Groups", 1)
    SH, SW, DH, DW = c.get("StrideHeight", 1), c.get("StrideWidth", 1), c.get("DilationHeight", 1), c.get("DilationWidth", 1)
    PT, PL, PB, PR = c.get("PadTop", 0), c.get("PadLeft", 0), c.get("PadBottom", 0), c.get("PadRight", 0)
    xzv = 0 if xz is None else int((xz.view(np.int8) if xs else xz)[0])
    xv = (x.view(np.int8) if xs else x).astype(np.int64).reshape(B, C, H, W) - xzv
    xp = np.zeros((B, C, H + PT + PB, W + PL + PR), np.int64)
    xp[:, :, PT:PT + H, PL:PL + W] = xv
    oh = (H + PT + PB - DH * (KH - 1) - 1) // SH + 1
    ow = (W + PL + PR - DW * (KW - 1) - 1) // SW + 1
    cols = np.stack([xp[:, :, kh * DH:kh * DH + SH * (oh - 1) + 1:SH, kw * DW:kw * DW + SW * (ow - 1) + 1:SW]
                     for kh in range(KH) for kw in range(KW)], axis=2)          # [B, C, KH*KW, oh, ow]
    wzv = np.zeros(M, np.int64) if wz is None else (wz.view(np.int8) if ws else wz).astype(np.int64)
    if wz is not None and not wz_vec:
        wzv = np.full(M, wzv[0])
    wv = (w.view(np.int8) if ws else w).astype(np.int64).reshape(M, -1) - wzv[:, None]
    cg, mg = C // G, M // G
    y = np.zeros((B, M, oh * ow), np.int64)
    for g in range(G):
        a = wv[g * mg:(g + 1) * mg]                                              # [mg, cg*KH*KW]
        bcol = cols[:, g * cg:(g + 1) * cg].reshape(B, cg * KH * KW, oh * ow)
        y[:, g * mg:(g + 1) * mg] = np.einsum("mk,bkn->bmn", a, bcol)
    return ((y & 0xFFFFFFFF).astype(np.uint32).view(np.int32)).ravel()


CONV_PIN_CASES = [
    dict(Batch=2, InChannels=4, Height=5, Width=6, OutChannels=3, KernelHeight=3, KernelWidth=3, PadTop=1, PadLeft=1,
         PadBottom=1, PadRight=1),
    dict(Batch=1, InChannels=3, Height=7, Width=5, OutChannels=2, KernelHeight=3, KernelWidth=2, StrideHeight=2,
         PadTop=2, PadRight=3),
    dict(Batch=1, InChannels=2, Height=8, Width=9, OutChannels=2, KernelHeight=3, KernelWidth=3, DilationHeight=2,
         DilationWidth=2, PadTop=2, PadLeft=2, PadBottom=2, PadRight=2),
    dict(Batch=2, InChannels=4, Height=4, Width=4, OutChannels=6, KernelHeight=3, KernelWidth=3, PadTop=1, PadLeft=1,
         PadBottom=1, PadRight=1, Groups=2),
    dict(Batch=1, InChannels=3, Height=5, Width=5, OutChannels=3, KernelHeight=3, KernelWidth=3, Groups=3),
]


def test_conv_integer_against_loops_and_an_im2col_product():
    rng = np.random.default_rng(11)
    for i, c in enumerate(CONV_PIN_CASES):
        for xs, ws, zmode in ((False, True, 2), (True, False, 1), (True, True, 0), (False, False, 2)):
            x = rng.integers(0, 256, c["Batch"] * c["InChannels"] * c["Height"] * c["Width"], dtype=np.uint8)
            w = rng.integers(0, 256, c["OutChannels"] * (c["InChannels"] // c.get("Groups", 1)) * c["KernelHeight"]
                             * c["KernelWidth"], dtype=np.uint8)
            xz = None if zmode == 0 else rng.integers(0, 256, 1, dtype=np.uint8)
            wz = None if zmode == 0 else rng.integers(0, 256, c["OutChannels"] if zmode == 2 else 1, dtype=np.uint8)
            got = oracle.conv_integer(c, x, xs, w, ws, xz, wz, zmode == 2)
            assert np.array_equal(got, _conv_loops(c, x, xs, w, ws, xz, wz, zmode == 2)), (i, xs, ws, zmode)
            assert np.array_equal(got, _conv_im2col(c, x, xs, w, ws, xz, wz, zmode == 2)), (i, xs, ws, zmode)


def test_conv_integer_pointwise_is_a_matrix_product():
    # A 1x1 convolution is W [Cout, Cin] times X [Cin, H*W] per image; with extreme bytes the int32 sums wrap.
    rng = np.random.default_rng(3)
    c = dict(Batch=2, InChannels=300, Height=3, Width=4, OutChannels=5, KernelHeight=1, KernelWidth=1)
    x = np.full(2 * 300 * 12, 255, np.uint8)
    w = rng.integers(0, 256, 5 * 300, dtype=np.uint8)
    got = oracle.conv_integer(c, x, False, w, False).reshape(2, 5, 12)
    want = w.astype(np.int64).reshape(5, 300) @ x.astype(np.int64).reshape(2, 300, 12)
    assert np.array_equal(got, want.astype(np.int32))
    x = np.full(2 * 300 * 12, 0x80, np.uint8)                         # int8 -128
    w = np.full(5 * 300, 0x80, np.uint8)
    xz, wz = np.array([0x7F], np.uint8), np.array([0x7F], np.uint8)   # int8 127: each term (-255)^2
    got = oracle.conv_integer(c, x, True, w, True, xz, wz)
    assert np.all(got == np.int32(((300 * 255 * 255) & 0xFFFFFFFF) - (1 << 32) if (300 * 255 * 255) >= (1 << 31)
                                  else 300 * 255 * 255))
