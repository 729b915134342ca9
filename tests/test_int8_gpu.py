"""GPU parity of the int8 path against the CPU oracle, through the host layer and the C ABI: the reference's
Int8Tests (tests/RecursiveAI.OneGpu.Kernels.Tests/Int8Tests.cs), case for case, bit-exact."""
import ctypes

import numpy as np
import pytest

import cases
import oracle
import onegpu_hip as og
from gpu_rig import CONFIG_OPTIONS, as_i8, as_u8, configs, device, run, run_int32, say, to_problem, binding, abi, check

pytestmark = pytest.mark.gpu


def test_closed_form():
    # MultiDeviceTests.cs:30-31, 40, 53-55
    d = device()
    with og.Int8Gemm(d) as gemm:
        a = d.CreateBuffer(np.array([1, 2, 3, 4, 5, 6], np.uint8))
        b = d.CreateBuffer(np.array([1, -1, 2, -2, 3, -3], np.int8))
        c = d.CreateBufferOf(og.ElementType.Int32, 6)
        for _ in range(3):
            run(d, lambda e: gemm.EncodeInt32(e, og.Int8GemmProblem(2, 3, 2), a, b, c))
        assert c.Read().tolist() == [-3, 5, -4, -5, 9, -6]


@pytest.mark.parametrize("config", ["default", "portable", "tiled only", "split k", "large tile"])
def test_edge_shapes_are_bit_exact(config):
    # EdgeShapesAreBitExact (Int8Tests.cs:214-283): every case, each kernel forced in turn.
    d = device()
    gemm = dict(configs(d, True))[config]
    bad_total = 0
    kernels = set()
    for i, c in enumerate(cases.edge_cases()):
        say(f"edge [{config}] case {i} {c.name} signed {c.a_signed}/{c.b_signed} zp {c.za_mode}/{c.zb_mode}")
        bad, k = run_int32(d, gemm, c, i + 1)
        kernels.add(k)
        if bad:
            say(f"MISMATCH [{config}] {c.name}: {bad} elements")
        bad_total += bad
    say(f"ROW int8 gemm | {config} | kernels {sorted(kernels)} | mismatching int32 sums {bad_total}")
    assert bad_total == 0


def test_model_shapes_are_bit_exact():
    # ModelShapesAreBitExact (Int8Tests.cs:285-317): u8 activations with a zero point, int8 weights stored N x K,
    # plus the same shapes with the weights stored K x N (the layout of the benchmark configurations).
    d = device()
    bad_total = 0
    for name, m, n, k in cases.MODEL_SHAPES:
        for trans in (True, False):
            c = cases.model_case(name, m, n, k)
            if not trans:
                c.p = cases.problem(m, n, k)
            data = cases.case_data(c, m + n + k)
            want = cases.reference_sums(c, data)
            for config, gemm in configs(d, m <= 128):
                say(f"model {name} trans {trans} [{config}]")
                bad, kernel = run_int32(d, gemm, c, m + n + k, want)
                say(f"ROW int8 gemm | u8 x i8 | {name} trans {trans}, {config} | {kernel} | mismatches {bad}")
                bad_total += bad
    assert bad_total == 0


def test_forcing_the_dot_variant_off_changes_nothing():
    # Int8Tests.cs:319-332
    d = device()
    chosen = og.Int8Gemm(d)
    forced = og.Int8Gemm(d, og.Int8GemmOptions(AllowPackedDot=False))
    c = cases.Case("forced", cases.problem(70, 90, 100), False, True, 1, 2)
    b1, _ = run_int32(d, chosen, c, 5)
    b2, _ = run_int32(d, forced, c, 5)
    assert b1 + b2 == 0
    assert forced.Variant == "portable-tile64x64x16"
    assert chosen.Variant != forced.Variant


def _float_case(d, gemm, m, n, k, scale_vec, with_ib, with_fb, seed):
    """FloatCase (Int8Tests.cs:334-373)."""
    a, b, za, zb, scale, ib, fb = cases.float_case_data(m, n, k, scale_vec, seed)
    p = cases.problem(m, n, k)
    want = oracle.int8_gemm(p, a, False, b, True, (za, False, 0), (zb, True, 0))
    expected = oracle.float_epilogue(want, n, scale, scale_vec, ib if with_ib else None, fb if with_fb else None)
    ba, bb = d.CreateBuffer(as_u8(a)), d.CreateBuffer(as_i8(b))
    bza, bzb = d.CreateBuffer(as_u8(za)), d.CreateBuffer(as_i8(zb))
    bs, bib, bfb = d.CreateBuffer(scale), d.CreateBuffer(ib), d.CreateBuffer(fb)
    bc = d.CreateBufferOf(og.ElementType.Float32, m * n)
    run(d, lambda e: gemm.EncodeFloat(e, to_problem(p), ba, bb, bc, og.Int8Operand(bs, 0, scale_vec),
                                      og.Int8Operand(bza, 0), og.Int8Operand(bzb, 0, True),
                                      og.Int8Operand(bfb, 0, True) if with_fb else None,
                                      og.Int8Operand(bib, 0, True) if with_ib else None))
    got = bc.Read()
    same = np.where(np.isnan(expected), np.isnan(got), got.view(np.uint32) == expected.view(np.uint32))
    return int(np.count_nonzero(~same))


def _requant_case(d, gemm, m, n, k, mult_vec, unsigned, zero_y, with_bias, seed, a_signed, b_signed):
    """RequantCase (Int8Tests.cs:375-466)."""
    a, b, za, mult, ib = cases.requant_case_data(m, n, k, mult_vec, seed)
    p = cases.problem(m, n, k, off_c=3)
    want = oracle.int8_gemm(p, a, a_signed, b, b_signed, (za, False, 0))
    expected = oracle.requant_array(want, n, mult, mult_vec, zero_y, unsigned, ib if with_bias else None)
    out = np.full(og.padded_bool_length(3 + m * n + 3) + 4, 0xA7, np.uint8)
    ba = d.CreateBuffer(as_i8(a) if a_signed else as_u8(a))
    bb = d.CreateBuffer(as_i8(b) if b_signed else as_u8(b))
    bz = d.CreateBuffer(as_i8(za) if a_signed else as_u8(za))
    bm, bib = d.CreateBuffer(mult), d.CreateBuffer(ib)
    y = d.CreateBuffer(out if unsigned else out.view(np.int8))
    run(d, lambda e: gemm.EncodeRequantized(e, to_problem(p), ba, bb, y, og.Int8Operand(bm, 0, mult_vec), zero_y,
                                            og.Int8Operand(bz, 0), None,
                                            og.Int8Operand(bib, 0, True) if with_bias else None))
    got = y.Read().view(np.uint8)
    bad = int(np.count_nonzero(got[3:3 + m * n] != expected))
    bad += int(np.count_nonzero(got[:3] != 0xA7)) + int(np.count_nonzero(got[3 + m * n:] != 0xA7))
    return bad


@pytest.mark.parametrize("config", ["default", "large tile"])
def test_float_and_requantized_forms_are_bit_exact(config):
    # FloatAndRequantizedFormsAreBitExact (Int8Tests.cs:468-501); "large tile" runs the same cases on the 256 x 256
    # kernels, whose epilogue is their own.
    d = device()
    gemm = dict(configs(d, True))[config]
    bad_f = bad_q = 0
    seed = 10
    for (m, n, k) in cases.FLOAT_SHAPES:
        for vec in (False, True):
            for ib, fb in ((False, False), (True, False), (False, True), (True, True)):
                say(f"float [{config}] {m}x{n}x{k} vec {vec} ib {ib} fb {fb}")
                bad_f += _float_case(d, gemm, m, n, k, vec, ib, fb, seed)
                seed += 1
        for vec in (False, True):
            for unsigned, zero in cases.REQUANT_OUT:
                say(f"requant [{config}] {m}x{n}x{k} vec {vec} u8 {unsigned} zero {zero}")
                bad_q += _requant_case(d, gemm, m, n, k, vec, unsigned, zero, (seed & 1) == 0, seed, (seed & 2) != 0,
                                       (seed & 4) != 0)
                seed += 1
    say(f"ROW float bits {bad_f} requant bytes {bad_q}")
    assert bad_f + bad_q == 0


# Shapes that reach every kernel: few rows on the tiled few-rows kernel (or split k), the 128 and 256 direct kernels
# (ragged M included), the register-staged 128 tile (K = 96), the generic kernel (unaligned rows), tiny products.
# The last three reach the one-launch few-rows kernel with its k-slices handed to the finishing tile (16 to 36 column
# slabs of 2 to 8 row bands), so its epilogues are checked after a real hand-off.
REQUANT_KERNEL_SHAPES = [(1, 1, 1), (5, 7, 9), (4, 272, 512), (16, 256, 1024), (64, 64, 96), (33, 257, 77),
                         (128, 384, 384), (130, 256, 512), (2, 8192, 128), (96, 208, 320), (3, 4608, 272),
                         (3, 4608, 1024), (4, 2048, 4096), (16, 2048, 2048)]
HANDOFF_SHAPES = REQUANT_KERNEL_SHAPES[-3:]


@pytest.mark.parametrize("fused", [True, False], ids=["one launch", "two passes"])
@pytest.mark.parametrize("config", list(CONFIG_OPTIONS))
def test_requantized_product_on_every_kernel(config, fused):
    # EncodeRequantized (Int8Gemm.cs:336-363) with the requantization in the product's store (one launch), and as the
    # reference runs it (the product into scratch, then Finish, 649-682), on each kernel a configuration reaches.
    d = device()
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config], FusedRequantize=fused))
    bad, seed, kernels = 0, 300, set()
    for (m, n, k) in REQUANT_KERNEL_SHAPES:
        for i, vec in enumerate((False, True, False, True)):
            unsigned, zero = cases.REQUANT_OUT[(seed + i) % len(cases.REQUANT_OUT)]
            say(f"requant [{config}, {'one launch' if fused else 'two passes'}] {m}x{n}x{k} vec {vec} u8 {unsigned} "
                f"zero {zero}")
            bad += _requant_case(d, gemm, m, n, k, vec, unsigned, zero, (seed & 1) == 0, seed, (seed & 2) != 0,
                                 (seed & 4) != 0)
            kernels.add(d.LastKernel)
            if fused and config == "default" and (m, n, k) in HANDOFF_SHAPES:
                assert d.LastKernel == "mfma-i8-rows16-xcd", d.LastKernel
            seed += 1
    say(f"ROW requantized [{config}, {'one launch' if fused else 'two passes'}] wrong bytes {bad}; kernels "
        f"{sorted(kernels)}")
    assert bad == 0
    if fused and config == "default":
        assert {"mfma-i8-rows16-tiles", "mfma-i8-rows16-xcd", "mfma-i8-direct128x128x64",
                "mfma-i8-tile128x128x128", "mfma-i8-generic128x128x64"} <= kernels, kernels
    if fused and config == "large tile":
        assert "mfma-i8-direct256x256x64" in kernels, kernels
    if not fused:
        assert kernels == {"int8-epilogue"}, kernels


# Activation scales for the scaled float product: ordinary, tiny (products in the denormal range, kept), huge
# (products that overflow to infinity) and NaN.
ACT_SCALES = [0.0123, 3.7e-3, 1e-30, 3e36, float("nan")]


@pytest.mark.parametrize("config", list(CONFIG_OPTIONS))
def test_scaled_float_product_on_every_kernel(config):
    # EncodeFloatScaled: MatMulIntegerToFloat with the column scale fl(actScale * wScale[n]) made in the product's
    # epilogue. Expected: numpy's float32 product (IEEE, round to nearest even) as the scale vector, then the oracle's
    # float steps (Int8Tests.cs:356-373), i.e. the reference's Mul + EncodeFloat chain.
    d = device()
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config]))
    bad, seed, kernels = 0, 700, set()
    for (m, n, k) in REQUANT_KERNEL_SHAPES:
        for i, vec in enumerate((True, False)):
            act = np.float32(ACT_SCALES[(seed + i) % len(ACT_SCALES)])
            with_ib, with_fb = (seed & 1) == 0, (seed & 2) == 0
            a, b, za, zb, wscale, ib, fb = cases.float_case_data(m, n, k, vec, seed)
            p = cases.problem(m, n, k)
            sums = oracle.int8_gemm(p, a, False, b, True, (za, False, 0), (zb, True, 0))
            with np.errstate(all="ignore"):
                colscale = (act * wscale.astype(np.float32)).astype(np.float32)
            expected = oracle.float_epilogue(sums, n, colscale, vec, ib if with_ib else None, fb if with_fb else None)
            say(f"scaled float [{config}] {m}x{n}x{k} vec {vec} act {act} ib {with_ib} fb {with_fb}")
            ba, bb = d.CreateBuffer(as_u8(a)), d.CreateBuffer(as_i8(b))
            bza, bzb = d.CreateBuffer(as_u8(za)), d.CreateBuffer(as_i8(zb))
            bs, bib, bfb = d.CreateBuffer(wscale), d.CreateBuffer(ib), d.CreateBuffer(fb)
            bact = d.CreateBuffer(np.array([0.0, act], np.float32))
            bc = d.CreateBufferOf(og.ElementType.Float32, m * n)
            run(d, lambda e: gemm.EncodeFloatScaled(e, to_problem(p), ba, bb, bc, og.Int8Operand(bact, 1),
                                                    og.Int8Operand(bs, 0, vec), og.Int8Operand(bza, 0),
                                                    og.Int8Operand(bzb, 0, True),
                                                    og.Int8Operand(bfb, 0, True) if with_fb else None,
                                                    og.Int8Operand(bib, 0, True) if with_ib else None))
            got = bc.Read()
            same = np.where(np.isnan(expected), np.isnan(got), got.view(np.uint32) == expected.view(np.uint32))
            bad += int(np.count_nonzero(~same))
            kernels.add(d.LastKernel)
            if config == "default" and (m, n, k) in HANDOFF_SHAPES:
                assert d.LastKernel == "mfma-i8-rows16-xcd", d.LastKernel
            seed += 1
    say(f"ROW scaled float [{config}] wrong values {bad}; kernels {sorted(kernels)}")
    assert bad == 0


@pytest.mark.parametrize("fused", [True, False], ids=["one launch", "two passes"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (4, 256, 64), (128, 128, 64)])
def test_requantization_rounds_half_to_even_and_saturates(shape, fused):
    # Int8Tests.cs:503-547 (there on a 1 x 1 x 1 product); here also on the few-rows tiled kernel and the 128 direct
    # kernel. Row m of A starts with the value under test and B's first row is all ones, so every byte of output row m
    # is that value requantized (rows past the values hold 0).
    m_, n_, k_ = shape
    d = device()
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(FusedRequantize=fused))
    bad = 0
    values = list(range(-9, 10))
    for mult, zero_y, unsigned in cases.REQUANT_TIES:
        for c0 in range(0, len(values), m_):
            avs = values[c0:c0 + m_]
            a = np.zeros((m_, k_), np.int8)
            a[:len(avs), 0] = avs
            b = np.zeros((k_, n_), np.int8)
            b[0, :] = 1
            with np.errstate(all="ignore"):
                want = np.array([oracle.requant(av, mult, zero_y, unsigned) & 0xFF for av in avs]
                                + [oracle.requant(0, mult, zero_y, unsigned) & 0xFF] * (m_ - len(avs)), np.uint8)
            ba, bb = d.CreateBuffer(a.ravel()), d.CreateBuffer(b.ravel())
            bm = d.CreateBuffer(np.array([mult], np.float32))
            y = d.CreateBufferOf(og.ElementType.UInt8 if unsigned else og.ElementType.Int8, m_ * n_)
            run(d, lambda e: gemm.EncodeRequantized(e, og.Int8GemmProblem(m_, n_, k_), ba, bb, y, og.Int8Operand(bm, 0),
                                                    zero_y))
            got = y.Read().view(np.uint8)[:m_ * n_].reshape(m_, n_)
            bad += int(np.count_nonzero(got != want[:, None]))
    say(f"ROW requantization ties {shape} {'one launch' if fused else 'two passes'}: wrong bytes {bad}, kernel "
        f"{d.LastKernel}")
    assert bad == 0


def test_dynamic_quantize_is_bit_exact():
    # DynamicQuantizeIsBitExact (Int8Tests.cs:617-703)
    d = device()
    k = og.DynamicQuantizeKernels(d)
    bad = 0
    OffX, OffY, OffS, OffZ = 1, 3, 2, 5
    for count, kind, seed in cases.dq_cases():
        say(f"dq count {count} kind {kind}")
        x = oracle.dq_input(count, seed, kind)
        wy, ws, wz = oracle.dynamic_quantize(x)
        xs = np.zeros(count + OffX, np.float32)
        xs[OffX:] = x
        bx = d.CreateBuffer(xs)
        y_init = np.full(((OffY + count + 3) & ~3) + 4, 0x3C, np.uint8)
        by = d.CreateBuffer(y_init)
        bs = d.CreateBufferOf(og.ElementType.Float32, 4)
        bz = d.CreateBuffer(np.full(8, 0xEE, np.uint8))
        run(d, lambda e: k.Encode(e, bx, OffX, count, by, OffY, bs, OffS, bz, OffZ))
        y, sc, zp = by.Read(), bs.Read(), bz.Read()
        here = int(np.count_nonzero(y[OffY:OffY + count] != wy))
        here += int(sc[OffS].view(np.uint32) != np.float32(ws).view(np.uint32)) + int(zp[OffZ] != wz)
        here += int(np.count_nonzero(y[:OffY] != 0x3C)) + int(np.count_nonzero(y[OffY + count:] != 0x3C))
        here += int(np.count_nonzero(np.delete(zp, OffZ) != 0xEE))
        if here:
            say(f"MISMATCH dq count {count} kind {kind}: {here} (scale {sc[OffS]!r} want {ws!r}, zero {zp[OffZ]} want {wz})")
        bad += here
    assert bad == 0


def test_dynamic_quantize_large_inputs():
    # Inputs past one pass of the quantize grid (2048 workgroups x 256 threads x 16 elements = 8,388,608): the
    # grid-stride loop, aligned and unaligned x and y, a ragged tail; the minimum and maximum placed in the last
    # elements, so the workgroup that reads them is one of the last.
    d = device()
    k = og.DynamicQuantizeKernels(d)
    bad = 0
    for count, off in ((9_000_003, 0), (8_388_608 * 2 + 5, 1)):
        x = oracle.dq_input(count, 31 + off, 0)
        x[-1], x[-2] = np.float32(7.5), np.float32(-6.25)
        say(f"dq large count {count} offset {off}")
        wy, ws, wz = oracle.dynamic_quantize(x)
        xs = np.zeros(count + off, np.float32)
        xs[off:] = x
        bx, by = d.CreateBuffer(xs), d.CreateBufferOf(og.ElementType.UInt8, count + off + 4)
        bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
        run(d, lambda e: k.Encode(e, bx, off, count, by, off, bs, 0, bz, 0))
        y = by.Read()[off:off + count]
        here = int(np.count_nonzero(y != wy)) + int(bs.Read()[0].view(np.uint32) != np.float32(ws).view(np.uint32))
        here += int(bz.Read()[0] != wz)
        if here:
            say(f"MISMATCH dq large count {count}: {here}")
        bad += here
    assert bad == 0


def test_dynamic_quantize_in_sequence():
    # Consecutive launches of different sizes and ranges on one device, each checked against the oracle: nothing of
    # one launch's ranges may leak into the next (the per-workgroup ranges live in a workspace the launches share).
    # Large and small launches alternate, so a larger launch's ranges past a smaller one's groups are still in the
    # workspace when the smaller one runs.
    d = device()
    k = og.DynamicQuantizeKernels(d)
    counts = [2_097_152, 1, 4097, 786_432, 2_097_153, 65_536, 2_000_001, 3, 1_048_577, 2_097_152, 257, 786_432,
              4_194_304, 4_194_303, 6_000_007, 6_000_007, 5, 4_194_305, 8_388_608]
    for i, count in enumerate(counts):
        kind = i % 7
        x = oracle.dq_input(count, 900 + i, kind)
        if i % 4 == 1:
            x = -np.abs(x)   # all-negative ranges: lo far from zero, hi = 0
        say(f"dq sequence {i}: count {count} kind {kind}")
        wy, ws, wz = oracle.dynamic_quantize(x)
        bx, by = d.CreateBuffer(x), d.CreateBufferOf(og.ElementType.UInt8, count + 4)
        bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
        run(d, lambda e: k.Encode(e, bx, 0, count, by, 0, bs, 0, bz, 0))
        here = int(np.count_nonzero(by.Read()[:count] != wy))
        here += int(bs.Read()[0].view(np.uint32) != np.float32(ws).view(np.uint32)) + int(bz.Read()[0] != wz)
        assert here == 0, f"launch {i}, count {count}: {here} wrong"


def test_dynamic_quantize_special_values():
    d = device()
    k = og.DynamicQuantizeKernels(d)
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    for x in ([0.0], [-0.0, 0.0], [nan, nan], [1.0, nan, -1.0], [inf, 1.0], [-inf, 2.0], [1e-42, 3e-42], [-1e-42],
              [1e30, -1e30], [255.0, 0.0], [-3.0, -2.0], [3e38, -3e38]):
        x = np.array(x, np.float32)
        wy, ws, wz = oracle.dynamic_quantize(x)
        bx, by = d.CreateBuffer(x), d.CreateBufferOf(og.ElementType.UInt8, 4)
        bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
        run(d, lambda e: k.Encode(e, bx, 0, x.size, by, 0, bs, 0, bz, 0))
        assert by.Read()[:x.size].tolist() == wy.tolist(), x
        s = bs.Read()[0]
        assert (np.isnan(s) and np.isnan(ws)) or s.view(np.uint32) == np.float32(ws).view(np.uint32), x
        assert bz.Read()[0] == wz, x


def test_dynamic_quantize_feeds_the_product_without_leaving_the_device():
    # Int8Tests.cs:705-751: DQ, the on-device scale product, MatMulIntegerToFloat, in stream order.
    d = device()
    dq, gemm = og.DynamicQuantizeKernels(d), og.Int8Gemm(d)
    M, N, K = 128, 384, 384
    x = oracle.rig_random(M * K, 3, -3.0, 5.0)
    wy, wscale, wzero = oracle.dynamic_quantize(x)
    w = oracle.bytes_(N * K, 4)
    wscales = (np.float32(0.002) + (np.arange(N) % 17).astype(np.float32) * np.float32(1e-4)).astype(np.float32)
    p = cases.problem(M, N, K, trans_b=True)
    sums = oracle.int8_gemm(p, wy, False, w, True, (np.array([wzero], np.uint8), False, 0))
    bx, by = d.CreateBuffer(x), d.CreateBufferOf(og.ElementType.UInt8, M * K)
    bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 1)
    bw, bws = d.CreateBuffer(as_i8(w)), d.CreateBuffer(wscales)
    bscale, bc = d.CreateBufferOf(og.ElementType.Float32, N), d.CreateBufferOf(og.ElementType.Float32, M * N)
    run(d, lambda e: dq.Encode(e, bx, 0, M * K, by, 0, bs, 0, bz, 0))
    check(abi().og_util_scale_product(d.Context, binding(bs), binding(bws), N, binding(bscale)), d)
    run(d, lambda e: gemm.EncodeFloat(e, to_problem(p), by, bw, bc, og.Int8Operand(bscale, 0, True), og.Int8Operand(bz, 0)))
    got = bc.Read()
    want = sums.astype(np.float32) * (np.float32(wscale) * wscales[np.arange(M * N) % N])
    assert np.count_nonzero(got.view(np.uint32) != want.astype(np.float32).view(np.uint32)) == 0


def test_products_wider_than_one_grid_axis_are_bit_exact():
    # ConvIntegerTests.cs:343-390: more than 65535 tiles along one axis.
    d = device()
    for (m, n) in ((3, 4_300_001), (4_300_001, 3), (2, 4_194_241)):
        k = 5
        a, b = oracle.bytes_(m * k, 11), oracle.bytes_(k * n, 12)
        za, zb = oracle.bytes_(1, 13), oracle.bytes_(n, 14)
        p = oracle.Gemm(m, n, k)
        want = oracle.int8_gemm(p, a, False, b, True, (za, False, 0), (zb, True, 0))
        ba, bb = d.CreateBuffer(as_u8(a)), d.CreateBuffer(as_i8(b))
        bza, bzb = d.CreateBuffer(as_u8(za)), d.CreateBuffer(as_i8(zb))
        for opts in (og.Int8GemmOptions(), og.Int8GemmOptions(AllowPackedDot=False), og.Int8GemmOptions(Tile=64)):
            say(f"wide {m}x{n} allow {opts.AllowPackedDot} tile {opts.Tile}")
            gemm = og.Int8Gemm(d, opts)
            bc = d.CreateBufferOf(og.ElementType.Int32, m * n)
            run(d, lambda e: gemm.EncodeInt32(e, og.Int8GemmProblem(m, n, k), ba, bb, bc, og.Int8Operand(bza, 0),
                                              og.Int8Operand(bzb, 0, True)))
            got = bc.Read()
            assert np.count_nonzero(got != want) == 0, (m, n, d.LastKernel)
            bc.Dispose()


@pytest.mark.parametrize("config, k, want_kernel", [
    ("default", 128, "mfma-i8-direct128x128x64"), ("large tile", 128, "mfma-i8-direct256x256x64"),
    ("default", 96, "mfma-i8-tile128x128x128"), ("large tile", 96, "mfma-i8-tile256x256x64")])
def test_padded_rows_of_b_with_a_ragged_width(config, k, want_kernel):
    # B stored K x N in rows of Ldb > N bytes with N not a multiple of 4 (ConvInteger's column matrices have this
    # shape): the final dword of B's last row holds valid columns and padding, and every column must come through.
    d = device()
    gemm = dict(configs(d, True))[config]
    m, n, ldb = 200, 750, 752
    rng = np.random.default_rng(k)
    a = rng.integers(0, 256, m * k, dtype=np.uint8)
    b = rng.integers(0, 256, k * ldb, dtype=np.uint8)
    za, zb = np.array([7], np.uint8), rng.integers(0, 256, n, dtype=np.uint8)
    p = oracle.Gemm(m, n, k, Ldb=ldb)
    want = oracle.int8_gemm(p, a, False, b, True, (za, False, 0), (zb, True, 0))
    ba, bb = d.CreateBuffer(a), d.CreateBuffer(b.view(np.int8))
    bza, bzb = d.CreateBuffer(za), d.CreateBuffer(zb.view(np.int8))
    bc = d.CreateBufferOf(og.ElementType.Int32, m * n)
    q = og.Int8GemmProblem(m, n, k)
    q.Ldb = ldb
    run(d, lambda e: gemm.EncodeInt32(e, q, ba, bb, bc, og.Int8Operand(bza, 0), og.Int8Operand(bzb, 0, True)))
    assert d.LastKernel == want_kernel
    bad = int(np.count_nonzero(bc.Read() != want))
    say(f"ROW padded B rows, N = 750 in rows of 752 [{d.LastKernel}]: {bad} elements differ")
    assert bad == 0


def test_b_ending_at_its_last_valid_byte_takes_another_kernel():
    # The same product through the C ABI with B's buffer declared to end at its last valid byte: the dword-wide reads
    # of the aligned kernels would leave it, so a kernel with byte-exact reads runs instead, with the same sums.
    d = device()
    m, n, k, ldb = 200, 750, 128, 752
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, m * k, dtype=np.uint8)
    b = rng.integers(0, 256, k * ldb, dtype=np.uint8)
    want = oracle.int8_gemm(oracle.Gemm(m, n, k, Ldb=ldb), a, False, b, True)
    ba, bb = d.CreateBuffer(a), d.CreateBuffer(b.view(np.int8))
    bc = d.CreateBufferOf(og.ElementType.Int32, m * n)
    L = abi()
    prm = L.GemmParams(M=m, N=n, K=k, Lda=k, Ldb=ldb, Flags=0x002, StrideC=m * n)
    none = L.Buf(None, 0)
    exact = L.Buf(bb.DevicePointer, (k - 1) * ldb + n)
    check(L.og_int8_gemm(d.Context, ctypes.byref(prm), 1, binding(ba), exact, binding(bc), none, none, none, none,
                         none), d)
    d.WaitIdle()
    kernel = L.og_last_kernel(d.Context).decode()
    assert "direct" not in kernel and "tile" not in kernel, kernel
    assert np.array_equal(bc.Read(), want)
    check(L.og_int8_gemm(d.Context, ctypes.byref(prm), 1, binding(ba), binding(bb), binding(bc), none, none, none,
                         none, none), d)
    d.WaitIdle()
    assert L.og_last_kernel(d.Context).decode() == "mfma-i8-direct128x128x64"
    assert np.array_equal(bc.Read(), want)


# Products whose 128 x 128 grid fills under half the chip and whose K has at least 8 stages: split along K.
SPLIT_SHAPES = [  # m, n, k, batch, transposed B
    (256, 256, 2304, 1, False), (200, 384, 1536, 1, False), (128, 256, 2048, 2, False), (1, 11008, 4096, 1, True),
    (130, 128, 4096, 1, True)]


@pytest.mark.parametrize("m, n, k, batch, trans", SPLIT_SHAPES)
def test_split_k_products_are_bit_exact(m, n, k, batch, trans):
    # The k slices each apply the zero points to their own range (every correction term is linear in the range);
    # the summing pass adds them and applies the bias and the epilogue: int32, float (scale, float bias), scaled
    # float and requantized outputs, both operand signednesses, zero points per row and column.
    d = device()
    gemm = og.Int8Gemm(d)
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(0, 256, batch * m * k, dtype=np.uint8)
    b = rng.integers(0, 256, batch * n * k, dtype=np.uint8)
    za, zb = rng.integers(0, 256, m, dtype=np.uint8), rng.integers(0, 256, n, dtype=np.uint8)
    ib = rng.integers(-5000, 5000, n).astype(np.int32)
    scale = (rng.random(n, dtype=np.float32) * np.float32(1e-4)).astype(np.float32)
    fb = rng.standard_normal(n).astype(np.float32)
    mult = (rng.random(n, dtype=np.float32) * np.float32(2e-6)).astype(np.float32)
    act = np.float32(0.37)
    p = oracle.Gemm(m, n, k, Batch=batch, TransposeB=int(trans), StrideA=m * k, StrideB=n * k)
    bad = 0
    for a_signed, b_signed in ((False, True), (True, False), (True, True)):
        sums = oracle.int8_gemm(p, a, a_signed, b, b_signed, (za, True, 0), (zb, True, 0))
        ba = d.CreateBuffer(a.view(np.int8) if a_signed else a)
        bb = d.CreateBuffer(b.view(np.int8) if b_signed else b)
        bza = d.CreateBuffer(za.view(np.int8) if a_signed else za)
        bzb = d.CreateBuffer(zb.view(np.int8) if b_signed else zb)
        q = to_problem(p)
        zpa, zpb = og.Int8Operand(bza, 0, True), og.Int8Operand(bzb, 0, True)
        bib, bsc, bfb = d.CreateBuffer(ib), d.CreateBuffer(scale), d.CreateBuffer(fb)
        # int32 with bias
        bc = d.CreateBufferOf(og.ElementType.Int32, batch * m * n)
        run(d, lambda e: gemm.EncodeInt32(e, q, ba, bb, bc, zpa, zpb, og.Int8Operand(bib, 0, True)))
        assert d.LastKernel == "mfma-i8-direct128x128x64-splitk", d.LastKernel
        want = (sums.astype(np.int64) + np.tile(ib, batch * m)).astype(np.int64)
        bad += int(np.count_nonzero(bc.Read() != ((want & 0xFFFFFFFF).astype(np.uint32).view(np.int32))))
        # float with scale per column and float bias
        bf = d.CreateBufferOf(og.ElementType.Float32, batch * m * n)
        run(d, lambda e: gemm.EncodeFloat(e, q, ba, bb, bf, og.Int8Operand(bsc, 0, True), zpa, zpb,
                                          og.Int8Operand(bfb, 0, True), og.Int8Operand(bib, 0, True)))
        wantf = oracle.float_epilogue(sums, n, scale, True, ib, fb)
        bad += int(np.count_nonzero(bf.Read().view(np.uint32) != wantf.view(np.uint32)))
        # scaled float: the column scale fl(act * scale[n])
        bact = d.CreateBuffer(np.array([act], np.float32))
        run(d, lambda e: gemm.EncodeFloatScaled(e, q, ba, bb, bf, og.Int8Operand(bact, 0), og.Int8Operand(bsc, 0, True),
                                                zpa, zpb))
        wants = oracle.float_epilogue(sums, n, (act * scale).astype(np.float32), True)
        bad += int(np.count_nonzero(bf.Read().view(np.uint32) != wants.view(np.uint32)))
        # requantized bytes
        by = d.CreateBufferOf(og.ElementType.UInt8, batch * m * n)
        bm = d.CreateBuffer(mult)
        run(d, lambda e: gemm.EncodeRequantized(e, q, ba, bb, by, og.Int8Operand(bm, 0, True), 131, zpa, zpb,
                                                og.Int8Operand(bib, 0, True)))
        wantq = oracle.requant_array(sums, n, mult, True, 131, True, ib)
        bad += int(np.count_nonzero(by.Read()[:batch * m * n] != wantq))
    say(f"ROW split-k {m}x{n}x{k} batch {batch} {'N x K' if trans else 'K x N'}: wrong values {bad}")
    assert bad == 0


def test_scratch_semantics():
    # Int8ScratchTests.cs:27-89
    d = device()
    N, K, Small, Large = 96, 64, 32, 160
    a = d.CreateBuffer(oracle.bytes_(Large * K + 4, 1))
    b = d.CreateBuffer(np.zeros(N * K + 4, np.int8))
    y = d.CreateBufferOf(og.ElementType.UInt8, Large * N + 4)
    mult = og.Int8Operand(d.CreateBuffer(np.array([0.001], np.float32)), 0)
    need = og.Int8Gemm.ScratchElements(og.Int8GemmProblem(Large, N, K))
    assert need == Large * N
    scratch = d.CreateBufferOf(og.ElementType.Int32, need)

    def pair(gemm, given):
        # The argument blocks the larger product adds after the smaller one (Int8ScratchTests.Pair).
        run(d, lambda e: gemm.EncodeRequantized(e, og.Int8GemmProblem(Small, N, K), a, b, y, mult, 3, scratch=given))
        first = gemm.BindGroupsCreated
        run(d, lambda e: gemm.EncodeRequantized(e, og.Int8GemmProblem(Large, N, K), a, b, y, mult, 3, scratch=given))
        return gemm.BindGroupsCreated - first

    for fused in (True, False):
        opts = og.Int8GemmOptions(FusedRequantize=fused)
        # The caller's scratch, sized once for the largest product: nothing new for the larger one.
        assert pair(og.Int8Gemm(d, opts), og.Int8Scratch(scratch)) == 0
        # Reserving the instance's own scratch up front does the same.
        gemm = og.Int8Gemm(d, opts)
        gemm.ReserveScratch(need)
        assert pair(gemm, None) == 0
        assert y.Read()[:Large * N].tolist() == [3] * (Large * N)   # B = 0: every sum is 0, so y = zeroPointY
        # Without either, the two-pass form's sums buffer grows and the larger product needs a new block.
        assert pair(og.Int8Gemm(d, opts), None) >= 0
    small = d.CreateBufferOf(og.ElementType.Int32, 100)
    with pytest.raises(og.GpuKernelShapeException) as ex:
        gemm.EncodeRequantized(d.BeginCommands(), og.Int8GemmProblem(64, 64, 8), a, b, y, mult, 0, scratch=og.Int8Scratch(small))
    assert ex.value.Argument == "scratch"


@pytest.mark.parametrize("config", ["tiles", "tiles two launches", "split k"])
def test_few_rows_kernels_are_bit_exact(config):
    # The few-rows products (M <= 16, B stored K x N) on the tiled kernel, in one launch (the last tile of a column slab
    # adds the slab's parts; shapes with at least 16 slabs) or two (a second kernel adds them), and on the split-k one
    # (partial sums per k-slice, then their sum): one slab or many, one tile per slab or several, K past the last full
    # tile or 64 rows, N past the last full slab, M = 16 (no spare MFMA row), batches, every signedness and zero-point
    # form, configuration 3's shape at M = 1, 4 and 16; one case three times in a row and a smaller M after a larger
    # one. Aligned operands; the tiled kernel takes K and N multiples of 16, the split-k one the rest.
    d = device()
    opts = {"tiles": og.Int8GemmOptions(), "tiles two launches": og.Int8GemmOptions(FewRowsOneLaunch=False),
            "split k": og.Int8GemmOptions(Tile=32)}[config]
    gemm = og.Int8Gemm(d, opts)
    shapes = [(1, 16, 4, 1), (1, 256, 64, 1), (4, 272, 100, 1), (16, 1024, 4096, 1), (7, 528, 1500, 1),
              (16, 4096, 64, 1), (2, 4096, 8192, 1), (3, 512, 320, 3), (1, 11008, 4096, 1), (5, 48, 12, 2),
              (16, 272, 4112, 2), (1, 32768, 512, 1), (15, 1040, 272, 1), (2, 1040, 272, 1),
              (16, 8208, 1040, 1), (7, 4112, 336, 2), (4, 8192, 16, 1), (3, 12288, 64, 1), (1, 8192, 8192, 1),
              (13, 8256, 208, 1), (4, 11008, 4096, 1), (16, 11008, 4096, 1), (8, 2048, 2048, 8)]
    bad_total, kernels = 0, set()
    for i, (m, n, k, batch) in enumerate(shapes):
        a_s, b_s = (i & 1) != 0, (i & 2) == 0
        za_mode, zb_mode = i % 3, (i // 3) % 3
        c = cases.Case(f"rows {m}x{n}x{k} b{batch}", cases.problem(m, n, k, batch=batch), a_s, b_s, za_mode, zb_mode)
        tiled = config != "split k" and k % 16 == 0 and n % 16 == 0
        one_launch = config == "tiles" and batch * ((n + 127) // 128) >= 16
        for rep in range(3 if i == 2 or i == 8 else 1):
            say(f"{config} case {c.name} signed {a_s}/{b_s} zp {za_mode}/{zb_mode} rep {rep}")
            bad, kernel = run_int32(d, gemm, c, 100 + i)
            d.WaitIdle()   # reports a one-launch product whose parts never arrived
            if bad:
                say(f"  {kernel}: {bad} wrong")
            kernels.add(kernel)
            if tiled:
                assert kernel == ("mfma-i8-rows16-xcd" if one_launch else "mfma-i8-rows16-tiles"), kernel
            else:
                assert kernel in ("mfma-i8-rows16-splitk", "mfma-i8-rows16-direct"), kernel
            bad_total += bad
    for vec in (False, True):
        say(f"{config} float vec {vec}")
        bad_total += _float_case(d, gemm, 4, 256, 128, vec, True, True, 77 + vec)
        bad_total += _float_case(d, gemm, 16, 1024, 512, vec, False, True, 79 + vec)
        bad_total += _float_case(d, gemm, 3, 8192, 192, vec, True, True, 81 + vec)
        # Column slabs of 8, 2 and 4 row bands: the finishing tile's float store after a real hand-off.
        for j, (m, n, k) in enumerate(HANDOFF_SHAPES):
            bad_total += _float_case(d, gemm, m, n, k, vec, j != 1, j != 0, 83 + 2 * j + vec)
            if config == "tiles":
                assert d.LastKernel == "mfma-i8-rows16-xcd", d.LastKernel
    say(f"ROW int8 gemm | few rows [{config}] | mismatches {bad_total}; kernels {sorted(kernels)}")
    assert bad_total == 0


@pytest.mark.parametrize("m", [1, 4, 16])
def test_c3_matmul_integer_to_float_few_rows(m):
    # Configuration 3 as the decode layer runs it: DynamicQuantizeLinear of N(0, 1) activations [m x 4096], then
    # MatMulIntegerToFloat with int8 weights [4096 x 11008] quantized symmetric per column from N(0, 0.02), the column
    # scale fl(actScale * wScale[n]) made in the product's epilogue (EncodeFloatScaled) and, as the reference chains
    # it, the scale vector made first (EncodeFloat). The one-launch few-rows kernel hands 8 k-slices of each of 86
    # column slabs to the slab's finishing tile. Against the oracle: DQ's bytes, scale and zero point, then every
    # output bit.
    K, N = 4096, 11008
    d = device()
    rng = np.random.default_rng(900 + m)
    x = rng.standard_normal(m * K).astype(np.float32)
    w = (rng.standard_normal(K * N) * 0.02).astype(np.float32).reshape(K, N)
    wscale = (np.abs(w).max(axis=0).astype(np.float32) / np.float32(127)).astype(np.float32)
    wq = oracle.quantize(w.ravel(), wscale, True, per_axis=True, axis_len=N, inner=1).view(np.int8)
    y_want, s_want, z_want = oracle.dynamic_quantize(x)
    bx, bq, bws = d.CreateBuffer(x), d.CreateBuffer(wq), d.CreateBuffer(wscale)
    by = d.CreateBufferOf(og.ElementType.UInt8, m * K)
    bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
    say(f"c3 float m {m}: DynamicQuantizeLinear")
    run(d, lambda e: og.DynamicQuantizeKernels(d).Encode(e, bx, 0, m * K, by, 0, bs, 0, bz, 0))
    y, s, z = by.Read()[:m * K], np.float32(bs.Read()[0]), int(bz.Read()[0])
    assert np.array_equal(y, y_want) and s == np.float32(s_want) and z == z_want
    sums = oracle.int8_gemm(cases.problem(m, N, K), y, False, wq.view(np.uint8), True, (np.array([z], np.uint8), False, 0))
    colscale = (s * wscale).astype(np.float32)
    want = oracle.float_epilogue(sums, N, colscale, True)
    gemm = og.Int8Gemm(d)
    p = og.Int8GemmProblem(m, N, K)
    for form in ("scaled in the epilogue", "scale vector first"):
        bc = d.CreateBufferOf(og.ElementType.Float32, m * N)
        say(f"c3 float m {m}: MatMulIntegerToFloat, {form}")
        if form == "scaled in the epilogue":
            run(d, lambda e: gemm.EncodeFloatScaled(e, p, by, bq, bc, og.Int8Operand(bs, 0), og.Int8Operand(bws, 0, True),
                                                    og.Int8Operand(bz, 0)))
        else:
            bsc = d.CreateBufferOf(og.ElementType.Float32, N)
            run(d, lambda e: (e.RecordScaleProduct(bs, bws, N, bsc),
                              gemm.EncodeFloat(e, p, by, bq, bc, og.Int8Operand(bsc, 0, True), og.Int8Operand(bz, 0))))
        d.WaitIdle()
        assert d.LastKernel == "mfma-i8-rows16-xcd", d.LastKernel
        got = bc.Read()
        bad = int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))
        say(f"ROW c3 MatMulIntegerToFloat m {m} ({form}): {bad} wrong values")
        assert bad == 0


@pytest.mark.parametrize("fused", [True, False], ids=["one launch", "two passes"])
@pytest.mark.parametrize("shape", [(64, 256, 512, 128), (4, 4096, 2048, 4096)], ids=["tiles", "few rows"])
def test_chained_qlinear_matmul(shape, fused):
    # The QLinearMatMul model format (docs/kernels.md:160-162; Int8Tests.cs:375-466 per layer): layer 1's requantized
    # uint8 output, with its zero point, is layer 2's A operand with that zero point; layer 2 requantizes to int8. The
    # two-pass form places both layers' int32 sums in one caller scratch buffer (Int8Scratch, at element offsets past
    # each other). Every byte of both layers against the oracle.
    m, k1, n1, n2 = shape
    d = device()
    rng = np.random.default_rng(950 + m)
    a = rng.integers(0, 256, m * k1, dtype=np.uint8)
    za = np.array([rng.integers(90, 160)] * 4, np.uint8)
    b1 = rng.integers(-127, 128, k1 * n1, dtype=np.int8)
    b2 = rng.integers(-127, 128, n1 * n2, dtype=np.int8)
    # Multipliers that spread each layer's bytes over about +-20 around its zero point (a few saturate): a sum of K
    # products of a - za (RMS ~74) and b (RMS ~73) with random signs spreads over about sqrt(K) * 5400.
    mult1 = ((rng.random(n1) + 0.5) * 20.0 / (np.sqrt(k1) * 5400.0)).astype(np.float32)
    mult2 = np.array([15.0 / (np.sqrt(n1) * 25.0 * 73.0)], np.float32)
    zy1, zy2 = 117, -5
    s1 = oracle.int8_gemm(cases.problem(m, n1, k1), a, False, b1.view(np.uint8), True, (za[:1], False, 0))
    y1 = oracle.requant_array(s1, n1, mult1, True, zy1, True)
    s2 = oracle.int8_gemm(cases.problem(m, n2, n1), y1, False, b2.view(np.uint8), True, (np.array([zy1], np.uint8), False, 0))
    y2 = oracle.requant_array(s2, n2, mult2, False, zy2, False)
    assert 10 < len(np.unique(y1)) and 10 < len(np.unique(y2)), "the layers' outputs span many values"
    ba, bza, bb1, bb2 = d.CreateBuffer(a), d.CreateBuffer(za), d.CreateBuffer(b1), d.CreateBuffer(b2)
    bm1, bm2 = d.CreateBuffer(mult1), d.CreateBuffer(mult2)
    by1 = d.CreateBufferOf(og.ElementType.UInt8, m * n1)
    by2 = d.CreateBufferOf(og.ElementType.Int8, m * n2)
    bzy1 = d.CreateBuffer(np.full(4, zy1, np.uint8))
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(FusedRequantize=fused))
    p1, p2 = og.Int8GemmProblem(m, n1, k1), og.Int8GemmProblem(m, n2, n1)
    e1 = og.Int8Gemm.ScratchElements(p1)
    scratch = d.CreateBufferOf(og.ElementType.Int32, e1 + og.Int8Gemm.ScratchElements(p2) + 8)
    say(f"chained qlinear {shape} {'one launch' if fused else 'two passes'}")

    def record(e):
        gemm.EncodeRequantized(e, p1, ba, bb1, by1, og.Int8Operand(bm1, 0, True), zy1, og.Int8Operand(bza, 0),
                               scratch=og.Int8Scratch(scratch, 0))
        gemm.EncodeRequantized(e, p2, by1, bb2, by2, og.Int8Operand(bm2, 0), zy2, og.Int8Operand(bzy1, 0),
                               scratch=og.Int8Scratch(scratch, e1 + 8))
    run(d, record)
    d.WaitIdle()
    got1, got2 = by1.Read()[:m * n1], by2.Read().view(np.uint8)[:m * n2]
    bad1 = int(np.count_nonzero(got1 != y1))
    bad2 = int(np.count_nonzero(got2 != y2.view(np.uint8)))
    say(f"ROW chained QLinearMatMul {shape} ({'one launch' if fused else 'two passes'}, {d.LastKernel}): wrong bytes "
        f"{bad1} + {bad2}")
    assert bad1 + bad2 == 0


def test_golden_fixtures_on_every_kernel():
    # The committed smoke and closed-form fixtures (tests/golden) through every kernel the chooser and the test hooks
    # reach, bit for bit.
    import os
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    f = np.load(os.path.join(golden, "c1_smoke.npz"), allow_pickle=False)
    m, n, k = (int(v) for v in f["shape"])
    cf = np.load(os.path.join(golden, "closed_form.npz"), allow_pickle=False)
    d = device()
    ba, bb = d.CreateBuffer(f["a"]), d.CreateBuffer(f["b"])
    bza, bzb = d.CreateBuffer(f["za"]), d.CreateBuffer(f["zb"])
    ca, cb = d.CreateBuffer(cf["a"]), d.CreateBuffer(cf["b"])
    bad = 0
    for config, gemm in configs(d, True):
        c = d.CreateBufferOf(og.ElementType.Int32, m * n)
        run(d, lambda e: gemm.EncodeInt32(e, og.Int8GemmProblem(m, n, k), ba, bb, c, og.Int8Operand(bza, 0),
                                          og.Int8Operand(bzb, 0, True)))
        got = c.Read()
        say(f"golden smoke [{config}] {d.LastKernel}: {int(np.count_nonzero(got != f['c']))} mismatches")
        bad += int(np.count_nonzero(got != f["c"]))
        c2 = d.CreateBufferOf(og.ElementType.Int32, 6)
        run(d, lambda e: gemm.EncodeInt32(e, og.Int8GemmProblem(2, 3, 2), ca, cb, c2))
        bad += int(np.count_nonzero(c2.Read() != cf["c"]))
    assert bad == 0


@pytest.mark.parametrize("config", ["default", "tiled only", "large tile"])
def test_seeded_random_products_are_bit_exact(config):
    # A seeded sweep beyond the reference's case lists: shapes, batches (shared or distinct B), both layouts of B,
    # signedness and zero-point modes, in three kinds of case: aligned rows with K a multiple of 64 (the direct and
    # few-rows kernels), aligned rows with K a multiple of 16 only (the register-staged tiles), and odd offsets with
    # padded rows (the generic kernel). Every product against the oracle, sentinels included.
    d = device()
    gemm = dict(configs(d, True))[config]
    rng = np.random.default_rng({"default": 11, "tiled only": 12, "large tile": 13}[config])
    bad, kernels = 0, set()
    for i in range(120):
        kind = i % 3
        batch = int(rng.choice([1, 1, 1, 2, 3]))
        trans = bool(rng.integers(0, 2))
        if kind < 2:
            m = int(rng.choice([1, 4, 16, 63, 128, 130, 256, 300]))
            n = 16 * int(rng.integers(1, 33))
            k = 64 * int(rng.integers(1, 17)) if kind == 0 else 16 * int(rng.integers(1, 40)) // 64 * 64 + 16 * int(rng.integers(1, 4))
            offs = {}
        else:
            m, n, k = (int(rng.integers(1, 300)) for _ in range(3))
            offs = dict(off_a=int(rng.integers(0, 20)), off_b=int(rng.integers(0, 20)), off_c=int(rng.integers(0, 9)),
                        lda_extra=int(rng.integers(0, 9)), ldb_extra=int(rng.integers(0, 9)))
        share = batch > 1 and bool(rng.integers(0, 2))
        c = cases.Case(f"random {i}: {m}x{n}x{k} b{batch}{' shared B' if share else ''}{' T' if trans else ''}",
                       cases.problem(m, n, k, batch=batch, trans_b=trans, share_b=share, **offs),
                       bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), int(rng.integers(0, 3)), int(rng.integers(0, 3)))
        say(f"[{config}] {c.name} signed {c.a_signed}/{c.b_signed} zp {c.za_mode}/{c.zb_mode} {offs}")
        here, kern = run_int32(d, gemm, c, 5000 + i)
        kernels.add(kern)
        assert here == 0, f"{c.name} [{config}, {kern}]: {here} wrong"
        bad += here
    say(f"ROW seeded random products [{config}]: 120 cases, mismatches {bad}; kernels {sorted(kernels)}")


@pytest.mark.parametrize("config", ["default", "large tile"])
def test_seeded_random_epilogues_are_bit_exact(config):
    # The float (scale per tensor or column, int and float biases) and requantized (multiplier per tensor or column,
    # either output type, zero point, bias) epilogues on seeded random shapes, aligned (the direct and few-rows kernels)
    # and not; the requantized ones both fused into the product's store and as the separate pass.
    d = device()
    rng = np.random.default_rng({"default": 21, "large tile": 22}[config])
    fused = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config], FusedRequantize=True))
    passes = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config], FusedRequantize=False))
    bad, kernels = 0, set()
    for i in range(24):
        if i % 2 == 0:
            m, n, k = int(rng.choice([1, 3, 16, 100, 128, 257])), 16 * int(rng.integers(1, 40)), 64 * int(rng.integers(1, 12))
        else:
            m, n, k = (int(rng.integers(1, 260)) for _ in range(3))
        vec, ib, fb = (bool(rng.integers(0, 2)) for _ in range(3))
        say(f"[{config}] epilogues {m}x{n}x{k} vec {vec} ib {ib} fb {fb}")
        bad += _float_case(d, fused, m, n, k, vec, ib, fb, 6000 + i)
        kernels.add(d.LastKernel)
        unsigned, zero = cases.REQUANT_OUT[i % len(cases.REQUANT_OUT)]
        for gemm in (fused, passes):
            bad += _requant_case(d, gemm, m, n, k, vec, unsigned, zero, ib, 6100 + i, bool(rng.integers(0, 2)),
                                 bool(rng.integers(0, 2)))
            kernels.add(d.LastKernel)
        assert bad == 0, f"{m}x{n}x{k}: {bad} wrong"
    say(f"ROW seeded random epilogues [{config}]: 24 shapes exact; kernels {sorted(kernels)}")


# K either side of 32768, where the direct kernels' zero-point corrections leave the full-rate 24-bit multiply for the
# 32-bit one. A column sum less K times B's zero point, in the signed domain, reaches 255 K: past 2^23 from K = 32897
# on, so a 24-bit multiply at K = 40960 would be wrong. The other kernels, whose corrections are 32-bit throughout,
# run the same sizes. (name, m, n, k, a signed, b signed, zp modes of A and B, configuration, kernel prefix.)
LARGE_K_CASES = [
    ("256 tile, both zero points", 256, 256, 40960, False, False, 2, 2, "large tile", "mfma-i8-direct256x256x64"),
    ("256 tile, both zero points, below the switch", 256, 256, 32704, False, False, 1, 2, "large tile",
     "mfma-i8-direct256x256x64"),
    ("256 tile ping-pong, A's zero point per row", 256, 256, 40960, False, True, 2, 0, "large tile",
     "mfma-i8-direct256x256x64"),
    ("128 tile split along K", 128, 128, 40960, False, False, 1, 2, "default", "mfma-i8-direct128x128x64"),
    ("128 tile whole, C misaligned for the staged store", 1152, 1920, 40960, False, False, 2, 2, "default",
     "mfma-i8-direct128x128x64"),
    ("register-staged tile, K not a multiple of 64", 64, 64, 40976, False, False, 2, 1, "tiled only",
     "mfma-i8-tile128x128x128"),
    ("generic kernel, unaligned rows", 64, 64, 40961, False, False, 1, 2, "tiled only", "mfma-i8-generic128x128x64"),
    ("few rows, one launch", 4, 2048, 40960, False, False, 1, 2, "default", "mfma-i8-rows16-xcd"),
    # 127 k-slices a column slab, the most its 7-bit count fields take; 128 go to the two-launch kernel.
    ("few rows, one launch, 127 k-slices", 3, 2048, 127 * 512, False, True, 2, 0, "default", "mfma-i8-rows16-xcd"),
    ("few rows, 128 k-slices", 3, 2048, 128 * 512, False, True, 2, 0, "default", "mfma-i8-rows16-tiles"),
]


def _large_k_data(c, adversarial: bool, seed: int) -> dict:
    """Random bytes, or the fill that makes every correction term extreme: A = 0 under a zero point of 255 (u8),
    B = 255 under a zero point of 0 (u8; int8 B without a zero point takes -128)."""
    data = cases.case_data(c, seed)
    if adversarial:
        data["a"][:] = 0x00
        data["b"][:] = 0xFF if not c.b_signed else 0x80
        if data["za"] is not None:
            data["za"][:] = 0xFF
        if data["zb"] is not None:
            data["zb"][:] = 0x00
    return data


@pytest.mark.parametrize("case", LARGE_K_CASES, ids=[c[0] for c in LARGE_K_CASES])
def test_large_k_corrections_are_bit_exact(case):
    name, m, n, k, a_s, b_s, za_mode, zb_mode, config, prefix = case
    d = device()
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config]))
    off_c = 1 if "misaligned" in name else 0
    c = cases.Case(name, cases.problem(m, n, k, off_c=off_c), a_s, b_s, za_mode, zb_mode)
    for adversarial in (False, True):
        say(f"large K [{config}] {name} {m}x{n}x{k} adversarial {adversarial}")
        data = _large_k_data(c, adversarial, 900 + k % 97 + m)
        want = cases.reference_sums(c, data)
        if adversarial:
            # Every product term is (0 - 255)(255 - 0), or (0 - 255)(-128) for int8 B: K of them, modulo 2^32.
            term = -255 * (-128 if b_s else 255)
            closed = np.int64(term) * np.int64(k)
            assert np.all(want == np.int32(np.uint32(closed & 0xFFFFFFFF).view(np.int32)))
        out = np.full(off_c + m * n + 2, 0x5A5A5A5A, np.int32)
        bc = d.CreateBuffer(out)
        ba = d.CreateBuffer(as_u8(data["a"]))
        bb = d.CreateBuffer(as_i8(data["b"]) if b_s else as_u8(data["b"]))
        za = og.Int8Operand(d.CreateBuffer(as_u8(data["za"])), 0, za_mode == 2) if data["za"] is not None else None
        zb = og.Int8Operand(d.CreateBuffer(as_u8(data["zb"])), 0, zb_mode == 2) if data["zb"] is not None else None
        run(d, lambda e: gemm.EncodeInt32(e, to_problem(c.p), ba, bb, bc, za, zb))
        d.WaitIdle()   # reports a one-launch product whose parts never arrived
        got = bc.Read()
        kernel = d.LastKernel
        bad = int(np.count_nonzero(got[off_c:off_c + m * n] != want))
        bad += int(np.count_nonzero(got[:off_c] != 0x5A5A5A5A)) + int(np.count_nonzero(got[off_c + m * n:] != 0x5A5A5A5A))
        say(f"ROW large K | {name} | {kernel} | adversarial {adversarial} | mismatches {bad}")
        assert kernel.startswith(prefix), kernel
        assert bad == 0


@pytest.mark.parametrize("config", ["default", "portable", "large tile"])
def test_empty_products_launch_nothing(config):
    # M = 0 or N = 0 (K any): every product form records nothing that runs and leaves its output alone (the
    # reference's Prepare returns Ok = false for these and records nothing); a ranged product counts no pairs from its
    # place in the submission on, also after a full ranged product into the same ranges.
    d = device()
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config]))
    fused = og.Int8Gemm(d, og.Int8GemmOptions(**CONFIG_OPTIONS[config], FusedRequantize=True))
    ranges = og.Int8Ranges(d.CreateBufferOf(og.ElementType.Float32, 2 * og.OG_RANGES_MAX))
    a = d.CreateBuffer(np.full(64 * 4096, 7, np.uint8))
    b = d.CreateBuffer(np.full(4096 * 64, 3, np.int8))
    scale = d.CreateBuffer(np.full(64, 0.5, np.float32))
    zb = d.CreateBuffer(np.zeros(64, np.int8))
    f64 = d.CreateBufferOf(og.ElementType.Float32, 64 * 64)
    for m, n, k in ((0, 64, 64), (64, 0, 64), (0, 0, 0), (0, 64, 4096), (3, 0, 4096)):
        say(f"empty [{config}] {m}x{n}x{k}")
        run(d, lambda e: gemm.EncodeFloatRanged(e, og.Int8GemmProblem(64, 64, 64), a, b, f64, og.Int8Operand(scale, 0, True),
                                                ranges))
        assert ranges.Groups >= 1
        c = d.CreateBuffer(np.full(16, 0x5A5A5A5A, np.int32))
        f = d.CreateBuffer(np.full(16, -77.0, np.float32))
        y = d.CreateBuffer(np.full(16, 0xA7, np.uint8))
        p = og.Int8GemmProblem(m, n, k)
        e = d.BeginCommands()
        e.BeginPassTiming(8)
        gemm.EncodeInt32(e, p, a, b, c, None, og.Int8Operand(zb, 0, True))
        gemm.EncodeFloat(e, p, a, b, f, og.Int8Operand(scale, 0, True))
        gemm.EncodeFloatRanged(e, p, a, b, f, og.Int8Operand(scale, 0, True), ranges)
        for g in (gemm, fused):
            g.EncodeRequantized(e, p, a, b, y, og.Int8Operand(scale, 0, True), 3)
        e.EndPassTiming()
        d.Submit(e)
        d.WaitIdle()
        assert d.ReadPassTimes() == [], "an empty product launched a kernel"
        assert ranges.Groups == 0, "an empty ranged product after a full one leaves no pairs counted"
        # In the other order, in one submission, the full product's pairs are the ones counted.
        e = d.BeginCommands()
        gemm.EncodeFloatRanged(e, p, a, b, f, og.Int8Operand(scale, 0, True), ranges)
        gemm.EncodeFloatRanged(e, og.Int8GemmProblem(64, 64, 64), a, b, f64, og.Int8Operand(scale, 0, True), ranges)
        d.Submit(e)
        d.WaitIdle()
        assert ranges.Groups >= 1
        assert c.Read().tolist() == [0x5A5A5A5A] * 16 and f.Read().tolist() == [-77.0] * 16
        assert y.Read().tolist() == [0xA7] * 16


def test_stream_tiles_reads_b_and_writes_nothing():
    # og_util_stream_tiles, the streaming floor the few-rows product is measured against: it runs as "stream-tiles"
    # over configuration 3's B and over a ragged shape, and leaves the sink alone (an all-zero B has checksum 0).
    d = device()
    L = abi()
    L.og_util_stream_tiles.argtypes = [ctypes.c_void_p, L.Buf, ctypes.c_uint32, ctypes.c_uint32, L.Buf]
    for k, n in ((4096, 11008), (1000, 144)):
        say(f"stream-tiles {k} x {n}")
        b = d.CreateBuffer(np.zeros(k * n, np.uint8))
        sink = d.CreateBuffer(np.full(4, 0x5A, np.uint8))
        check(L.og_util_stream_tiles(d.Context, binding(b), k, n, binding(sink)), d)
        d.WaitIdle()
        assert d.LastKernel == "stream-tiles"
        assert np.array_equal(sink.Read()[:4], np.full(4, 0x5A, np.uint8))
