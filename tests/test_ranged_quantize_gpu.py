"""Quantizing a layer's float output without DynamicQuantizeLinear's read pass (no counterpart in the reference: there,
quantizing a MatMulIntegerToFloat output starts with the DqMinMax dispatch, DynamicQuantize.hlsl:35-69, that reads the
whole tensor; the chain is Int8Tests.cs:705-751's).

Int8Gemm.EncodeFloatRanged (og_int8_gemm_float_ranged) writes the float product and, from its kernels' epilogue, the
(min, max) of what each workgroup stored; DynamicQuantizeKernels.EncodeRanged (og_dynamic_quantize_ranged) is then the
quantize pass alone. Checked against the oracle, bit for bit, on every kernel family a ranged product can take (the
ones with a range epilogue and the ones followed by a range pass): the float output, the recorded range (its combined
minimum and maximum are the output's NaN-ignoring ones), DynamicQuantizeLinear's y, scale and zero point, and the
following layer's product on the quantized bytes."""
from __future__ import annotations

import numpy as np
import pytest

import cases
import oracle
import onegpu_hip as og
from gpu_rig import CONFIG_OPTIONS, as_i8, as_u8, device, run, say

pytestmark = pytest.mark.gpu

# (label, m, n, k, batch, options, the kernel the product takes, whether that kernel writes the ranges itself)
CASES = [
    ("direct 128", 256, 384, 512, 1, {}, "mfma-i8-direct128x128x64", True),
    ("direct 128, batch 3", 128, 256, 320, 3, {}, "mfma-i8-direct128x128x64", True),
    ("configuration 2, layer 1", 1024, 3072, 768, 1, {}, "mfma-i8-direct128x128x64", True),
    ("direct 128, ragged", 200, 144, 192, 1, {}, "mfma-i8-direct128x128x64", True),
    ("split k", 256, 256, 2304, 1, {}, "mfma-i8-direct128x128x64-splitk", True),
    ("split k, ragged", 200, 144, 1536, 1, {}, "mfma-i8-direct128x128x64-splitk", True),
    ("few rows, one launch", 4, 2048, 4096, 1, {}, "mfma-i8-rows16-xcd", True),
    ("few rows, one launch, 16 rows", 16, 4608, 1024, 1, {}, "mfma-i8-rows16-xcd", True),
    ("256 tile (range pass)", 512, 512, 256, 1, {"Tile": 256}, "mfma-i8-direct256x256x64", False),
    ("register-staged tile (range pass)", 64, 64, 96, 1, {}, "mfma-i8-tile128x128x128", False),
    ("few rows, two launches (range pass)", 3, 2048, 512, 1, {"FewRowsOneLaunch": False}, "mfma-i8-rows16-tiles", False),
    ("portable (range pass)", 70, 90, 100, 1, {"AllowPackedDot": False}, "portable-tile64x64x16", False),
]


def _layer(d, gemm, m, n, k, batch, seed, act_scale, fbias=False, ibias=False, nan_scale=False):
    """One ranged float product: u8 A with a scalar zero point, int8 B [k x n] per batch with per-column scales; the
    column scale fl(act * wscale[n]) in the epilogue (EncodeFloatScaled's form). Returns (device buffers, expected C)."""
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, batch * m * k, dtype=np.uint8)
    za = np.array([rng.integers(90, 160)] * 4, np.uint8)
    b = rng.integers(-127, 128, batch * k * n, dtype=np.int8)
    wscale = (rng.random(n, dtype=np.float32) * np.float32(0.02) + np.float32(1e-3)).astype(np.float32)
    if nan_scale:
        wscale[n // 3] = np.float32("nan")
        wscale[n // 2] = np.float32(3e38)   # products past the float range: +-inf
    fb = (rng.standard_normal(n) * 5).astype(np.float32)
    ib = rng.integers(-1000, 1000, n, dtype=np.int32)
    p = cases.problem(m, n, k, batch=batch)
    sums = oracle.int8_gemm(p, a, False, b.view(np.uint8), True, (za[:1], False, 0))
    with np.errstate(all="ignore"):
        colscale = (np.float32(act_scale) * wscale).astype(np.float32)
        want = oracle.float_epilogue(sums, n, colscale, True, ib if ibias else None, fb if fbias else None)
    bufs = dict(a=d.CreateBuffer(as_u8(a)), b=d.CreateBuffer(as_i8(b)), za=d.CreateBuffer(za),
                ws=d.CreateBuffer(wscale), act=d.CreateBuffer(np.array([act_scale], np.float32)),
                fb=d.CreateBuffer(fb), ib=d.CreateBuffer(ib), c=d.CreateBufferOf(og.ElementType.Float32, batch * m * n))
    return bufs, want, p


def _same_bits(got, want):
    same = np.where(np.isnan(want), np.isnan(got), got.view(np.uint32) == want.view(np.uint32))
    return int(np.count_nonzero(~same))


@pytest.mark.parametrize("label, m, n, k, batch, opts, want_kernel, from_epilogue", CASES, ids=[c[0] for c in CASES])
def test_ranged_product_then_quantize_without_a_read_pass(label, m, n, k, batch, opts, want_kernel, from_epilogue):
    d = device()
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(**opts))
    dq = og.DynamicQuantizeKernels(d)
    ranges = og.Int8Ranges(d.CreateBufferOf(og.ElementType.Float32, 2 * og.OG_RANGES_MAX))
    seed = sum(map(ord, label))
    special = label.startswith("direct 128,") or label.startswith("split k,") or "portable" in label
    for variant in ("plain", "biases", "special") if special else ("plain", "biases"):
        say(f"ranged [{label}] {batch} x {m}x{n}x{k} {variant}")
        bufs, want, p = _layer(d, gemm, m, n, k, batch, seed, 0.0123, fbias=variant != "plain",
                               ibias=variant != "plain", nan_scale=variant == "special")
        run(d, lambda e: gemm.EncodeFloatRanged(e, og.Int8GemmProblem(m, n, k) if batch == 1 else _problem(m, n, k, batch),
                                                bufs["a"], bufs["b"], bufs["c"], og.Int8Operand(bufs["ws"], 0, True), ranges,
                                                og.Int8Operand(bufs["za"], 0), None,
                                                og.Int8Operand(bufs["fb"], 0, True) if variant != "plain" else None,
                                                og.Int8Operand(bufs["ib"], 0, True) if variant != "plain" else None,
                                                og.Int8Operand(bufs["act"], 0)))
        d.WaitIdle()
        assert d.LastKernel == want_kernel, d.LastKernel
        c = bufs["c"].Read()
        assert _same_bits(c, want) == 0, "the ranged product's output equals the plain product's"
        groups = ranges.Groups
        assert 1 <= groups <= og.OG_RANGES_MAX
        r = ranges.Buffer.Read()[:2 * groups].reshape(groups, 2)
        finite = c[~np.isnan(c)]
        assert r[:, 0].min() == finite.min() and r[:, 1].max() == finite.max(), "the pairs cover C's range"
        if from_epilogue and variant == "plain":
            say(f"  {groups} ranges from the {want_kernel} epilogue")

        # DynamicQuantizeLinear of C from the recorded ranges: the quantize pass alone.
        y = d.CreateBufferOf(og.ElementType.UInt8, c.size)
        s = d.CreateBufferOf(og.ElementType.Float32, 1)
        z = d.CreateBufferOf(og.ElementType.UInt8, 4)
        run(d, lambda e: dq.EncodeRanged(e, bufs["c"], 0, c.size, y, 0, s, 0, z, 0, ranges))
        d.WaitIdle()
        assert d.LastKernel == "dq-quantize"
        wy, ws_, wz = oracle.dynamic_quantize(c)
        got_y, got_s, got_z = y.Read()[:c.size], np.float32(s.Read()[0]), int(z.Read()[0])
        bad = int(np.count_nonzero(got_y != wy))
        say(f"ROW ranged DQ [{label}] {variant}: groups {groups}, wrong bytes {bad}, scale {got_s} / {ws_}, zp {got_z} / {wz}")
        assert bad == 0 and got_s.view(np.uint32) == np.float32(ws_).view(np.uint32) and got_z == wz

        if variant == "plain":
            # The next layer on the quantized bytes: y [batch*m x n] (zero point z) times int8 W2 [n x 64], its column
            # scale fl(scale * w2scale[j]).
            rng = np.random.default_rng(seed + 1)
            n2 = 64
            w2 = rng.integers(-127, 128, n * n2, dtype=np.int8)
            w2s = (rng.random(n2, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
            bw2, bw2s = d.CreateBuffer(as_i8(w2)), d.CreateBuffer(w2s)
            c2 = d.CreateBufferOf(og.ElementType.Float32, batch * m * n2)
            p2 = og.Int8GemmProblem(batch * m, n2, n)
            run(d, lambda e: og.Int8Gemm(d).EncodeFloatScaled(e, p2, y, bw2, c2, og.Int8Operand(s, 0),
                                                              og.Int8Operand(bw2s, 0, True), og.Int8Operand(z, 0)))
            sums2 = oracle.int8_gemm(cases.problem(batch * m, n2, n), wy, False, w2.view(np.uint8), True,
                                     (np.array([wz], np.uint8), False, 0))
            want2 = oracle.float_epilogue(sums2, n2, (np.float32(ws_) * w2s).astype(np.float32), True)
            bad2 = _same_bits(c2.Read(), want2)
            say(f"  next layer ({d.LastKernel}): {bad2} wrong values")
            assert bad2 == 0


def _problem(m, n, k, batch):
    p = og.Int8GemmProblem(m, n, k)
    p.Batch, p.StrideA, p.StrideB = batch, m * k, k * n
    return p


def test_ranged_pass_reports_a_missing_range():
    # EncodeRanged before any ranged product filled the ranges: the pass refuses (argument "groups"), it does not
    # quantize with a made-up range.
    d = device()
    ranges = og.Int8Ranges(d.CreateBufferOf(og.ElementType.Float32, 2 * og.OG_RANGES_MAX))
    x = d.CreateBuffer(np.ones(64, np.float32))
    y, s, z = (d.CreateBufferOf(og.ElementType.UInt8, 64), d.CreateBufferOf(og.ElementType.Float32, 1),
               d.CreateBufferOf(og.ElementType.UInt8, 4))
    with pytest.raises(og.GpuKernelShapeException) as ex:
        run(d, lambda e: og.DynamicQuantizeKernels(d).EncodeRanged(e, x, 0, 64, y, 0, s, 0, z, 0, ranges))
    assert ex.value.Argument == "groups"
    d.WaitIdle()


def test_ranged_seeded_random_shapes():
    # 24 seeded random shapes (aligned ones that take the range epilogues and ragged ones that take a range pass),
    # batch 1 or 2, with and without biases: the float output, the recorded ranges and the quantize pass alone against
    # the oracle's DynamicQuantizeLinear of that output, bit for bit.
    d = device()
    gemm = og.Int8Gemm(d)
    dq = og.DynamicQuantizeKernels(d)
    ranges = og.Int8Ranges(d.CreateBufferOf(og.ElementType.Float32, 2 * og.OG_RANGES_MAX))
    rng = np.random.default_rng(2024)
    kernels = set()
    for i in range(24):
        if i % 2 == 0:
            m, n, k = int(rng.choice([1, 4, 16, 100, 256, 333])), 16 * int(rng.integers(1, 48)), 64 * int(rng.integers(1, 20))
        else:
            m, n, k = (int(rng.integers(1, 300)) for _ in range(3))
        batch = int(rng.integers(1, 3))
        biases = bool(rng.integers(0, 2))
        say(f"ranged random {i}: {batch} x {m}x{n}x{k} biases {biases}")
        bufs, want, _ = _layer(d, gemm, m, n, k, batch, 7000 + i, float(rng.random() * 0.05 + 1e-3), fbias=biases,
                               ibias=biases)
        run(d, lambda e: gemm.EncodeFloatRanged(e, og.Int8GemmProblem(m, n, k) if batch == 1 else _problem(m, n, k, batch),
                                                bufs["a"], bufs["b"], bufs["c"], og.Int8Operand(bufs["ws"], 0, True), ranges,
                                                og.Int8Operand(bufs["za"], 0), None,
                                                og.Int8Operand(bufs["fb"], 0, True) if biases else None,
                                                og.Int8Operand(bufs["ib"], 0, True) if biases else None,
                                                og.Int8Operand(bufs["act"], 0)))
        d.WaitIdle()
        kernels.add(d.LastKernel)
        c = bufs["c"].Read()
        assert _same_bits(c, want) == 0, f"case {i}: the float output"
        groups = ranges.Groups
        assert 1 <= groups <= og.OG_RANGES_MAX
        r = ranges.Buffer.Read()[:2 * groups].reshape(groups, 2)
        finite = c[~np.isnan(c)]
        assert r[:, 0].min() == finite.min() and r[:, 1].max() == finite.max(), f"case {i}: the ranges"
        y = d.CreateBufferOf(og.ElementType.UInt8, c.size)
        s = d.CreateBufferOf(og.ElementType.Float32, 1)
        z = d.CreateBufferOf(og.ElementType.UInt8, 4)
        run(d, lambda e: dq.EncodeRanged(e, bufs["c"], 0, c.size, y, 0, s, 0, z, 0, ranges))
        d.WaitIdle()
        wy, ws_, wz = oracle.dynamic_quantize(c)
        got_y, got_s, got_z = y.Read()[:c.size], np.float32(s.Read()[0]), int(z.Read()[0])
        assert np.array_equal(got_y, wy) and got_s.view(np.uint32) == np.float32(ws_).view(np.uint32) and got_z == wz, \
            f"case {i}: DynamicQuantizeLinear from the ranges"
    say(f"ROW ranged seeded random: 24 shapes exact; kernels {sorted(kernels)}")
