"""ConvIntegerKernels on the GPU against the oracle's restatement of ConvIntegerTests.Reference, bit for bit
(ConvIntegerTests.cs): the edge geometries (pointwise, padding, strides, dilation, groups, depthwise, 1-D, offsets,
extremes, caller scratch that makes the batch run in chunks), the Whisper stem and the ResNet / MobileNet shapes, each
on the MFMA products and on the portable one, depthwise both directly and through the column matrix."""
from __future__ import annotations

import numpy as np
import pytest

import cases
import oracle
import onegpu_hip as og
from gpu_rig import device, run, say

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A5A5A5A


def _problem(p: dict) -> og.ConvProblem:
    q = og.ConvProblem()
    for key, v in p.items():
        setattr(q, key, v)
    return q


def _bytes_of(a: np.ndarray, signed: bool) -> np.ndarray:
    """The bytes as the operand's type, padded to a whole word (ConvIntegerTests.Cast)."""
    pad = np.zeros((a.size + 3) & ~3, np.uint8)
    pad[:a.size] = a
    return pad.view(np.int8) if signed else pad


def _run_case(d, conv, c: dict, seed: int) -> tuple[int, str]:
    """ConvIntegerTests.Run (ConvIntegerTests.cs:91-174): wrong elements (inside and around y) and the kernel."""
    p = c["p"]
    q = _problem(p)
    oh, ow = q.OutHeight, q.OutWidth
    cin_g = p["InChannels"] // p["Groups"]
    off_x, off_w, off_y = p.get("OffsetX", 0), p.get("OffsetW", 0), p.get("OffsetY", 0)
    x_len = off_x + p["Batch"] * p["InChannels"] * p["Height"] * p["Width"] + 4
    w_len = off_w + p["OutChannels"] * cin_g * p["KernelHeight"] * p["KernelWidth"] + 4
    x, w = cases.conv_bytes(x_len, seed), cases.conv_bytes(w_len, seed + 1)
    xz = None if c["xzm"] == 0 else cases.conv_bytes(1, seed + 2)
    wz = None if c["wzm"] == 0 else cases.conv_bytes(p["OutChannels"] if c["wzm"] == 2 else 1, seed + 3)
    if c["fill"] >= 0:
        x[:] = c["fill"]
        w[:] = c["fill"] ^ 0xFF
        if xz is not None:
            xz[:] = c["fill"]
        if wz is not None:
            wz[:] = c["fill"] ^ 0x80
    want = oracle.conv_integer(p, x[off_x:], c["xs"], w[off_w:], c["ws"], xz, wz, c["wzm"] == 2, threads=16)
    got0 = np.full(off_y + want.size + 2, SENTINEL, np.int32)
    bx, bw = d.CreateBuffer(_bytes_of(x, c["xs"])), d.CreateBuffer(_bytes_of(w, c["ws"]))
    bxz = None if xz is None else d.CreateBuffer(_bytes_of(xz, c["xs"]))
    bwz = None if wz is None else d.CreateBuffer(_bytes_of(wz, c["ws"]))
    by = d.CreateBuffer(got0)
    scratch, scratch_off = None, 0
    if c["scratch_images"] > 0:
        scratch_off = 8
        n = scratch_off + c["scratch_images"] * og.ConvIntegerKernels.ScratchBytesPerImage(q)
        scratch = d.CreateBufferOf(og.ElementType.Int8 if c["xs"] else og.ElementType.UInt8, n)
    run(d, lambda e: conv.Encode(e, q, bx, bw, by, None if bxz is None else og.Int8Operand(bxz, 0),
                                 None if bwz is None else og.Int8Operand(bwz, 0, c["wzm"] == 2), scratch, scratch_off))
    got = by.Read()
    bad = int(np.count_nonzero(got[off_y:off_y + want.size] != want))
    bad += int(np.count_nonzero(got[:off_y] != SENTINEL)) + int(np.count_nonzero(got[off_y + want.size:] != SENTINEL))
    return bad, d.LastKernel


def _configs(d):
    """ConvIntegerTests.Check's two families (ConvIntegerTests.cs:197-221), plus depthwise through the column matrix."""
    out = [("mfma", og.ConvIntegerKernels(d)), ("portable", og.ConvIntegerKernels(d, og.Int8GemmOptions(AllowPackedDot=False)))]
    k = og.ConvIntegerKernels(d)
    k.DirectDepthwise = False
    out.append(("mfma, depthwise as products", k))
    return out


def test_onnx_specification_examples():
    # The ONNX ConvInteger specification's two examples, as known answers: x = 2..10 (3 x 3, uint8, zero point 1),
    # w = 2 x 2 ones; without padding [12, 16, 24, 28], with padding 1 the 4 x 4 result below. Run on the column
    # matrix path and on the portable product.
    d = device()
    x = d.CreateBuffer(_bytes_of(np.array([2, 3, 4, 5, 6, 7, 8, 9, 10], np.uint8), False))
    w = d.CreateBuffer(_bytes_of(np.ones(4, np.uint8), False))
    xz = d.CreateBuffer(_bytes_of(np.array([1], np.uint8), False))
    want = {0: [12, 16, 24, 28], 1: [1, 3, 5, 3, 5, 12, 16, 9, 11, 24, 28, 15, 7, 15, 17, 9]}
    for name, conv in _configs(d)[:2]:
        for pad, expected in want.items():
            q = _problem(cases.conv_problem(1, 1, 3, 3, 1, 2, 2, pad=pad))
            y = d.CreateBufferOf(og.ElementType.Int32, len(expected))
            run(d, lambda e: conv.Encode(e, q, x, w, y, og.Int8Operand(xz, 0)))
            assert y.Read().tolist() == expected, (name, pad)


def test_edge_geometries_are_bit_exact():
    # EdgeGeometriesAreBitExact (ConvIntegerTests.cs:235-275).
    d = device()
    bad_total, seed, kernels = 0, 100, set()
    for name, conv in _configs(d):
        for c in cases.conv_edge_cases():
            if name.startswith("mfma, depthwise") and c["p"]["InChannels"] != c["p"]["Groups"]:
                continue
            say(f"conv [{name}] {c['name']}")
            bad, kern = _run_case(d, conv, c, seed)
            kernels.add(kern)
            assert bad == 0, f"{c['name']} [{name}]: {bad} elements differ ({kern})"
            bad_total += bad
            seed += 1
    say(f"ROW conv integer edge geometries: 0 mismatches; kernels {sorted(kernels)}")
    assert "conv-depthwise-i8" in kernels and "portable-tile64x64x16" in kernels


@pytest.mark.parametrize("index", range(len(cases.conv_model_cases())))
def test_model_shapes_are_bit_exact(index):
    # WhisperStemIsBitExact and ResNetShapesAreBitExact (ConvIntegerTests.cs:277-307).
    d = device()
    c = cases.conv_model_cases()[index]
    for name, conv in _configs(d)[:2]:
        say(f"conv [{name}] {c['name']}")
        bad, kern = _run_case(d, conv, c, 500 + index)
        say(f"ROW conv integer {c['name']} [{name}, {kern}]: {bad} elements differ")
        assert bad == 0


def test_padded_depth_with_groups_and_chunks():
    # K = CinG * KH * KW not a multiple of 64 (and at least 64) is padded to one: the column matrices get rows of x's
    # zero point and the weights are copied into padded rows by the pack launch of the first chunk of images. Groups,
    # caller scratch that holds 1 or 2 images (a batch of 3 runs in chunks, the later chunks reusing the weight copy)
    # at an offset that leaves the copy to align its own start, and every zero-point form.
    d = device()
    conv = og.ConvIntegerKernels(d)
    base = cases.conv_problem(3, 80, 9, 11, 48, 3, 3, stride=1, pad=1, groups=2)   # K = 40 * 9 = 360 -> 384
    seed = 900
    for scratch_images, xs, ws, xzm, wzm in ((1, False, True, 1, 2), (2, True, False, 1, 1), (0, False, False, 0, 2),
                                             (2, True, True, 1, 0)):
        c = dict(name=f"padded depth, groups 2, scratch {scratch_images}", p=base, xs=xs, ws=ws, xzm=xzm, wzm=wzm,
                 fill=-1, scratch_images=scratch_images)
        say(f"conv {c['name']} signed {xs}/{ws} zp {xzm}/{wzm}")
        bad, kern = _run_case(d, conv, c, seed)
        seed += 1
        assert bad == 0, f"{c['name']}: {bad} elements differ ({kern})"
        assert kern.startswith("mfma-i8-direct"), kern


def test_warm_calls_allocate_nothing_new():
    # WarmCallsBuildNoBindGroups (ConvIntegerTests.cs:331-347): the second identical call reuses the family's columns.
    d = device()
    conv = og.ConvIntegerKernels(d)
    q = _problem(cases.conv_problem(1, 3, 10, 10, 4, 3, 3, pad=1))
    x, w, y = d.CreateBuffer(np.zeros(304, np.uint8)), d.CreateBuffer(np.zeros(112, np.int8)), d.CreateBufferOf(og.ElementType.Int32, 400)
    run(d, lambda e: conv.Encode(e, q, x, w, y))
    created = conv.BindGroupsCreated
    run(d, lambda e: conv.Encode(e, q, x, w, y))
    assert conv.BindGroupsCreated == created
    assert np.count_nonzero(y.Read()) == 0


@pytest.mark.parametrize("m, n", [(3, 4_300_001), (4_300_001, 3), (2, 4_194_241)])
def test_products_wider_than_one_grid_axis_are_bit_exact(m, n):
    # ProductsWiderThanOneGridAxisAreBitExact (ConvIntegerTests.cs:349-390): products whose tile grid would not fit one
    # 65535-wide dispatch axis, wide and tall, on the chosen, portable and split-k kernels.
    d = device()
    k = 5
    a, b = cases.conv_bytes(m * k, 11), cases.conv_bytes(k * n, 12)
    za, zb = cases.conv_bytes(1, 13), cases.conv_bytes(n, 14)
    want = oracle.int8_gemm(oracle.Gemm(m, n, k), a, False, b, True, (za, False, 0), (zb, True, 0))
    for opts in (og.Int8GemmOptions(), og.Int8GemmOptions(AllowPackedDot=False), og.Int8GemmOptions(Tile=32)):
        gemm = og.Int8Gemm(d, opts)
        ba, bb = d.CreateBuffer(_bytes_of(a, False)), d.CreateBuffer(_bytes_of(b, True))
        bza, bzb = d.CreateBuffer(_bytes_of(za, False)), d.CreateBuffer(_bytes_of(zb, True))
        bc = d.CreateBufferOf(og.ElementType.Int32, m * n)
        run(d, lambda e: gemm.EncodeInt32(e, og.Int8GemmProblem(m, n, k), ba, bb, bc, og.Int8Operand(bza, 0),
                                          og.Int8Operand(bzb, 0, True)))
        bad = int(np.count_nonzero(bc.Read() != want))
        say(f"ROW wide product {m} x {n} x {k} [{d.LastKernel}]: {bad} elements differ")
        assert bad == 0


def test_seeded_random_convolutions_are_bit_exact():
    # A seeded sweep of geometries beyond the reference's lists: batches, channel and group counts (depthwise among
    # them), windows, strides, dilations and paddings chosen per axis, every signedness and zero-point form; depths of
    # 64 and more that are not multiples of 64 take the padded pack. Each against the oracle, output sentinels included.
    d = device()
    conv = og.ConvIntegerKernels(d)
    rng = np.random.default_rng(77)
    kernels = set()
    for i in range(30):
        groups = int(rng.choice([1, 1, 2, 3, 4]))
        cin_g, cout_g = int(rng.integers(1, 24)), int(rng.integers(1, 20))
        if i % 5 == 4:
            cin_g = 1   # depthwise-shaped groups
            groups = int(rng.integers(2, 9))
        kh, kw = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        sh, sw, dh, dw = (int(rng.integers(1, 4)) for _ in range(4))
        pt, pb, pl, pr = (int(rng.integers(0, 3)) for _ in range(4))
        h = int(rng.integers(max(1, dh * (kh - 1) + 1 - pt - pb), 24))
        w = int(rng.integers(max(1, dw * (kw - 1) + 1 - pl - pr), 24))
        p = cases.conv_problem(int(rng.integers(1, 4)), cin_g * groups, h, w, cout_g * groups, kh, kw, groups=groups)
        p.update(StrideHeight=sh, StrideWidth=sw, DilationHeight=dh, DilationWidth=dw, PadTop=pt, PadBottom=pb,
                 PadLeft=pl, PadRight=pr)
        s = int(rng.integers(0, 4))
        c = dict(name=f"random {i}: {p['Batch']}x{p['InChannels']}x{h}x{w} -> {p['OutChannels']}, {kh}x{kw} s{sh},{sw} "
                      f"d{dh},{dw} groups {groups}", p=p, xs=(s & 1) != 0, ws=(s & 2) != 0, xzm=int(rng.integers(0, 2)),
                 wzm=int(rng.integers(0, 3)), fill=-1, scratch_images=int(rng.integers(0, 3)))
        say(f"conv {c['name']} signed {c['xs']}/{c['ws']} zp {c['xzm']}/{c['wzm']} scratch {c['scratch_images']}")
        bad, kern = _run_case(d, conv, c, 3000 + i)
        kernels.add(kern)
        assert bad == 0, f"{c['name']}: {bad} elements differ ({kern})"
    say(f"ROW seeded random convolutions: 30 geometries exact; kernels {sorted(kernels)}")
