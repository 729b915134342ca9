"""Writes the committed fixtures of the int8 path (run from the repository root: python tests/golden/make_golden.py).

The reference holds no golden vectors for this path (its tests compute CPU references on the fly), so these are the
build's own: inputs and outputs of

  c1_smoke.npz     MatMulInteger smoke (the reference's CPU-runnable configuration): A uint8 [64 x 128] uniform 0..255
                   with scalar a_zp 128, B int8 [128 x 64] uniform -128..127 with per-column b_zp uniform -8..8, seed 0,
                   int32 C [64 x 64] (Int8Tests.cs:52-82 semantics);
  closed_form.npz  the 2 x 2 x 3 product with known sums [[-3, 5, -4], [-5, 9, -6]] (MultiDeviceTests.cs:30-31, 53-55);
  dq_vectors.npz   DynamicQuantizeLinear on inputs chosen for ties, NaN, zeros, one-signed ranges, denormals and the
                   float extremes (Int8Tests.cs:576-615 semantics).

Every output is computed twice, by the C oracle and independently with numpy (int64 matmul; float32 arithmetic with
round-half-to-even), and written only when both agree.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402


def c1_smoke():
    m, n, k = 64, 64, 128
    a = oracle.synth_uniform_i32(m * k, 0, 0, 0, 255).astype(np.uint8)
    b = oracle.synth_uniform_i32(k * n, 0, 1, -128, 127).astype(np.int8)
    za = np.array([128], np.uint8)
    zb = oracle.synth_uniform_i32(n, 0, 2, -8, 8).astype(np.int8)
    c = oracle.int8_gemm(oracle.Gemm(m, n, k), a, False, b.view(np.uint8), True, (za, False, 0), (zb.view(np.uint8), True, 0))
    ref = (a.reshape(m, k).astype(np.int64) - 128) @ (b.reshape(k, n).astype(np.int64) - zb.astype(np.int64)[None, :])
    ref = ref.astype(np.int64).astype(np.uint32).view(np.int32).ravel()   # wrap modulo 2^32
    assert np.array_equal(c, ref), "oracle and numpy disagree on the smoke product"
    return dict(a=a, b=b, za=za, zb=zb, c=c.astype(np.int32), shape=np.array([m, n, k], np.int32))


def closed_form():
    a = np.array([1, 2, 3, 4, 5, 6], np.uint8)
    b = np.array([1, -1, 2, -2, 3, -3], np.int8)
    c = oracle.int8_gemm(oracle.Gemm(2, 3, 2), a, False, b.view(np.uint8), True)
    want = np.array([-3, 5, -4, -5, 9, -6], np.int32)
    assert np.array_equal(c, want), c
    return dict(a=a, b=b, c=want)


def numpy_dynamic_quantize(x):
    """DynamicQuantizeLinear in numpy float32: range widened to include 0, NaN ignored, scale (hi - lo) / 255 (1 when
    zero), zero point rint(-lo / scale) clamped to 0..255, y = clamp(rint(x / scale) + zp), NaN -> 0."""
    x = np.asarray(x, np.float32)
    finite = x[~np.isnan(x)]
    lo = np.float32(min(0.0, float(finite.min()))) if finite.size else np.float32(0)
    hi = np.float32(max(0.0, float(finite.max()))) if finite.size else np.float32(0)
    with np.errstate(all="ignore"):
        scale = np.float32(np.float32(hi - lo) / np.float32(255))
        if scale == 0 or not np.isfinite(scale):
            scale = np.float32(1) if scale == 0 else scale
        zp = int(np.clip(np.rint(np.float32(-lo) / scale), 0, 255))
        q = np.rint(x / scale)
        y = np.where(np.isnan(x), 0, np.clip(q + zp, 0, 255)).astype(np.uint8)
    return y, scale, zp


def dq_vectors():
    cases = [
        np.array([0.0], np.float32),
        np.array([-0.0, 0.0], np.float32),
        np.array([np.nan, np.nan], np.float32),
        np.array([1.0, np.nan, -1.0], np.float32),
        np.array([255.0, 0.0, 127.5, 128.5, 0.5, 1.5, 2.5], np.float32),   # ties at scale 1
        np.array([-3.0, -2.0, -1.0], np.float32),                          # all negative: hi widened to 0
        np.array([2.0, 3.0, 4.0], np.float32),                             # all positive: lo widened to 0
        np.array([1e-42, 3e-42, -2e-42], np.float32),                      # denormals
        np.array([3e38, -3e38, 1.0], np.float32),                          # range overflows to inf
        np.array([1e30, -1e30, 0.0], np.float32),
        oracle.dq_input(1000, 7, 0),
        oracle.dq_input(777, 9, 1),
    ]
    xs, ys, scales, zps, offs = [], [], [], [], [0]
    for x in cases:
        y, s, z = oracle.dynamic_quantize(x)
        ny, ns, nz = numpy_dynamic_quantize(x)
        with np.errstate(over="ignore"):
            finite_range = np.isfinite(np.float32(np.nanmax(np.abs(x))) * 2) if np.any(~np.isnan(x)) else True
        if finite_range:   # (a range that overflows float32 is the oracle's alone: its special-input test pins it)
            assert np.array_equal(y, ny) and np.float32(s).view(np.uint32) == ns.view(np.uint32) and z == nz, x[:8]
        xs.append(x)
        ys.append(y)
        scales.append(np.float32(s))
        zps.append(z)
        offs.append(offs[-1] + x.size)
    return dict(x=np.concatenate(xs), y=np.concatenate(ys), scale=np.array(scales, np.float32),
                zero=np.array(zps, np.uint8), offsets=np.array(offs, np.int64))


def main():
    for name, fn in (("c1_smoke", c1_smoke), ("closed_form", closed_form), ("dq_vectors", dq_vectors)):
        data = fn()
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **data)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
