"""The committed fixtures (tests/golden/make_golden.py) against the oracle and against numpy, on the CPU."""
import os

import numpy as np

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def test_smoke_fixture_reproduces():
    f = load("c1_smoke")
    m, n, k = (int(v) for v in f["shape"])
    a, b, za, zb, c = f["a"], f["b"], f["za"], f["zb"], f["c"]
    assert (a.dtype, b.dtype, c.dtype, a.size, b.size, c.size) == (np.uint8, np.int8, np.int32, m * k, k * n, m * n)
    got = oracle.int8_gemm(oracle.Gemm(m, n, k), a, False, b.view(np.uint8), True, (za, False, 0), (zb.view(np.uint8), True, 0))
    assert np.array_equal(got, c)
    ref = (a.reshape(m, k).astype(np.int64) - int(za[0])) @ (b.reshape(k, n).astype(np.int64) - zb.astype(np.int64)[None, :])
    assert np.array_equal(ref.astype(np.uint32).view(np.int32).ravel(), c)
    # the inputs are the seeded generator's (seed 0)
    assert np.array_equal(a, oracle.synth_uniform_i32(m * k, 0, 0, 0, 255).astype(np.uint8))


def test_closed_form_fixture():
    f = load("closed_form")
    assert f["c"].tolist() == [-3, 5, -4, -5, 9, -6]
    got = oracle.int8_gemm(oracle.Gemm(2, 3, 2), f["a"], False, f["b"].view(np.uint8), True)
    assert np.array_equal(got, f["c"])


def test_dynamic_quantize_fixture():
    f = load("dq_vectors")
    offs = f["offsets"]
    for i in range(len(offs) - 1):
        x = f["x"][offs[i]:offs[i + 1]]
        y, s, z = oracle.dynamic_quantize(x)
        assert np.array_equal(y, f["y"][offs[i]:offs[i + 1]]), i
        assert np.float32(s).view(np.uint32) == f["scale"][i].view(np.uint32), i
        assert z == int(f["zero"][i]), i
