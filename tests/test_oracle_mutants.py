"""The oracle's pins have teeth (CPU only): each pin of tests/test_oracle.py, written here as a check that takes an
implementation, passes for the oracle and fails for implementations with one plausible mistake planted (a dropped
zero point, a transposed operand, a flipped sign, one rounding instead of two, half away from zero instead of half to
even, a range not adjusted to include 0, truncation instead of rounding, an unwrapped negative index, padding with 0
instead of the zero point). The mutants are small Python functions over the pins' tiny inputs; nothing here is used
to check the GPU."""
import numpy as np
import pytest

import cases
import oracle
from test_oracle import _conv_loops, numpy_sums


# ------------------------------------------------------------------ pins, each taking the implementation

def pin_sums(gemm) -> bool:
    """The reference's closed form and numpy's int64 product on zero-point cases (gemm: oracle.int8_gemm's shape)."""
    p = oracle.Gemm(2, 3, 2)
    a = np.array([1, 2, 3, 4], np.uint8)
    b = np.array([1, -1, 2, -2, 3, -3], np.int8).view(np.uint8)
    if gemm(p, a, False, b, True).tolist() != [-3, 5, -4, -5, 9, -6]:
        return False
    rng = np.random.default_rng(9)
    for m, n, k in ((3, 5, 7), (4, 2, 9)):
        p = oracle.Gemm(m, n, k)
        a = rng.integers(0, 256, m * k, dtype=np.uint8)
        b = rng.integers(0, 256, k * n, dtype=np.uint8)
        za = (np.array([200], np.uint8), False, 0)
        zb = (rng.integers(0, 256, n, dtype=np.uint8), True, 0)
        if not np.array_equal(gemm(p, a, False, b, True, za, zb), numpy_sums(p, a, False, b, True, za, zb)):
            return False
    return True


def pin_float_epilogue(epi) -> bool:
    """Two float32 roundings (numpy float32 arithmetic) (epi: oracle.float_epilogue's shape)."""
    rng = np.random.default_rng(0)
    sums = rng.integers(-2**31, 2**31, 2000, dtype=np.int64).astype(np.int32)
    n = 20
    scale = rng.uniform(1e-5, 1e-2, n).astype(np.float32)
    fb = rng.uniform(-2, 2, n).astype(np.float32)
    cols = np.arange(sums.size) % n
    want = (sums.astype(np.float32) * scale[cols]).astype(np.float32) + fb[cols]
    return np.array_equal(epi(sums, n, scale, True, None, fb).view(np.uint32), want.view(np.uint32))


def pin_requant(requant) -> bool:
    """The explicit tie and saturation expectations."""
    return (requant(5, 0.5, 0, True) == 2 and requant(7, 0.5, 0, True) == 4 and requant(-5, 0.5, 0, False) == -2
            and requant(1, 1e9, 3, True) == 255 and requant(1, float("nan"), 5, False) == -128)


def pin_dq(dq) -> bool:
    """The ONNX DynamicQuantizeLinear examples and the hand-derived vectors (dq: x -> (y, scale, zero point))."""
    for x, want_y, want_z in cases.DQ_ONNX_EXAMPLES:
        y, _, z = dq(np.array(x, np.float32))
        if list(y) != want_y or z != want_z:
            return False
    for x, want_y, want_s, want_z in cases.DQ_HAND_VECTORS:
        y, s, z = dq(np.array(x, np.float32))
        if (list(y), float(s), z) != (want_y, want_s, want_z):
            return False
    return True


def pin_f2h(f2h) -> bool:
    """numpy's float16 cast (round to nearest even) on values that round up, down and to even."""
    vals = np.array([1.0, 1.0 + 2**-11, 1.0 + 3 * 2**-11, 1.0 + 2**-10 + 2**-12, 65504.0, 65520.0, 6e-8, -2.5e-5,
                     0.1, -3.14159], np.float32)
    with np.errstate(over="ignore"):   # 65520 rounds to infinity
        return all(f2h(float(v)) == int(np.float32(v).astype(np.float16).view(np.uint16)) for v in vals)


def pin_gather(gather) -> bool:
    """The ONNX Gather examples and the negative-index known answer."""
    d0 = np.array([[1.0, 1.2], [2.3, 3.4], [4.5, 5.7]], np.float32)
    out, bad = gather(d0, d0.shape, 0, [0, 1, 1, 2])
    if bad is not None or out.tolist() != np.array([1.0, 1.2, 2.3, 3.4, 2.3, 3.4, 4.5, 5.7], np.float32).tolist():
        return False
    out, bad = gather(np.arange(4, dtype=np.uint8), [4], 0, [-1, -4, 4, 0, -5])
    return out.tolist() == [3, 0, 0, 0, 0] and bad == 2


def pin_conv(conv) -> bool:
    """The ONNX ConvInteger examples, the second with padding (padded taps take x's zero point)."""
    x = np.array([2, 3, 4, 5, 6, 7, 8, 9, 10], np.uint8)
    c = dict(Batch=1, InChannels=1, Height=3, Width=3, OutChannels=1, KernelHeight=2, KernelWidth=2)
    if conv(c, x, False, np.ones(4, np.uint8), False, np.array([1], np.uint8)).tolist() != [12, 16, 24, 28]:
        return False
    c.update(PadTop=1, PadLeft=1, PadBottom=1, PadRight=1)
    return conv(c, x, False, np.ones(4, np.uint8), False, np.array([1], np.uint8)).tolist() == \
        [1, 3, 5, 3, 5, 12, 16, 9, 11, 24, 28, 15, 7, 15, 17, 9]


# ------------------------------------------------------------------ mutants

def _wrap32(v):
    return ((np.asarray(v, np.int64) + 2**31) % 2**32 - 2**31).astype(np.int32)


def _sums_mutant(kind):
    def gemm(p, a, a_signed, b, b_signed, za=None, zb=None):
        A = (a.view(np.int8) if a_signed else a).astype(np.int64)[:p.M * p.K].reshape(p.M, p.K)
        B = (b.view(np.int8) if b_signed else b).astype(np.int64)[:p.K * p.N].reshape(p.K, p.N)
        if kind == "transposed B" and p.K == p.N:
            B = B.T
        elif kind == "transposed B":
            B = B.ravel().reshape(p.N, p.K).T
        if za is not None:
            z = (za[0].view(np.int8) if a_signed else za[0]).astype(np.int64)
            zv = z[:p.M][:, None] if za[1] else z[0]
            A = A + zv if kind == "zero point of A added" else A - zv
        if zb is not None and kind != "zero point of B dropped":
            z = (zb[0].view(np.int8) if b_signed else zb[0]).astype(np.int64)
            B = B - (z[:p.N][None, :] if zb[1] else z[0])
        return _wrap32((A @ B).ravel())
    return gemm


def _epilogue_one_rounding(sums, n, scale, scale_vec, ibias=None, fbias=None):
    cols = np.arange(sums.size) % n
    s = scale[cols] if scale_vec else scale[0]
    f = 0.0 if fbias is None else fbias[cols].astype(np.float64)
    return (sums.astype(np.float64) * np.asarray(s, np.float64) + f).astype(np.float32)


def _requant_half_away(acc, mult, zero, unsigned):
    lo, hi = (0, 255) if unsigned else (-128, 127)
    v = np.float32(acc) * np.float32(mult)
    if np.isnan(v):
        return lo
    r = np.float32(np.sign(v) * np.floor(abs(v) + np.float32(0.5)))
    return int(min(max(r, np.float32(lo - zero)), np.float32(hi - zero))) + zero


def _dq_mutant(kind):
    def dq(x):
        x = np.asarray(x, np.float32)
        lo, hi = np.float32(x.min()), np.float32(x.max())
        if kind != "range not adjusted to include 0":
            lo, hi = min(lo, np.float32(0)), max(hi, np.float32(0))
        scale = np.float32(hi - lo) / np.float32(256 if kind == "scale over 256" else 255)
        rnd = (lambda v: np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))) if kind == "half away from zero" \
            else np.rint
        z = rnd(np.float32(lo / scale) if kind == "zero point sign flipped" else np.float32(0) - np.float32(lo / scale))
        zp = int(min(max(z, 0), 255))
        y = np.clip(rnd((x / scale).astype(np.float32)) + np.float32(zp), 0, 255).astype(np.uint8)
        return y, scale, zp
    return dq


def _f2h_truncating(f):
    b = int(np.float32(f).view(np.uint32))
    sign, exp, man = b >> 31, (b >> 23) & 0xFF, b & 0x7FFFFF
    e = exp - 127 + 15
    if e >= 31:
        return (sign << 15) | 0x7C00
    if e <= 0:
        return (sign << 15) | ((man | 0x800000) >> (14 - e)) if e > -10 else sign << 15
    return (sign << 15) | (e << 10) | (man >> 13)


def _gather_no_negative(data, shape, axis, indices, wide=False):
    n_axis, out, bad = shape[axis], [], None
    flat = np.asarray(data).reshape(shape)
    for i, v in enumerate(indices):
        if 0 <= v < n_axis:
            out.append(np.take(flat, [v], axis=axis))
        else:
            bad = i if bad is None else bad
            out.append(np.zeros_like(np.take(flat, [0], axis=axis)))
    return np.concatenate(out, axis=axis).ravel(), bad


def _conv_pad_zero(c, x, xs, w, ws, xz=None, wz=None, wz_vec=False):
    # Padded taps contribute (0 - xz)(w - wz) instead of nothing: the padding is filled with 0, not x's zero point.
    c2 = {k: v for k, v in c.items() if not k.startswith("Pad")}
    PT, PL, PB, PR = (c.get(k, 0) for k in ("PadTop", "PadLeft", "PadBottom", "PadRight"))
    H, W = c["Height"] + PT + PB, c["Width"] + PL + PR
    xp = np.zeros((c["Batch"], c["InChannels"], H, W), np.uint8)
    xp[:, :, PT:PT + c["Height"], PL:PL + c["Width"]] = x.reshape(c["Batch"], c["InChannels"], c["Height"], c["Width"])
    c2.update(Height=H, Width=W)
    return _conv_loops(c2, xp.ravel(), xs, w, ws, xz, wz, wz_vec)


# ------------------------------------------------------------------ the oracle passes every pin ...

def test_the_oracle_passes_every_pin():
    assert pin_sums(oracle.int8_gemm)
    assert pin_sums(oracle.int8_gemm_identity)
    assert pin_float_epilogue(oracle.float_epilogue)
    assert pin_requant(oracle.requant)
    assert pin_dq(oracle.dynamic_quantize)
    assert pin_f2h(oracle.f2h)
    assert pin_gather(oracle.gather)
    assert pin_conv(lambda c, x, xs, w, ws, xz=None: oracle.conv_integer(c, x, xs, w, ws, xz))


# ------------------------------------------------------------------ ... and each mutant fails one

@pytest.mark.parametrize("kind", ["zero point of B dropped", "transposed B", "zero point of A added"])
def test_sums_pins_catch(kind):
    assert not pin_sums(_sums_mutant(kind))


def test_float_epilogue_pin_catches_one_rounding():
    assert not pin_float_epilogue(_epilogue_one_rounding)


def test_requant_pin_catches_half_away_from_zero():
    assert not pin_requant(_requant_half_away)


@pytest.mark.parametrize("kind", ["half away from zero", "zero point sign flipped", "range not adjusted to include 0",
                                  "scale over 256"])
def test_dq_pins_catch(kind):
    assert not pin_dq(_dq_mutant(kind))


def test_f2h_pin_catches_truncation():
    assert not pin_f2h(_f2h_truncating)


def test_gather_pin_catches_unwrapped_negative_indices():
    assert not pin_gather(_gather_no_negative)


def test_conv_pin_catches_zero_padding():
    assert not pin_conv(_conv_pad_zero)


# ------------------------------------------------------------------ the large-K GPU case has teeth

def _identity_one(k, a_byte, za, b_byte, zb, mul) -> int:
    """One output of the product kernels' signed-domain identity for constant uint8 operands and zero points,
    C = acc - w' s - z' (t - K w') modulo 2^32 (s, t the byte sums, z', w' the zero points, all moved by -128), with
    the two correction products formed by `mul`."""
    s, t = k * (a_byte - 128), k * (b_byte - 128)
    zp, wp = za - 128, zb - 128
    acc = k * (a_byte - 128) * (b_byte - 128)
    v = (acc - mul(wp, s) - mul(zp, t - k * wp)) & 0xFFFFFFFF
    return v - (1 << 32) if v & 0x80000000 else v


def _mul32(a, b) -> int:
    return (a * b) & 0xFFFFFFFF


def _mul24(a, b) -> int:
    """The 24-bit multiply: each operand's low 24 bits as a signed number, the product's low 32 bits."""
    def sx(x):
        x &= 0xFFFFFF
        return x - (1 << 24) if x & 0x800000 else x
    return (sx(a) * sx(b)) & 0xFFFFFFFF


def test_large_k_case_catches_a_24_bit_correction_multiply():
    # The adversarial fill of test_large_k_corrections_are_bit_exact (A = 0 under zero point 255, B = 255 under zero
    # point 0): the identity with 32-bit products gives the definition's sums at both sizes; with the 24-bit multiply
    # it still does at K = 32704, below the kernels' switch, and no longer at K = 40960.
    import test_int8_gpu
    sizes = {c[3] for c in test_int8_gpu.LARGE_K_CASES}
    assert {32704, 40960} <= sizes
    for k in (32704, 40960):
        want = int(np.int64(-255 * 255 * k).astype(np.int64) & 0xFFFFFFFF)
        want = want - (1 << 32) if want & 0x80000000 else want
        assert _identity_one(k, 0x00, 0xFF, 0xFF, 0x00, _mul32) == want
        assert (_identity_one(k, 0x00, 0xFF, 0xFF, 0x00, _mul24) == want) == (k < 32768)
