"""The reference tests' case lists for the int8 path, restated as data, plus the data each case runs on.

Every list cites the reference test it restates (tests/RecursiveAI.OneGpu.Kernels.Tests/...); the data comes from the
oracle's restatement of the same generators, so a case here holds the same bytes as the reference test's case.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import oracle

# Int8Tests.cs:9-21 (ModelShapes): BERT and MiniLM projections at 128 tokens, batch 1 and 8.
MODEL_SHAPES = [
    ("minilm qkv/proj b1x128", 128, 384, 384),
    ("minilm ffn-up b1x128", 128, 1536, 384),
    ("minilm ffn-down b1x128", 128, 384, 1536),
    ("bert proj b1x128", 128, 768, 768),
    ("bert ffn-up b1x128", 128, 3072, 768),
    ("bert ffn-down b1x128", 128, 768, 3072),
    ("minilm ffn-up b8x128", 1024, 1536, 384),
    ("bert proj b8x128", 1024, 768, 768),
    ("bert ffn-up b8x128", 1024, 3072, 768),
    ("bert ffn-down b8x128", 1024, 768, 3072),
]

# Int8Tests.cs:219 (EdgeShapesAreBitExact shapes).
EDGE_SHAPES = [(1, 1, 1), (1, 1, 0), (3, 5, 7), (64, 64, 16), (65, 63, 17), (1, 257, 33), (130, 1, 31), (17, 129, 1),
               (2, 2, 4096), (33, 31, 300), (4, 4, 32), (7, 9, 31), (40, 40, 65), (5, 3, 63), (33, 40, 96)]


def problem(m, n, k, batch=1, trans_b=False, off_a=0, off_b=0, off_c=0, lda_extra=0, ldb_extra=0, share_b=False):
    """Int8Tests.Problem (Int8Tests.cs:196-210)."""
    p = oracle.Gemm(m, n, k, Batch=batch, TransposeB=trans_b, OffsetA=off_a, OffsetB=off_b, OffsetC=off_c)
    p.Lda = k + lda_extra
    p.Ldb = (k if trans_b else n) + ldb_extra
    p.StrideA = m * p.Lda
    p.StrideB = 0 if share_b else (n if trans_b else k) * p.Ldb
    if batch == 1:
        p.StrideA = 0
        p.StrideB = 0
    return p


@dataclass
class Case:
    """Int8Tests.Case (Int8Tests.cs:99-106): signedness, zero-point modes (0 none, 1 scalar, 2 vector), extreme fill."""

    name: str
    p: oracle.Gemm
    a_signed: bool
    b_signed: bool
    za_mode: int
    zb_mode: int
    fill: int = -1
    data: dict = field(default_factory=dict)


def edge_cases() -> list[Case]:
    """Every case of EdgeShapesAreBitExact (Int8Tests.cs:214-270), in the reference's order."""
    cases = []
    for (m, n, k) in EDGE_SHAPES:
        for s in range(4):
            for za in range(3):
                zb = (za + s) % 3
                cases.append(Case(f"{m}x{n}x{k}", problem(m, n, k, off_a=za, off_b=1 + zb, off_c=s),
                                  (s & 1) != 0, (s & 2) != 0, za, zb))
    cases.append(Case("transposed B", problem(40, 70, 50, trans_b=True, off_a=3, off_b=1), False, True, 1, 2))
    cases.append(Case("padded rows", problem(21, 22, 23, lda_extra=5, ldb_extra=3, off_a=2, off_b=3), True, True, 2, 1))
    cases.append(Case("batch 5 shared B", problem(9, 70, 33, batch=5, share_b=True, off_a=1, off_b=2), False, True, 1, 2))
    cases.append(Case("batch 3", problem(70, 9, 33, batch=3, off_a=3, off_b=1, off_c=3), False, False, 2, 1))
    for fill in (0x00, 0x7F, 0x80, 0xFF):
        for s in range(4):
            cases.append(Case(f"extreme {fill:02X}", problem(37, 41, 77, trans_b=(s & 1) != 0), (s & 1) != 0,
                              (s & 2) != 0, 1 + (s & 1), 2 - (s & 1), fill))
    for fill in (0x00, 0x7F, 0x80, 0xFF):
        for s in range(4):
            for (m, n, k) in ((33, 35, 4096), (3, 70, 4096), (65, 64, 1024)):
                cases.append(Case(f"long extreme {fill:02X} {m}x{n}x{k}", problem(m, n, k, trans_b=(s & 1) != 0),
                                  (s & 1) != 0, (s & 2) != 0, (s + fill) % 3, (s + 1) % 3, fill))
    return cases


def model_case(name, m, n, k) -> Case:
    """ModelShapesAreBitExact (Int8Tests.cs:285-317): u8 activations with a scalar zero point, int8 weights stored N x K."""
    return Case(name, problem(m, n, k, trans_b=True), False, True, 1, 0)


def case_data(c: Case, seed: int) -> dict:
    """The buffers of RunInt32 (Int8Tests.cs:118-133): raw bytes of A, B and the zero points, extremes filled."""
    p = c.p
    lda = p.Lda if p.Lda else p.K
    ldb = p.Ldb if p.Ldb else (p.K if p.TransposeB else p.N)
    len_a = p.OffsetA + (p.Batch - 1) * p.StrideA + p.M * lda + 4
    len_b = p.OffsetB + (p.Batch - 1) * p.StrideB + (p.N if p.TransposeB else p.K) * ldb + 4
    a = oracle.bytes_(len_a, seed)
    b = oracle.bytes_(len_b, seed + 1)
    za = None if c.za_mode == 0 else oracle.bytes_(1 + (p.M if c.za_mode == 2 else 0), seed + 2)
    zb = None if c.zb_mode == 0 else oracle.bytes_(1 + (p.N if c.zb_mode == 2 else 0), seed + 3)
    if c.fill >= 0:
        a[:] = c.fill
        b[:] = c.fill ^ 0xFF
        if za is not None:
            za[:] = c.fill
        if zb is not None:
            zb[:] = c.fill ^ 0x80
    return {"a": a, "b": b, "za": za, "zb": zb}


def reference_sums(c: Case, d: dict) -> np.ndarray:
    """The oracle's definition-form sums for a case (dense Batch*M*N int32)."""
    za = None if d["za"] is None else (d["za"], c.za_mode == 2, 0)
    zb = None if d["zb"] is None else (d["zb"], c.zb_mode == 2, 0)
    return oracle.int8_gemm(c.p, d["a"], c.a_signed, d["b"], c.b_signed, za, zb)


# Int8Tests.cs:626 (DynamicQuantizeIsBitExact counts) and the seven input kinds of 638-646.
DQ_COUNTS = [1, 2, 3, 255, 256, 257, 1023, 1024, 1025, 4097, 128 * 384, 128 * 768, 1024 * 768, 1024 * 384 + 17,
             262144 + 3]
DQ_KINDS = [0, 1, 2, 3, 4, 5, 6]


def dq_cases():
    """(count, kind, seed) in the reference's order: seed counts up from 1 across counts x kinds."""
    seed = 1
    for count in DQ_COUNTS:
        for kind in DQ_KINDS:
            yield count, kind, seed
            seed += 1


# DequantizeTests.cs:93-97 and 263-267: (shape, axis, perAxis).
DEQUANT_SHAPES = [
    ([1], 0, False), ([7], 0, True), ([5, 6], 0, True), ([5, 6], 1, True), ([5, 6], -1, False), ([2, 3, 4, 5], 1, True),
    ([2, 3, 4, 5], -1, True), ([1031, 3], 0, True), ([3, 257], 1, True), ([4, 1, 9], 2, True), ([100003], 0, False),
    ([384, 768], 1, True),
]

# Beyond the reference's shapes: tensors of several 4096-element blocks (the aligned kernels' vector path), per axis
# with inner 5 and 4100 (an axis step inside a run of four elements and across blocks), per column with axes of 300
# and 4096 (runs of four columns read with one vector load) and of 7 (the axis wraps inside a run), and a per-tensor
# count with a ragged last block.
DEQUANT_SHAPES_BLOCKS = [([64, 96, 5], 1, True), ([3, 4100], 0, True), ([8, 7, 300], 2, True), ([33, 4096], 1, True),
                         ([2000, 7], 1, True), ([5, 4099], -1, False)]

# DequantizeTests.cs:270: the scale sets of QuantizeIsExact.
QUANT_SCALE_SETS = [[0.5], [1.0], [0.0137, 0.25, 3.3], [1.0 / 255.0, 0.09999], [1e-6, 1e3, 0.7]]


def axis_split(shape, axis, per_axis):
    """(count, axisLen, inner) as DequantizeKernels.Encode splits the tensor (DequantizeKernels.cs:93-107)."""
    count = int(np.prod(shape)) if shape else 1
    if not per_axis:
        return count, 1, 1
    ax = axis + len(shape) if axis < 0 else axis
    inner = int(np.prod(shape[ax + 1:])) if ax + 1 < len(shape) else 1
    return count, shape[ax], inner


# FloatAndRequantizedFormsAreBitExact (Int8Tests.cs:468-501).
FLOAT_SHAPES = [(1, 1, 1), (5, 7, 9), (64, 65, 100), (130, 70, 384), (128, 384, 384), (33, 257, 77)]
REQUANT_OUT = [(True, 128), (False, 0), (True, 0), (False, -5), (True, 255), (False, 127)]

# RequantizationRoundsHalfToEvenAndSaturates (Int8Tests.cs:503-547): (multiplier, zeroY, unsigned).
REQUANT_TIES = [(0.5, 10, True), (0.5, -10, False), (2.5, 0, True), (1e9, 3, True), (-1e9, 3, False),
                (float("nan"), 5, True), (float("nan"), 5, False), (float("inf"), 1, False), (0.0, 7, True)]

# The three worked examples of the ONNX DynamicQuantizeLinear specification (x, expected y, expected zero point):
# a range across zero, an all-negative input (max adjusted to 0) and an all-positive one (min adjusted to 0).
DQ_ONNX_EXAMPLES = [
    ([0, 2, -3, -2.5, 1.34, 0.5], [153, 255, 0, 26, 221, 179], 153),
    ([-1.0, -2.1, -1.3, -2.5, -3.34, -4.0], [191, 121, 172, 96, 42, 0], 255),
    ([1, 2.1, 1.3, 2.5, 3.34, 4.0, 1.5, 2.6, 3.9, 4.0, 3.0, 2.345], [64, 134, 83, 159, 213, 255, 96, 166, 249, 255, 191,
                                                                    149], 0),
]

# Vectors derived by hand, all values exact in float32 (x, expected y, expected scale, expected zero point):
#  - range [0, 255]: scale 1, zero point 0, and x / scale lands on .5: rounds half to even (0.5 -> 0, 1.5 -> 2,
#    2.5 -> 2);
#  - all negative: the range [-255, 0], zero point rne(255) = 255 clamps nothing; -0.5 rounds to -0, giving 255;
#  - range [-127.5, 127.5]: zero point rne(127.5) = 128 (the even neighbour), 127.5 -> 128 + 128 = 256 clamps to 255,
#    -127.5 -> -128 + 128 = 0, +-0.5 -> 0 + 128.
DQ_HAND_VECTORS = [
    ([0, 255, 0.5, 1.5, 2.5], [0, 255, 0, 2, 2], 1.0, 0),
    ([-255, -1, -0.5], [0, 254, 255], 1.0, 255),
    ([-127.5, 127.5, 0.5, -0.5], [0, 255, 128, 128], 1.0, 128),
]


def float_case_data(m, n, k, scale_vec, seed):
    """FloatCase inputs (Int8Tests.cs:334-373): u8 A with scalar zp, int8 B with per-column zp, scales and biases."""
    a = oracle.bytes_(m * k + 4, seed)
    b = oracle.bytes_(k * n + 4, seed + 1)
    za = oracle.bytes_(1, seed + 2)
    zb = oracle.bytes_(n, seed + 3)
    i = np.arange(max(n if scale_vec else 1, 1))
    scale = (np.float32(0.0007) + ((i * 37 + seed) % 101).astype(np.float32) * np.float32(1.3e-5)).astype(np.float32)
    cols = np.arange(n)
    ib = (((cols * 7919) % 20001) - 10000).astype(np.int32)
    fb = ((((cols * 31) % 201) - 100).astype(np.float32) * np.float32(0.0137)).astype(np.float32)
    return a, b, za, zb, scale, ib, fb


def requant_case_data(m, n, k, mult_vec, seed):
    """RequantCase inputs (Int8Tests.cs:375-399)."""
    a = oracle.bytes_(m * k + 4, seed)
    b = oracle.bytes_(k * n + 4, seed + 1)
    za = oracle.bytes_(1, seed + 2)
    i = np.arange(n if mult_vec else 1)
    mult = (np.float32(0.00011) + ((i * 13 + seed) % 59).astype(np.float32) * np.float32(2.7e-6)).astype(np.float32)
    cols = np.arange(n)
    ib = (((cols * 6007) % 4001) - 2000).astype(np.int32)
    return a, b, za, mult, ib


# ------------------------------------------------------------------ gather (GatherTests.cs, IndexRig.cs)

# GatherIsExact's shapes (GatherTests.cs:78-82): (data shape, axis, index count).
GATHER_CASES = [([10], 0, 7), ([10], -1, 1), ([5, 6], 0, 9), ([5, 6], 1, 4), ([5, 6], -1, 11), ([2, 3, 4, 5], 2, 6),
                ([2, 3, 4, 5], -4, 3), ([1, 7], 1, 5), ([4, 1, 9], 0, 8), ([3, 257], 1, 300), ([1031, 3], 0, 1500),
                ([2, 3, 4, 5, 6], 3, 2)]

_M32 = 0xFFFFFFFF


def index_rig_make(dtype, i: np.ndarray) -> np.ndarray:
    """IndexRig.Make<T>(i) (IndexRig.cs:17-57): a hashed payload of every bit pattern (finite floats and halves)."""
    i = np.asarray(i, np.int64)
    h = ((i.astype(np.uint64) * np.uint64(2654435761) + np.uint64(0x9E3779B9)) & np.uint64(_M32))
    h ^= h >> np.uint64(15)
    h = (h * np.uint64(0x85EBCA6B)) & np.uint64(_M32)
    h ^= h >> np.uint64(13)
    dt = np.dtype(dtype)
    if dt == np.float32:
        return (((h & np.uint64(0xFFFFF)).astype(np.int64) - 0x80000).astype(np.float32) / np.float32(1024)).astype(np.float32)
    if dt == np.float16:
        return (((h & np.uint64(0xFFF)).astype(np.int64) - 0x800).astype(np.float32) / np.float32(16)).astype(np.float16)
    if dt in (np.int32, np.uint32):
        return h.astype(np.uint32).view(np.int32).astype(dt) if dt == np.int32 else h.astype(np.uint32)
    if dt in (np.uint8, np.int8):
        return (h >> np.uint64(8)).astype(np.uint8).view(dt)
    if dt == np.int64:
        lo = ((i * 40503 + 17) & _M32).astype(np.uint64)
        return ((h << np.uint64(32)) ^ lo).view(np.int64)
    raise ValueError(dt)


def index_rig_fill(dtype, length: int, seed: int) -> np.ndarray:
    """IndexRig.Fill<T> (IndexRig.cs:62-72), without the padding (the tests pad their buffers themselves)."""
    return index_rig_make(dtype, np.arange(length) + seed * 7919)


def index_rig_random_index(i, n_axis: int, seed: int) -> np.ndarray:
    """IndexRig.RandomIndex (IndexRig.cs:109-117): deterministic indices in [-len, len), some negative."""
    i = np.asarray(i, np.int64)
    h = (((i + seed * 104729) & _M32).astype(np.uint64) * np.uint64(2246822519)) & np.uint64(_M32)
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(3266489917)) & np.uint64(_M32)
    return (h % np.uint64(2 * n_axis)).astype(np.int64) - n_axis


# ------------------------------------------------------------------ ConvInteger (ConvIntegerTests.cs)

def conv_bytes(length: int, seed: int) -> np.ndarray:
    """ConvIntegerTests.Bytes (ConvIntegerTests.cs:19-29): a 32-bit LCG, the top byte of each state. Computed a block
    at a time: the state j steps on is A_j * s + C_j (mod 2^32)."""
    a, c, block = 1664525, 1013904223, 4096
    A, C = np.empty(block, np.uint64), np.empty(block, np.uint64)
    av, cv = 1, 0
    for j in range(block):
        av, cv = (av * a) & _M32, (cv * a + c) & _M32
        A[j], C[j] = av, cv
    out = np.empty(length, np.uint8)
    s = (seed * 2654435761 + 7) & _M32
    for start in range(0, length, block):
        n = min(block, length - start)
        states = (A[:n] * np.uint64(s) + C[:n]) & np.uint64(_M32)
        out[start:start + n] = (states >> np.uint64(24)).astype(np.uint8)
        s = int(states[n - 1])
    return out


def conv_problem(batch, cin, h, w, cout, kh, kw, stride=1, dilation=1, pad=0, groups=1) -> dict:
    """ConvIntegerTests.P (ConvIntegerTests.cs:183-195) as a dict of ConvProblem fields."""
    return dict(Batch=batch, InChannels=cin, Height=h, Width=w, OutChannels=cout, KernelHeight=kh, KernelWidth=kw,
                StrideHeight=stride, StrideWidth=stride, DilationHeight=dilation, DilationWidth=dilation, PadTop=pad,
                PadBottom=pad, PadLeft=pad, PadRight=pad, Groups=groups)


def conv1d(batch, cin, length, cout, kernel, stride=1, dilation=1, pad_begin=0, pad_end=0, groups=1) -> dict:
    """ConvProblem.Conv1D (ConvProblem.cs:127-136)."""
    return dict(Batch=batch, InChannels=cin, Height=1, Width=length, OutChannels=cout, KernelHeight=1,
                KernelWidth=kernel, StrideHeight=1, StrideWidth=stride, DilationHeight=1, DilationWidth=dilation,
                PadTop=0, PadBottom=0, PadLeft=pad_begin, PadRight=pad_end, Groups=groups)


def conv_spread(name: str, p: dict) -> list:
    """ConvIntegerTests.Spread (ConvIntegerTests.cs:223-233): the four signedness combinations; zero points none /
    one / per channel in turn."""
    return [dict(name=f"{name} s{s}", p=p, xs=(s & 1) != 0, ws=(s & 2) != 0, xzm=1 - (s & 1), wzm=(s + 1) % 3,
                 fill=-1, scratch_images=0) for s in range(4)]


def conv_edge_cases() -> list:
    """EdgeGeometriesAreBitExact's cases (ConvIntegerTests.cs:235-275)."""
    cases = []
    cases += conv_spread("1x1 pointwise", conv_problem(2, 5, 7, 9, 6, 1, 1))
    cases += conv_spread("3x3 pad1", conv_problem(1, 3, 10, 13, 4, 3, 3, pad=1))
    cases += conv_spread("3x3 stride2 pad1 odd", conv_problem(2, 4, 9, 11, 5, 3, 3, stride=2, pad=1))
    cases += conv_spread("5x5 dilation2", conv_problem(1, 2, 14, 15, 3, 5, 5, dilation=2, pad=4))
    cases += conv_spread("groups 2", conv_problem(2, 4, 8, 8, 6, 3, 3, pad=1, groups=2))
    cases += conv_spread("depthwise", conv_problem(2, 6, 9, 10, 6, 3, 3, pad=1, groups=6))
    cases += conv_spread("1d k3", conv1d(2, 5, 31, 7, 3, pad_begin=1, pad_end=1))
    cases += conv_spread("1d stride2", conv1d(1, 4, 40, 6, 3, stride=2, pad_begin=1, pad_end=1))
    cases += conv_spread("1x1 image", conv_problem(3, 8, 1, 1, 4, 1, 1))
    cases += conv_spread("kernel = image", conv_problem(1, 3, 5, 5, 2, 5, 5))
    asym = conv_problem(1, 3, 12, 9, 4, 3, 2)
    asym.update(PadTop=2, PadBottom=0, PadLeft=0, PadRight=3, StrideHeight=2)
    cases += conv_spread("asymmetric padding", asym)
    off = conv_problem(2, 3, 6, 7, 5, 3, 3, pad=1)
    off.update(OffsetX=3, OffsetW=5, OffsetY=7)
    cases += conv_spread("offsets", off)
    for s in range(4):
        for fill in (0, 127, 128, 255):
            cases.append(dict(name=f"extremes {fill} s{s}", p=conv_problem(1, 17, 6, 6, 3, 3, 3, pad=1),
                              xs=(s & 1) != 0, ws=(s & 2) != 0, xzm=1, wzm=2, fill=fill, scratch_images=0))
    # This library's own paths: 1 x 1 unit-stride convolutions over 16-byte image rows multiply x in place (grouped,
    # and with a per-channel zero point), and the same shape with x at an odd offset goes through the pack.
    cases += conv_spread("1x1 in place, groups 2", conv_problem(2, 8, 8, 8, 6, 1, 1, groups=2))
    pw_off = conv_problem(2, 4, 4, 8, 5, 1, 1)
    pw_off.update(OffsetX=3)
    cases += conv_spread("1x1 at an odd offset", pw_off)
    cases.append(dict(name="chunked batch, scratch for 1 image", p=conv_problem(3, 3, 8, 8, 4, 3, 3, pad=1), xs=False,
                      ws=False, xzm=1, wzm=1, fill=-1, scratch_images=1))
    cases.append(dict(name="grouped, scratch for 2 images", p=conv_problem(3, 4, 8, 8, 6, 3, 3, pad=1, groups=2),
                      xs=True, ws=True, xzm=1, wzm=2, fill=-1, scratch_images=2))
    return cases


def conv_model_cases() -> list:
    """WhisperStemIsBitExact and ResNetShapesAreBitExact (ConvIntegerTests.cs:277-307)."""
    c = lambda name, p, xs, ws, wzm: dict(name=name, p=p, xs=xs, ws=ws, xzm=1, wzm=wzm, fill=-1, scratch_images=0)  # noqa: E731
    return [
        c("whisper conv1 u8 x i8 w", conv1d(1, 80, 3000, 768, 3, pad_begin=1, pad_end=1), False, True, 1),
        c("whisper conv1 u8 x u8 w, per channel", conv1d(1, 80, 3000, 768, 3, pad_begin=1, pad_end=1), False, False, 2),
        c("whisper conv2 u8 x i8 w", conv1d(1, 768, 1500, 768, 3, stride=2, pad_begin=1, pad_end=1), False, True, 1),
        c("resnet stem 7x7/2", conv_problem(1, 3, 224, 224, 64, 7, 7, stride=2, pad=3), False, True, 1),
        c("resnet 3x3 56x56", conv_problem(1, 64, 56, 56, 64, 3, 3, pad=1), False, True, 2),
        c("resnet 1x1 56x56 b2", conv_problem(2, 64, 56, 56, 256, 1, 1), True, True, 1),
        c("mobilenet depthwise 3x3", conv_problem(1, 96, 28, 28, 96, 3, 3, pad=1, groups=96), False, True, 2),
    ]
