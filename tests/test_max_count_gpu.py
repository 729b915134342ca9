"""The element-wise passes at the largest counts the boundary takes: DynamicQuantizeLinear at 2^31 - 1 elements (a
float32 tensor of 8 GiB, whose last block of 4096 elements holds 4095), DequantizeLinear (uint8 to float32) and
QuantizeLinear (float32 to uint8) at 2^31 - 4 (a byte tensor's buffer holds whole 32-bit words, as the reference's
GpuKernelBuffers.PaddedBoolLength requires, and at most 2^31 - 1 elements; its last block holds 4092), each checked
against the oracle over every element; and a product and a gather whose output or table reaches the boundary's
element limit, against closed forms. The inputs repeat a short pattern whose period (4099) does not divide the
block, so they are cheap to make; the extreme values of x sit at its first and last elements, in the first and the
last workgroup."""
from __future__ import annotations

import gc

import numpy as np
import pytest

import oracle
import onegpu_hip as og
from gpu_rig import device, run, say

pytestmark = pytest.mark.gpu

MAX = 2**31 - 1
MAX4 = 2**31 - 4   # the largest whole number of 32-bit words of bytes


@pytest.fixture(scope="module")
def x_max():
    base = ((np.arange(4099, dtype=np.float32) * np.float32(0.37)) % np.float32(8.0) - np.float32(3.0)).astype(np.float32)
    x = np.resize(base, MAX)
    x[0], x[-1] = np.float32(-6.25), np.float32(7.5)
    yield x
    del x
    gc.collect()


def _same(got: np.ndarray, want: np.ndarray) -> int:
    """Mismatching elements, compared in chunks of 2^28 so no temporary the size of the tensor is made."""
    bad = 0
    for i in range(0, want.size, 1 << 28):
        bad += int(np.count_nonzero(got[i:i + (1 << 28)] != want[i:i + (1 << 28)]))
    return bad


def test_dynamic_quantize_at_the_largest_count(x_max):
    d = device()
    k = og.DynamicQuantizeKernels(d)
    say(f"dq at count {MAX}")
    bx, by = d.CreateBuffer(x_max), d.CreateBufferOf(og.ElementType.UInt8, MAX)
    bs, bz = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
    run(d, lambda e: k.Encode(e, bx, 0, MAX, by, 0, bs, 0, bz, 0))
    got = by.Read()
    scale, zero = bs.Read()[0], int(bz.Read()[0])
    del bx, by
    wy, ws, wz = oracle.dynamic_quantize(x_max)
    bad = _same(got, wy)
    say(f"ROW dq at count {MAX} | scale {scale!r} want {ws!r} | zero {zero} want {wz} | mismatching bytes {bad}")
    assert np.float32(scale).view(np.uint32) == np.float32(ws).view(np.uint32) and zero == wz
    assert bad == 0


def test_dequantize_at_the_largest_count():
    d = device()
    k = og.DequantizeKernels(d)
    say(f"dequantize u8 -> f32 at count {MAX4}")
    q = np.resize((np.arange(251, dtype=np.uint32) * 97 % 256).astype(np.uint8), MAX4)
    scale, zero = np.array([0.0375], np.float32), np.array([131, 0, 0, 0], np.uint8)
    bq, bs, bzp = d.CreateBuffer(q), d.CreateBuffer(scale), d.CreateBuffer(zero)
    bo = d.CreateBufferOf(og.ElementType.Float32, MAX4)
    run(d, lambda e: k.Encode(e, bq, 0, [MAX4], 0, False, bs, 0, bzp, 0, bo, 0))
    kernel = d.LastKernel
    got = bo.Read()
    del bo, bq
    want = oracle.dequantize(q, scale, zero=zero[:1])
    bad = _same(got.view(np.uint32), want.view(np.uint32))
    say(f"ROW dequantize at count {MAX4} | {kernel} | mismatching elements {bad}")
    assert bad == 0


def test_quantize_at_the_largest_count(x_max):
    d = device()
    k = og.DequantizeKernels(d)
    say(f"quantize f32 -> u8 at count {MAX4}")
    x = x_max[:MAX4]
    scale, zero = np.array([0.05], np.float32), np.array([117, 0, 0, 0], np.uint8)
    bx, bs, bzp = d.CreateBuffer(x), d.CreateBuffer(scale), d.CreateBuffer(zero)
    bo = d.CreateBufferOf(og.ElementType.UInt8, MAX4)
    run(d, lambda e: k.EncodeQuantize(e, bx, 0, [MAX4], 0, False, bs, 0, bzp, 0, bo, 0))
    kernel = d.LastKernel
    got = bo.Read()
    del bo, bx
    want = oracle.quantize(x, scale, False, zero=zero[:1])
    bad = _same(got, want)
    say(f"ROW quantize at count {MAX4} | {kernel} | mismatching bytes {bad}")
    assert bad == 0


def test_product_at_the_largest_output():
    # C of 32768 x 65520 int32 (2,146,959,360 elements, 8 GiB), just under the boundary's limit of 2^31 elements, so
    # output indices reach the top of the range. A[m][k] = m % 251 (uint8) under a zero point of 7, B[k][n] = n % 13 - 6
    # (int8): C[m][n] = K (m % 251 - 7)(n % 13 - 6), a closed form checked for every element in chunks of rows.
    d = device()
    m, n, k = 32768, 65520, 64
    gemm = og.Int8Gemm(d)
    say(f"product at the largest output {m}x{n}x{k}")
    a = np.repeat((np.arange(m) % 251).astype(np.uint8), k)
    b = np.tile(((np.arange(n) % 13) - 6).astype(np.int8), k)
    ba, bb = d.CreateBuffer(a), d.CreateBuffer(b)
    bz = d.CreateBuffer(np.array([7, 0, 0, 0], np.uint8))
    bc = d.CreateBufferOf(og.ElementType.Int32, m * n)
    run(d, lambda e: gemm.EncodeInt32(e, og.Int8GemmProblem(m, n, k), ba, bb, bc, og.Int8Operand(bz, 0), None))
    kernel = d.LastKernel
    got = bc.Read()
    del bc
    col = (np.arange(n) % 13 - 6).astype(np.int64)
    bad = 0
    for r0 in range(0, m, 1024):
        row = (np.arange(r0, r0 + 1024) % 251 - 7).astype(np.int64)
        want = (k * row[:, None] * col[None, :]).astype(np.int32)
        bad += int(np.count_nonzero(got[r0 * n:(r0 + 1024) * n].reshape(1024, n) != want))
    say(f"ROW product at the largest output | {kernel} | mismatching elements {bad}")
    assert bad == 0


def test_gather_from_a_table_past_4_gib():
    # An int32 table of 524287 rows x 4096 (8 GiB, just under 2^31 elements): its last rows start past 2^32 bytes.
    # Element j of row r holds r * 4096 + j, so each gathered row names the row it came from; negative indices count
    # from the end.
    d = device()
    k = og.GatherKernels(d)
    rows, inner = 524287, 4096
    say(f"gather from a table of {rows} x {inner} int32")
    data = np.arange(rows * inner, dtype=np.int32)
    idx = np.array([rows - 1, -1, 0, 262144, rows - 2, -rows, 524000, 7], np.int64)
    bd, bi = d.CreateBuffer(data), d.CreateBuffer(idx)
    del data
    bo = d.CreateBuffer(np.full(idx.size * inner, -999, np.int32))
    status = og.GpuIndexStatus(d)
    run(d, lambda e: k.EncodeGather(e, bd, 0, [rows, inner], 0, bi, 0, int(idx.size), bo, 0, status))
    status.ThrowIfFailed()
    kernel = d.LastKernel
    got = bo.Read().reshape(idx.size, inner)
    row = np.where(idx < 0, idx + rows, idx)
    want = (row[:, None] * inner + np.arange(inner)[None, :]).astype(np.int32)
    bad = int(np.count_nonzero(got != want))
    say(f"ROW gather past 4 GiB | {kernel} | mismatching elements {bad}")
    assert bad == 0
