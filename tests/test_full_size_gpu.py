"""The BASELINE configurations' products at their full sizes, on the GPU, checked through properties that hold at any
size plus sampled rows from the oracle:

  - column sums: sum_m C[m, n] = sum_k u[k] (B[k, n] - zb[n]) with u[k] = sum_m (A[m, k] - za[m]);
  - row sums:    sum_n C[m, n] = sum_k (A[m, k] - za[m]) w[k] with w[k] = sum_n (B[k, n] - zb[n]);

both in int64 and compared modulo 2^32 (the sums wrap). Every element of C enters both, so a wrong element, row,
column, tile or zero-point term shows, at the cost of two matrix-vector products on the host.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import onegpu_hip as og
from gpu_rig import device, run, say


def _wrap32(v: np.ndarray) -> np.ndarray:
    return (np.asarray(v, np.int64) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def _checks(a, b, za, zb, c, a_signed, b_signed, trans_b=False):
    """Mismatches of C's column and row sums against the two matrix-vector products (A [M, K], B [K, N] or [N, K])."""
    av = a.view(np.int8).astype(np.int64) if a_signed else a.astype(np.int64)
    bv = b.view(np.int8).astype(np.int64) if b_signed else b.astype(np.int64)
    if trans_b:
        bv = bv.T
    zav = np.zeros(av.shape[0], np.int64) if za is None else (za.view(np.int8) if a_signed else za).astype(np.int64)
    zbv = np.zeros(bv.shape[1], np.int64) if zb is None else (zb.view(np.int8) if b_signed else zb).astype(np.int64)
    if zav.size == 1:
        zav = np.full(av.shape[0], zav[0], np.int64)
    if zbv.size == 1:
        zbv = np.full(bv.shape[1], zbv[0], np.int64)
    u = av.sum(axis=0) - zav.sum()                      # [K]
    w = bv.sum(axis=1) - zbv.sum()                      # [K]
    col_want = _wrap32(u @ bv - u.sum() * zbv)          # sum_k u[k] (B[k, n] - zb[n])
    row_want = _wrap32(av @ w - zav * w.sum())          # sum_k (A[m, k] - za[m]) w[k]
    c64 = c.astype(np.int64)
    col_got = _wrap32(c64.sum(axis=0))
    row_got = _wrap32(c64.sum(axis=1))
    return int(np.count_nonzero(col_got != col_want)), int(np.count_nonzero(row_got != row_want))


def _product(d, m, n, k, a_signed, b_signed, za_per_row, zb_per_col, seed, trans_b=False, batch=1):
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, (batch, m, k), dtype=np.uint8)
    b = rng.integers(0, 256, (batch, n, k) if trans_b else (batch, k, n), dtype=np.uint8)
    za = rng.integers(0, 256, m if za_per_row else 1, dtype=np.uint8)
    zb = rng.integers(0, 256, n if zb_per_col else 1, dtype=np.uint8)
    ba = d.CreateBuffer(a.ravel().view(np.int8) if a_signed else a.ravel())
    bb = d.CreateBuffer(b.ravel().view(np.int8) if b_signed else b.ravel())
    bza = d.CreateBuffer(za.view(np.int8) if a_signed else za)
    bzb = d.CreateBuffer(zb.view(np.int8) if b_signed else zb)
    bc = d.CreateBufferOf(og.ElementType.Int32, batch * m * n)
    p = og.Int8GemmProblem(m, n, k)
    p.TransposeB = trans_b
    p.Batch = batch
    p.StrideA, p.StrideB = m * k, n * k
    gemm = og.Int8Gemm(d)
    run(d, lambda e: gemm.EncodeInt32(e, p, ba, bb, bc, og.Int8Operand(bza, 0, za_per_row),
                                      og.Int8Operand(bzb, 0, zb_per_col)))
    return a, b, za, zb, bc.Read().reshape(batch, m, n), d.LastKernel


@pytest.mark.parametrize("m, n, k, a_signed, b_signed, za_row, zb_col, trans_b", [
    (5, 7, 9, False, True, True, False, False), (6, 4, 33, True, False, True, True, True),
    (16, 20, 64, False, False, False, True, False), (3, 3, 3, True, True, False, False, True)])
def test_checksums_equal_the_oracle_and_catch_a_wrong_element(m, n, k, a_signed, b_signed, za_row, zb_col, trans_b):
    # The host side of the full-size checks, on the CPU: the two sums agree with the oracle's whole product, and one
    # element changed by 1 shows in both.
    rng = np.random.default_rng(m * n + k)
    a = rng.integers(0, 256, (m, k), dtype=np.uint8)
    b = rng.integers(0, 256, (n, k) if trans_b else (k, n), dtype=np.uint8)
    za = rng.integers(0, 256, m if za_row else 1, dtype=np.uint8)
    zb = rng.integers(0, 256, n if zb_col else 1, dtype=np.uint8)
    g = oracle.Gemm(m, n, k, TransposeB=int(trans_b))
    c = oracle.int8_gemm(g, a.ravel(), a_signed, b.ravel(), b_signed, (za, za_row, 0), (zb, zb_col, 0)).reshape(m, n)
    assert _checks(a, b, za, zb, c, a_signed, b_signed, trans_b) == (0, 0)
    c2 = c.copy()
    c2[m // 2, n // 2] += 1
    assert _checks(a, b, za, zb, c2, a_signed, b_signed, trans_b) == (1, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("name, m, n, k, a_signed, b_signed, za_row, zb_col, trans_b, batch, want_kernel", [
    ("configuration 4 (4096^3, u8 A, per-row zero point, B K x N)", 4096, 4096, 4096, False, True, True, False, False,
     1, "mfma-i8-direct256x256x64"),
    ("4096^3 with both zero points per row / column, u8 B stored N x K", 4096, 4096, 4096, True, False, True, True,
     True, 1, "mfma-i8-direct256x256x64"),
    ("configuration 2's product (1024 x 3072 x 768)", 1024, 3072, 768, False, True, False, False, False, 1,
     "mfma-i8-direct128x128x64"),
    # 3 x 2 x 16 tiles of 256 leave most CUs idle, so the 128 tile takes it (batched).
    ("configuration 5's per-batch shape, 3 batches (512 x 4096 x 4096)", 512, 4096, 4096, False, True, False, False,
     False, 3, "mfma-i8-direct128x128x64"),
])
def test_full_size_products(name, m, n, k, a_signed, b_signed, za_row, zb_col, trans_b, batch, want_kernel):
    d = device()
    say(f"full size: {name}")
    a, b, za, zb, c, kernel = _product(d, m, n, k, a_signed, b_signed, za_row, zb_col, 40 + m % 7, trans_b, batch)
    assert kernel == want_kernel, kernel
    bad_cols = bad_rows = bad_sampled = 0
    rows = np.array([0, 1, m // 3, m - 1])
    for bi in range(batch):
        bc, br = _checks(a[bi], b[bi], za, zb, c[bi], a_signed, b_signed, trans_b)
        bad_cols += bc
        bad_rows += br
        g = oracle.Gemm(m, n, k, TransposeB=int(trans_b))
        want = oracle.int8_gemm_rows(g, a[bi].ravel(), a_signed, b[bi].ravel(), b_signed, rows,
                                     (za, za_row, 0), (zb, zb_col, 0))
        bad_sampled += int(np.count_nonzero(c[bi][rows] != want))
    say(f"ROW full size | {name} | {kernel} | column sums off {bad_cols}, row sums off {bad_rows}, "
        f"sampled rows off {bad_sampled}")
    assert bad_cols == 0 and bad_rows == 0 and bad_sampled == 0


@pytest.mark.gpu
def test_configuration_5_at_full_size():
    # Configuration 5 as the bench runs it: 32 batches of 512 x 4096 x 4096 with 32 distinct weight matrices, the
    # activations one DynamicQuantizeLinear of N(0, 1) over all 67 M elements (uint8 with its scalar zero point), int8
    # weights with no zero point. The 32 batches fill the chip with 256 x 256 tiles. Every batch is checked through
    # its column and row sums and four oracle rows.
    d = device()
    batch, m, n, k = 32, 512, 4096, 4096
    rng = np.random.default_rng(55)
    say("full size: configuration 5 (32 x 512 x 4096 x 4096, distinct B, DQ'd activations)")
    x = rng.standard_normal(batch * m * k, dtype=np.float32)
    a, _, zp = oracle.dynamic_quantize(x)
    del x
    za = np.array([zp], np.uint8)
    b = rng.integers(-127, 128, (batch, k, n), dtype=np.int8)
    ba, bb, bza = d.CreateBuffer(a), d.CreateBuffer(b.ravel()), d.CreateBuffer(za)
    bc = d.CreateBufferOf(og.ElementType.Int32, batch * m * n)
    p = og.Int8GemmProblem(m, n, k)
    p.Batch = batch
    p.StrideA, p.StrideB = m * k, k * n
    gemm = og.Int8Gemm(d)
    run(d, lambda e: gemm.EncodeInt32(e, p, ba, bb, bc, og.Int8Operand(bza, 0)))
    kernel = d.LastKernel
    assert kernel == "mfma-i8-direct256x256x64", kernel
    c = bc.Read().reshape(batch, m, n)
    a = a.reshape(batch, m, k)
    bad_cols = bad_rows = bad_sampled = 0
    rows = np.array([0, 1, 171, m - 1])
    g = oracle.Gemm(m, n, k)
    for bi in range(batch):
        bcols, brows = _checks(a[bi], b[bi].view(np.uint8), za, None, c[bi], False, True)
        bad_cols += bcols
        bad_rows += brows
        want = oracle.int8_gemm_rows(g, a[bi].ravel(), False, b[bi].ravel().view(np.uint8), True, rows, (za, False, 0))
        bad_sampled += int(np.count_nonzero(c[bi][rows] != want))
    say(f"ROW full size | configuration 5 | {kernel} | zero point {zp} | column sums off {bad_cols}, row sums off "
        f"{bad_rows}, sampled rows off {bad_sampled}")
    assert bad_cols == 0 and bad_rows == 0 and bad_sampled == 0
