"""GatherKernels.EncodeGather on the GPU against the oracle's index map, bit for bit (GatherTests.cs): every payload
width with int32 and int64 indices, negative and invalid indices with the status word, odd offsets, and the int8
embedding lookups that feed the first int8 product."""
from __future__ import annotations

import numpy as np
import pytest

import cases
import oracle
import onegpu_hip as og
from gpu_rig import device, run, say

pytestmark = pytest.mark.gpu

OFF_DATA, OFF_IDX, OFF_OUT = 1, 2, 3   # GatherTests.cs:6

PAYLOADS = [(np.float32, np.int32), (np.float32, np.int64), (np.float16, np.int32), (np.float16, np.int64),
            (np.int32, np.int32), (np.uint32, np.int64), (np.int64, np.int32), (np.int64, np.int64),
            (np.uint8, np.int32), (np.int8, np.int64)]   # GatherTests.cs:86-96


def _padded(dtype, n: int) -> int:
    """IndexRig.Padded (IndexRig.cs:13-15): halves and bytes end on a 32-bit word."""
    size = np.dtype(dtype).itemsize
    return og.padded_half_length(n) if size == 2 else og.padded_bool_length(max(n, 1)) if size == 1 else n


def _sentinel(dtype):
    """IndexRig.Make<T>(-999), the value the tests fill the output with (GatherTests.cs:36-38)."""
    return cases.index_rig_make(dtype, np.array([-999 & 0xFFFFFFFF]))[0]


def _gather_case(d, k, dtype, itype, shape, axis, count, seed, idx_values=None, with_status=True):
    """GatherCase (GatherTests.cs:8-68): returns (wrong elements, status position or None, kernel)."""
    n = int(np.prod(shape))
    n_axis = shape[axis]
    data = cases.index_rig_fill(dtype, _padded(dtype, n + OFF_DATA), seed)
    if idx_values is None:
        idx_values = cases.index_rig_random_index(np.arange(count), n_axis, seed)
    idx = np.zeros(count + OFF_IDX, itype)
    idx[OFF_IDX:] = np.asarray(idx_values).astype(itype)
    want, want_bad = oracle.gather(data[OFF_DATA:OFF_DATA + n], shape, axis, idx_values, itype == np.int64)
    total = want.size
    sentinel = _sentinel(dtype)
    out = np.full(_padded(dtype, total + OFF_OUT + 2), sentinel, dtype)
    bd, bi, bo = d.CreateBuffer(data), d.CreateBuffer(idx if idx.size else np.zeros(1, itype)), d.CreateBuffer(out)
    status = og.GpuIndexStatus(d) if with_status else None
    run(d, lambda e: k.EncodeGather(e, bd, OFF_DATA, list(shape), axis, bi, OFF_IDX, count, bo, OFF_OUT, status))
    pos = None
    if status is not None:
        try:
            status.ThrowIfFailed()
        except og.GpuKernelIndexException as ex:
            assert ex.Operation == "Gather"
            pos = ex.Position
    got = bo.Read()
    wv, gv = want.view(np.uint8).reshape(total, -1), got[OFF_OUT:OFF_OUT + total].view(np.uint8).reshape(total, -1)
    bad = int(np.count_nonzero((gv != wv).any(axis=1)))
    sv = np.array([sentinel], dtype).view(np.uint8)
    edges = np.concatenate([got[:OFF_OUT], got[OFF_OUT + total:]]).view(np.uint8).reshape(-1, sv.size)
    bad += int(np.count_nonzero((edges != sv).any(axis=1)))
    if with_status:
        assert pos == want_bad, (pos, want_bad)
    return bad, pos, d.LastKernel


def test_onnx_specification_examples():
    # The ONNX Gather specification's two examples as known answers, with int8 payloads (the values times 10): axis 0
    # with indices [[0, 1], [1, 2]], and axis 1 with indices [[0, 2]].
    d = device()
    k = og.GatherKernels(d)
    d0 = np.array([10, 12, 23, 34, 45, 57, 0, 0], np.int8)           # [[1.0, 1.2], [2.3, 3.4], [4.5, 5.7]] x 10
    out = d.CreateBufferOf(og.ElementType.Int8, 8)
    i0 = d.CreateBuffer(np.array([0, 1, 1, 2], np.int32))
    run(d, lambda e: k.EncodeGather(e, d.CreateBuffer(d0), 0, [3, 2], 0, i0, 0, 4, out, 0))
    assert out.Read()[:8].tolist() == [10, 12, 23, 34, 23, 34, 45, 57]
    d1 = np.array([10, 12, 19, 23, 34, 39, 45, 57, 59, 0, 0, 0], np.int8)   # the 3 x 3 example x 10
    i1 = d.CreateBuffer(np.array([0, 2], np.int64))
    run(d, lambda e: k.EncodeGather(e, d.CreateBuffer(d1), 0, [3, 3], 1, i1, 0, 2, out, 0))
    assert out.Read()[:6].tolist() == [10, 19, 23, 39, 45, 59]


def test_gather_is_exact():
    # GatherIsExact (GatherTests.cs:73-100): 12 shapes x 10 payload / index types, negative indices, odd offsets.
    d = device()
    k = og.GatherKernels(d)
    bad, seed, kernels = 0, 1, set()
    for shape, axis, count in cases.GATHER_CASES:
        for dtype, itype in PAYLOADS:
            say(f"gather {shape} axis {axis} count {count} {np.dtype(dtype).name}/{np.dtype(itype).name}")
            b, _, kern = _gather_case(d, k, dtype, itype, shape, axis, count, seed)
            bad += b
            kernels.add(kern)
            seed += 1
    say(f"ROW gather: {len(cases.GATHER_CASES) * len(PAYLOADS)} cases, wrong elements {bad}, kernels {sorted(kernels)}")
    assert bad == 0


@pytest.mark.parametrize("dtype, itype", [(np.uint8, np.int32), (np.int8, np.int64), (np.float32, np.int64)])
def test_invalid_indices_give_zeros_and_the_smallest_position(dtype, itype):
    # An index outside its axis reads nothing and the status names the smallest offending position (Gather.hlsl:35-40;
    # GatherKernels.cs:16-19); without a status the zeros come silently.
    d = device()
    k = og.GatherKernels(d)
    shape, axis = [6, 40], 0
    vals = [3, -6, 6, 1, -7, 2, 5, 100, -1]
    if itype == np.int64:
        vals += [1 << 33, -(1 << 40)]   # do not fit an int32
    b, pos, _ = _gather_case(d, k, dtype, itype, shape, axis, len(vals), 77, idx_values=vals)
    assert b == 0 and pos == 2
    b, pos, _ = _gather_case(d, k, dtype, itype, shape, axis, len(vals), 78, idx_values=vals, with_status=False)
    assert b == 0 and pos is None


def test_aligned_rows_take_the_vector_path():
    # 16-byte aligned tensors and rows copy 16 bytes at a time; odd offsets fall back to bytes. Both exact.
    d = device()
    k = og.GatherKernels(d)
    vocab, hidden, count = 1000, 768, 333
    table = cases.index_rig_fill(np.int8, vocab * hidden + 64, 9)
    ids = cases.index_rig_random_index(np.arange(count), vocab, 9).astype(np.int32)
    want, bad_pos = oracle.gather(table[:vocab * hidden], [vocab, hidden], 0, ids)
    for off_data, off_out, want_kernel in ((0, 0, "gather-rows16"), (16, 32, "gather-rows16"), (1, 3, "gather-bytes")):
        bt, bi = d.CreateBuffer(table), d.CreateBuffer(ids)
        bo = d.CreateBufferOf(og.ElementType.Int8, og.padded_bool_length(count * hidden + off_out))
        run(d, lambda e: k.EncodeGather(e, bt, off_data, [vocab, hidden], 0, bi, 0, count, bo, off_out))
        w = oracle.gather(table[off_data:off_data + vocab * hidden], [vocab, hidden], 0, ids)[0]
        got = bo.Read()[off_out:off_out + count * hidden]
        assert d.LastKernel == want_kernel
        assert np.array_equal(got, w), (off_data, off_out)
    assert bad_pos is None and want.size == count * hidden


@pytest.mark.parametrize("vocab, hidden", [(30522, 384), (30522, 768), (250002, 768)])
def test_int8_embedding_lookups_are_exact(vocab, hidden):
    # EmbeddingLookupsAreExact (GatherTests.cs:104-160) with int8 tables: the vocabularies and widths of the reference
    # models, batch 1 and 8 of 512 token ids.
    d = device()
    k = og.GatherKernels(d)
    rng = np.random.default_rng(vocab + hidden)
    table = rng.integers(-128, 128, vocab * hidden, dtype=np.int8)
    bt = d.CreateBuffer(table)
    for batch in (1, 8):
        ids = rng.integers(-vocab, vocab, batch * 512).astype(np.int64)
        bi = d.CreateBuffer(ids)
        bo = d.CreateBufferOf(og.ElementType.Int8, batch * 512 * hidden)
        status = og.GpuIndexStatus(d)
        run(d, lambda e: k.EncodeGather(e, bt, 0, [vocab, hidden], 0, bi, 0, batch * 512, bo, 0, status))
        status.ThrowIfFailed()
        want = table.reshape(vocab, hidden)[np.where(ids < 0, ids + vocab, ids)].ravel()
        got = bo.Read()[:want.size]
        bad = int(np.count_nonzero(got != want))
        say(f"ROW int8 embedding {vocab} x {hidden}, {batch} x 512 tokens ({d.LastKernel}): wrong bytes {bad}")
        assert bad == 0


def test_seeded_random_gathers_are_exact():
    # Seeded random ranks, extents, axes, index counts, payload widths and index types; indices drawn from the whole
    # valid range with negatives, and in every third case a few out of range (zero rows and the smallest position).
    # GatherCase's offsets (GatherTests.cs:6) leave the rows unaligned, so these take the byte copies; the 16-byte
    # copies have the aligned and embedding tests above.
    d = device()
    k = og.GatherKernels(d)
    rng = np.random.default_rng(99)
    kernels = set()
    for i in range(40):
        rank = int(rng.integers(1, 5))
        shape = [int(rng.integers(1, 9)) for _ in range(rank)]
        if rng.integers(0, 2):
            shape[-1] = int(rng.choice([16, 48, 64, 384]))   # rows that can take the 16-byte copies
        axis = int(rng.integers(0, rank))
        count = int(rng.integers(1, 40))
        dtype, itype = PAYLOADS[int(rng.integers(0, len(PAYLOADS)))]
        n_axis = shape[axis]
        vals = rng.integers(-n_axis, n_axis, count)
        if i % 3 == 2 and count > 0:
            for j in rng.integers(0, count, 2):
                vals[j] = n_axis + int(rng.integers(0, 5)) if rng.integers(0, 2) else -n_axis - 1 - int(rng.integers(0, 5))
        say(f"gather random {i}: shape {shape} axis {axis} count {count} {np.dtype(dtype).name}/{np.dtype(itype).name}")
        bad, _, kern = _gather_case(d, k, dtype, itype, shape, axis, count, 700 + i, idx_values=vals.tolist())
        kernels.add(kern)
        assert bad == 0, f"case {i}: {bad} wrong"
    say(f"ROW seeded random gathers: 40 cases exact; kernels {sorted(kernels)}")
