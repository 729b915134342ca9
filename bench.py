"""Benchmark of the MI355X int8 quantized-matmul path on BASELINE.json's configurations.

One JSON line on stdout. `value` is the headline metric's first half: int8 TOPS of MatMulInteger at M = N = K = 4096
(configuration 4: uint8 A with a per-row zero point, int8 B stored K x N, int32 out), whole-job throughput over
exactly --steps products with inputs resident in HBM, bracketed by device synchronisation. The second half, GB/s of
the M = 1, K = 4096, N = 11008 decode GEMV (configuration 3, weights rotated over 9 copies so the 45 MB matrix cannot
sit in the 256 MiB Infinity Cache), is in `gemv_m1`; the other configurations are in `configs`.

`roofline` is for the dominant kernel (the 4096^3 MFMA product): algorithmic ops 2*M*N*K per launch over the average
launch duration measured with HIP events on the stream the kernel runs on. `cpu_baseline` times the oracle (a C
restatement of the reference's CPU reference, multithreaded) on a bounded sample of rows of the same product.
Every configuration's output is checked against the oracle (sampled rows) before it is reported.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "onegpu-csharp_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

import onegpu_hip as og  # noqa: E402

PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA (5.0 POPS)
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E (8 TB/s)
METRIC = "int8 TOPS (% of MFMA peak) at 4096³; GB/s (% of HBM) at M=1 GEMV"


# ------------------------------------------------------------------ C ABI utilities (synthetic data on the device)

class _Buf(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_uint64)]


_L = None


def _abi():
    global _L
    if _L is None:
        _L = ctypes.CDLL(og.LIB_PATH)
        _L.og_util_synth.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32, _Buf,
                                     ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double]
        _L.og_util_col_absmax_scale.argtypes = [ctypes.c_void_p, _Buf, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
                                                _Buf]
        _L.og_util_scale_product.argtypes = [ctypes.c_void_p, _Buf, _Buf, ctypes.c_uint32, _Buf]
        _L.og_timing_region_begin.argtypes = [ctypes.c_void_p]
        _L.og_timing_region_end.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]
        _L.og_last_error.argtypes = [ctypes.c_void_p]
        _L.og_last_error.restype = ctypes.c_char_p
    return _L


def _b(buf):
    return _Buf(buf.DevicePointer, buf.Size)


def _ok(st, d):
    if st != 0:
        raise RuntimeError(f"C ABI status {st}: {_abi().og_last_error(d.Context).decode()}")


def synth(d, etype, n, seed, tensor, lo, hi, kind):
    b = d.CreateBufferOf(etype, n)
    _ok(_abi().og_util_synth(d.Context, kind, seed, tensor, _b(b), 0, n, lo, hi), d)
    return b


def sym_weights(d, k, n, seed, tensor, q=None, q_off=0, scale=None, scale_off=0):
    """N(0, 0.02) float weights [K, N] -> per-column scale max|w| / 127 -> QuantizeLinear to int8 (axis 1), into new
    buffers or at element offsets of the given ones (a batch of weight matrices and their scale vectors)."""
    w = synth(d, og.ElementType.Float32, k * n, seed, tensor, 0.0, 0.02, 2)
    scale = d.CreateBufferOf(og.ElementType.Float32, n) if scale is None else scale
    q = d.CreateBufferOf(og.ElementType.Int8, k * n) if q is None else q
    _ok(_abi().og_util_col_absmax_scale(d.Context, _b(w), k, n, 127.0,
                                        _Buf(scale.DevicePointer + 4 * scale_off, 4 * n)), d)
    e = d.BeginCommands()
    og.DequantizeKernels(d).EncodeQuantize(e, w, 0, [k, n], 1, True, scale, scale_off, None, 0, q, q_off)
    d.Submit(e)
    d.WaitIdle()
    w.Dispose()
    return q, scale


# ------------------------------------------------------------------ timing

def timed(d, record, steps, warmup):
    """Runs `record(encoder, i)` warmup times untimed; then `steps` times back to back in one encoder, bracketed by
    device synchronisation for the wall time and by one HIP event pair on the library's stream for the device time;
    then `steps` more times with an event pair around every dispatch, for the kernel names and a per-dispatch split.
    Returns (wall seconds, event seconds of the back-to-back steps, [(ms, kernel)] per dispatch of the second run)."""
    L = _abi()
    for i in range(warmup):
        e = d.BeginCommands()
        record(e, i)
        d.Submit(e)
    d.WaitIdle()
    e = d.BeginCommands()
    for i in range(steps):
        record(e, warmup + i)
    region = ctypes.c_float(0.0)
    t0 = time.perf_counter()
    _ok(L.og_timing_region_begin(d.Context), d)
    d.Submit(e)
    _ok(L.og_timing_region_end(d.Context, ctypes.byref(region)), d)
    d.WaitIdle()
    wall = time.perf_counter() - t0
    e = d.BeginCommands()
    e.BeginPassTiming(steps)
    for i in range(steps):
        record(e, warmup + steps + i)
    e.EndPassTiming()
    d.Submit(e)
    d.WaitIdle()
    return wall, region.value * 1e-3, d.ReadPassTimes()


def kernel_stats(times, name_prefix=None):
    ms = [t for t, k in times if name_prefix is None or k.startswith(name_prefix)]
    return statistics.mean(ms), statistics.median(ms), (times[0][1] if times else "")


def per_kernel_us(times):
    """{kernel: {"mean_us", "median_us", "n"}} over the individually timed dispatches (one HIP event pair around each,
    so a short kernel's figure includes the dispatch's own start-up of about 1-2 us)."""
    per = {}
    for t, k in times:
        per.setdefault(k, []).append(t * 1e3)
    return {k: {"mean_us": statistics.mean(v), "median_us": statistics.median(v), "n": len(v)} for k, v in per.items()}


# ------------------------------------------------------------------ configurations

def c4_square(d, steps, warmup, check=True, constant=False, trans_b=False, plain=False):
    """Configuration 4: 4096^3, A uint8 U{0..255} with per-row a_zp U{100..156}, B int8 U{-127..127}, int32 out.
    constant=True fills A, B and the zero points with one value each instead (the same work on operands that do not
    toggle: the matrix cores then draw less power and the chip holds a higher clock); trans_b=True reads the same bytes
    of B as stored N x K (a different product, the same work: the layout's cost alone); plain=True reads A as int8
    with no zero point (int8 x int8 as torch._int_mm computes it, no byte sums or flips)."""
    M = N = K = 4096
    a = synth(d, og.ElementType.Int8 if plain else og.ElementType.UInt8, M * K, 4, 0,
              *((0x37, 0x37) if constant else ((-128, 127) if plain else (0, 255))), 0)
    za = synth(d, og.ElementType.UInt8, M, 4, 1, *((128, 128) if constant else (100, 156)), 0)
    b = synth(d, og.ElementType.Int8, K * N, 4, 2, *((-13, -13) if constant else (-127, 127)), 0)
    c = d.CreateBufferOf(og.ElementType.Int32, M * N)
    gemm = og.Int8Gemm(d)
    p = og.Int8GemmProblem(M, N, K)
    p.TransposeB = trans_b
    zpa = None if plain else og.Int8Operand(za, 0, True)
    wall, region, times = timed(d, lambda e, i: gemm.EncodeInt32(e, p, a, b, c, zpa), steps, warmup)
    pair_ms, pair_med_ms, kname = kernel_stats(times)
    res = {"ops": 2.0 * M * N * K, "wall_s": wall, "kernel_mean_ms": region / steps * 1e3,
           "event_pair_mean_ms": pair_ms, "event_pair_median_ms": pair_med_ms, "kernel": kname,
           "bytes": M * K + K * N + M + 4 * M * N}
    if check:
        import oracle
        rows = np.array([0, 1, 777, 2048, 4095])
        A, B, Z = a.Read(), b.Read(), za.Read()
        want = oracle.int8_gemm_rows(oracle.Gemm(M, N, K), A, False, B.view(np.uint8), True, rows, (Z, True, 0))
        got = c.Read().reshape(M, N)[rows]
        res["check"] = "bit-exact on sampled rows" if np.array_equal(got, want) else "MISMATCH"
        res["host_operands"] = (A, B, Z)
    return res


def c3_gemv(d, m, steps, warmup, copies=9, check=True, n=11008, opts=None):
    """Configuration 3: A = DynamicQuantizeLinear(N(0,1) [m x 4096]); B int8 [4096 x n] symmetric per column
    (N(0, 0.02)); MatMulIntegerToFloat with scale = actScale * wScale[n]. `copies` weight matrices rotate. n = 1376 is
    one GPU's share of an 8-way column split of configuration 3's weights. `opts`: Int8GemmOptions fields (the
    two-launch few-rows form: FewRowsOneLaunch=False)."""
    K, N = 4096, n
    x = synth(d, og.ElementType.Float32, m * K, 3, 10, 0.0, 1.0, 2)
    ya = d.CreateBufferOf(og.ElementType.UInt8, m * K)
    s = d.CreateBufferOf(og.ElementType.Float32, 1)
    z = d.CreateBufferOf(og.ElementType.UInt8, 4)
    e = d.BeginCommands()
    og.DynamicQuantizeKernels(d).Encode(e, x, 0, m * K, ya, 0, s, 0, z, 0)
    d.Submit(e)
    ws = []
    for cidx in range(copies):
        q, wscale = sym_weights(d, K, N, 3, 20 + cidx)
        sc = d.CreateBufferOf(og.ElementType.Float32, N)
        _ok(_abi().og_util_scale_product(d.Context, _b(s), _b(wscale), N, _b(sc)), d)
        ws.append((q, sc))
    c = d.CreateBufferOf(og.ElementType.Float32, m * N)
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(**(opts or {})))
    p = og.Int8GemmProblem(m, N, K)
    zpa = og.Int8Operand(z, 0)
    wall, region, times = timed(d, lambda e, i: gemm.EncodeFloat(e, p, ya, ws[i % copies][0], c,
                                                                  og.Int8Operand(ws[i % copies][1], 0, True), zpa),
                                steps, warmup)
    # A few-rows product may be split into two dispatches (partial sums, then their sum); its time is both.
    n_disp = len(times) // steps
    step_ms = [sum(times[i * n_disp + j][0] for j in range(n_disp)) for i in range(steps)]
    bytes_ = K * N + m * K + 4 * m * N + 4 * N + 4 + 1
    res = {"m": m, "ops": 2.0 * m * N * K, "bytes": bytes_, "wall_s": wall, "step_mean_ms": region / steps * 1e3,
           "event_pair_step_mean_ms": statistics.mean(step_ms), "event_pair_step_median_ms": statistics.median(step_ms),
           "kernels": [k for _, k in times[:n_disp]],
           "dispatch_mean_ms": [statistics.mean(times[i * n_disp + j][0] for i in range(steps)) for j in range(n_disp)]}
    if check:
        import oracle
        last = (warmup + 2 * steps - 1) % copies   # the weight copy of the last launch timed() recorded
        q, sc = ws[last]
        Y, Z, Q, SC = ya.Read(), int(z.Read()[0]), q.Read(), sc.Read()
        sums = oracle.int8_gemm(oracle.Gemm(m, N, K), Y, False, Q.view(np.uint8), True, (np.array([Z], np.uint8), False, 0))
        want = oracle.float_epilogue(sums, N, SC, True)
        got = c.Read()
        res["check"] = "bit-exact" if np.array_equal(got.view(np.uint32), want.view(np.uint32)) else "MISMATCH"
    return res


def c2_bert_ffn(d, steps, warmup, check=True, fused_scale=True):
    """Configuration 2: DQ [1024 x 768] N(0,1) -> MatMulIntegerToFloat with W [768 x 3072] symmetric per column.
    Each step is the whole layer on one stream: DynamicQuantizeLinear (two passes), then the product with the column
    scale fl(actScale * wScale[n]) made in its epilogue (fused_scale), or, as the reference chains it, the elementwise
    scale product as a dispatch of its own followed by EncodeFloat with that vector."""
    M, K, N = 1024, 768, 3072
    x = synth(d, og.ElementType.Float32, M * K, 2, 30, 0.0, 1.0, 2)
    q, wscale = sym_weights(d, K, N, 2, 31)
    ya = d.CreateBufferOf(og.ElementType.UInt8, M * K)
    s = d.CreateBufferOf(og.ElementType.Float32, 1)
    z = d.CreateBufferOf(og.ElementType.UInt8, 4)
    sc = d.CreateBufferOf(og.ElementType.Float32, N)
    c = d.CreateBufferOf(og.ElementType.Float32, M * N)
    dq, gemm = og.DynamicQuantizeKernels(d), og.Int8Gemm(d)
    p = og.Int8GemmProblem(M, N, K)

    def step(e, i):
        dq.Encode(e, x, 0, M * K, ya, 0, s, 0, z, 0)
        if fused_scale:
            gemm.EncodeFloatScaled(e, p, ya, q, c, og.Int8Operand(s, 0), og.Int8Operand(wscale, 0, True),
                                   og.Int8Operand(z, 0))
        else:
            e.RecordScaleProduct(s, wscale, N, sc)
            gemm.EncodeFloat(e, p, ya, q, c, og.Int8Operand(sc, 0, True), og.Int8Operand(z, 0))

    wall, region, times = timed(d, step, steps, warmup)
    per = per_kernel_us(times)
    # Bytes each dispatch moves at least once: the range pass reads x; the quantize pass reads x and writes y (the
    # per-workgroup ranges are a few KB); the product reads A, B and the scales and writes the float32 output.
    kbytes = {"dq-minmax": 4 * M * K, "dq-quantize": 4 * M * K + M * K + 5, "scale-product": 8 * N + 4}
    for k in per:
        per[k]["bytes"] = kbytes.get(k, M * K + K * N + 4 * M * N + 4 * N + 5)
        per[k]["gbs_median"] = per[k]["bytes"] / (per[k]["median_us"] * 1e-6) / 1e9
        per[k]["hbm_frac_median"] = per[k]["gbs_median"] / PEAK_HBM_GBS
    res = {"ops": 2.0 * M * N * K, "wall_s": wall, "chain_mean_ms": region / steps * 1e3, "per_kernel": per,
           "chain_bytes": 4 * M * K + K * N + 4 * N + 4 * M * N}
    if check:
        import oracle
        Y, Z, Q, WS = ya.Read(), int(z.Read()[0]), q.Read(), wscale.Read()
        wy, ws_, wz = oracle.dynamic_quantize(x.Read())
        ok_dq = np.array_equal(Y, wy) and wz == Z and np.float32(s.Read()[0]) == np.float32(ws_)
        SC = (np.float32(ws_) * WS.astype(np.float32)).astype(np.float32)
        rows = np.array([0, 5, 511, 1023])
        sums = oracle.int8_gemm_rows(oracle.Gemm(M, N, K), Y, False, Q.view(np.uint8), True, rows, (np.array([Z], np.uint8), False, 0))
        want = oracle.float_epilogue(sums.ravel(), N, SC, True).reshape(len(rows), N)
        got = c.Read().reshape(M, N)[rows]
        res["check"] = "bit-exact" if ok_dq and np.array_equal(got.view(np.uint32), want.view(np.uint32)) else "MISMATCH"
    return res


def c2_two_layer(d, steps, warmup, ranged=True, check=True):
    """Configuration 2 as the BERT FFN's two layers: DQ(x [1024 x 768]) -> MatMulIntegerToFloat with W1 [768 x 3072]
    -> h [1024 x 3072] -> DQ(h) -> MatMulIntegerToFloat with W2 [3072 x 768] (both per-column symmetric, scales made in
    the epilogue). ranged=True: layer 1 records the range of h as it stores it (EncodeFloatRanged), so DQ(h) is its
    quantize pass alone (EncodeRanged); ranged=False: DQ(h) runs both passes, as the reference chains it
    (Int8Tests.cs:705-751 per layer)."""
    M, K, N = 1024, 768, 3072
    x = synth(d, og.ElementType.Float32, M * K, 2, 30, 0.0, 1.0, 2)
    w1, s1 = sym_weights(d, K, N, 2, 31)
    w2, s2 = sym_weights(d, N, K, 2, 32)
    ya, yh = d.CreateBufferOf(og.ElementType.UInt8, M * K), d.CreateBufferOf(og.ElementType.UInt8, M * N)
    sa, sh = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.Float32, 1)
    za, zh = d.CreateBufferOf(og.ElementType.UInt8, 4), d.CreateBufferOf(og.ElementType.UInt8, 4)
    h = d.CreateBufferOf(og.ElementType.Float32, M * N)
    out = d.CreateBufferOf(og.ElementType.Float32, M * K)
    ranges = og.Int8Ranges(d.CreateBufferOf(og.ElementType.Float32, 2 * og.OG_RANGES_MAX))
    dq, gemm = og.DynamicQuantizeKernels(d), og.Int8Gemm(d)
    p1, p2 = og.Int8GemmProblem(M, N, K), og.Int8GemmProblem(M, K, N)

    def step(e, i):
        dq.Encode(e, x, 0, M * K, ya, 0, sa, 0, za, 0)
        if ranged:
            gemm.EncodeFloatRanged(e, p1, ya, w1, h, og.Int8Operand(s1, 0, True), ranges, og.Int8Operand(za, 0),
                                   activationScale=og.Int8Operand(sa, 0))
            dq.EncodeRanged(e, h, 0, M * N, yh, 0, sh, 0, zh, 0, ranges)
        else:
            gemm.EncodeFloatScaled(e, p1, ya, w1, h, og.Int8Operand(sa, 0), og.Int8Operand(s1, 0, True),
                                   og.Int8Operand(za, 0))
            dq.Encode(e, h, 0, M * N, yh, 0, sh, 0, zh, 0)
        gemm.EncodeFloatScaled(e, p2, yh, w2, out, og.Int8Operand(sh, 0), og.Int8Operand(s2, 0, True),
                               og.Int8Operand(zh, 0))

    wall, region, times = timed(d, step, steps, warmup)
    # Per dispatch of a step, in order (the step launches the same kernel names more than once).
    nd = len(times) // steps
    per = {}
    for j in range(nd):
        ms = [times[i * nd + j][0] * 1e3 for i in range(steps)]
        per[f"{j}: {times[j][1]}"] = {"mean_us": statistics.mean(ms), "median_us": statistics.median(ms)}
    res = {"ops": 2.0 * 2 * M * N * K, "wall_s": wall, "chain_mean_ms": region / steps * 1e3, "per_kernel": per,
           "dispatches": nd, "range_groups": ranges.Groups if ranged else None}
    if check:
        import oracle
        H = h.Read()
        wy, ws_, wz = oracle.dynamic_quantize(H)
        ok = np.array_equal(yh.Read()[:M * N], wy) and int(zh.Read()[0]) == wz and \
            np.float32(sh.Read()[0]).view(np.uint32) == np.float32(ws_).view(np.uint32)
        rows = np.array([0, 5, 511, 1023])
        W2, S2 = w2.Read(), s2.Read()
        sums = oracle.int8_gemm_rows(oracle.Gemm(M, K, N), wy, False, W2.view(np.uint8), True, rows,
                                     (np.array([wz], np.uint8), False, 0))
        want = oracle.float_epilogue(sums.ravel(), K, (np.float32(ws_) * S2.astype(np.float32)).astype(np.float32),
                                     True).reshape(len(rows), K)
        ok = ok and np.array_equal(out.Read().reshape(M, K)[rows].view(np.uint32), want.view(np.uint32))
        res["check"] = "bit-exact (DQ of h on every element, layer 2 on sampled rows)" if ok else "MISMATCH"
    return res


class C5:
    """Configuration 5's operands, resident on the device: x [32 x 512 x 4096] float32 N(0,1); 32 distinct int8 weight
    matrices [4096 x 4096] (each N(0, 0.02) quantized symmetric per column) with their 32 x 4096 column scales."""
    Bt, M, K, N = 32, 512, 4096, 4096

    def __init__(self, d):
        Bt, M, K, N = self.Bt, self.M, self.K, self.N
        self.x = synth(d, og.ElementType.Float32, Bt * M * K, 5, 40, 0.0, 1.0, 2)
        self.b = d.CreateBufferOf(og.ElementType.Int8, Bt * K * N)
        self.wscale = d.CreateBufferOf(og.ElementType.Float32, Bt * N)
        for i in range(Bt):
            sym_weights(d, K, N, 5, 41 + i, self.b, i * K * N, self.wscale, i * N)
        self.ya = d.CreateBufferOf(og.ElementType.UInt8, Bt * M * K)
        self.s = d.CreateBufferOf(og.ElementType.Float32, 1)
        self.z = d.CreateBufferOf(og.ElementType.UInt8, 4)
        self.c = d.CreateBufferOf(og.ElementType.Int32, Bt * M * N)
        self.sc = d.CreateBufferOf(og.ElementType.Float32, Bt * N)
        self.y = d.CreateBufferOf(og.ElementType.Float32, Bt * M * N)
        self.p = og.Int8GemmProblem(M, N, K)
        self.p.Batch, self.p.StrideA, self.p.StrideB = Bt, M * K, K * N
        self.dq, self.gemm, self.deq = og.DynamicQuantizeKernels(d), og.Int8Gemm(d), og.DequantizeKernels(d)
        self.ops = 2.0 * Bt * M * N * K
        self.product_bytes = Bt * (M * K + K * N + 4 * M * N)

    def quantize(self, e):
        self.dq.Encode(e, self.x, 0, self.Bt * self.M * self.K, self.ya, 0, self.s, 0, self.z, 0)

    def product(self, e):
        self.gemm.EncodeInt32(e, self.p, self.ya, self.b, self.c, og.Int8Operand(self.z, 0))

    def rescale(self, e):
        # y[b, m, n] = DequantizeLinear(c[b, m, n], fl(actScale * wScale[b, n])): the 32 x 4096 scale vector on the
        # device, then one per-column DequantizeLinear per batch (each batch has its own column scales).
        e.RecordScaleProduct(self.s, self.wscale, self.Bt * self.N, self.sc)
        for i in range(self.Bt):
            self.deq.Encode(e, self.c, i * self.M * self.N, [self.M, self.N], 1, True, self.sc, i * self.N, None, 0,
                            self.y, i * self.M * self.N)

    def check(self, with_y):
        import oracle
        Bt, M, K, N = self.Bt, self.M, self.K, self.N
        X = self.x.Read()
        wy, ws_, wz = oracle.dynamic_quantize(X)
        del X
        Y, Z = self.ya.Read(), int(self.z.Read()[0])
        ok = np.array_equal(Y, wy) and Z == wz and np.float32(self.s.Read()[0]) == np.float32(ws_)
        del wy
        Bh = self.b.Read().view(np.uint8)
        pr = oracle.Gemm(M, N, K, Batch=Bt, StrideA=M * K, StrideB=K * N)
        rows = np.array([0, 511, 7 * M + 100, 31 * M + 511])
        want = oracle.int8_gemm_rows(pr, Y, False, Bh, True, rows, (np.array([Z], np.uint8), False, 0))
        C = self.c.Read().reshape(Bt * M, N)
        ok = ok and np.array_equal(C[rows], want)
        if with_y:
            sc = (np.float32(ws_) * self.wscale.Read().astype(np.float32)).astype(np.float32).reshape(Bt, 1, N)
            wanty = (C.reshape(Bt, M, N).astype(np.float32) * sc).astype(np.float32)
            ok = ok and np.array_equal(self.y.Read().view(np.uint32), wanty.reshape(-1).view(np.uint32))
        return ok


def c5_batched(d, steps, warmup, check=True, c5=None):
    """Configuration 5's product alone: 32 x (u8 A [512 x 4096], one DQ of N(0,1)) x (32 distinct int8 B [4096 x 4096]),
    int32 out. The DQ runs once before the timed region."""
    c5 = c5 or C5(d)
    e = d.BeginCommands()
    c5.quantize(e)
    d.Submit(e)
    d.WaitIdle()
    wall, region, times = timed(d, lambda e, i: c5.product(e), steps, warmup)
    _, med, kname = kernel_stats(times)
    res = {"ops": c5.ops, "bytes": c5.product_bytes, "wall_s": wall, "kernel_mean_ms": region / steps * 1e3,
           "event_pair_median_ms": med, "kernel": kname}
    if check:
        res["check"] = "bit-exact on sampled rows" if c5.check(False) else "MISMATCH"
    return res, c5


def c5_chain(d, steps, warmup, check=True, c5=None):
    """Configuration 5 as BASELINE states it, one step = DynamicQuantizeLinear of the 67 M activations (two passes) ->
    the batched int32 product -> DequantizeLinear to float32 with each batch's column scales (a scale-product dispatch,
    then one per batch). Checked whole: the DQ and the rescale against the oracle on every element, the sums on
    sampled rows."""
    c5 = c5 or C5(d)

    def step(e, i):
        c5.quantize(e)
        c5.product(e)
        c5.rescale(e)

    wall, region, times = timed(d, step, steps, warmup)
    per = per_kernel_us(times)
    n_act, n_out = c5.Bt * c5.M * c5.K, c5.Bt * c5.M * c5.N
    kbytes = {"dq-minmax": 4 * n_act, "dq-quantize": 5 * n_act + 5, "scale-product": 8 * c5.Bt * c5.N + 4}
    for k in per:
        # A rescale dispatch moves one batch's int32 in and float32 out, a batched one (every batch's pass in one
        # launch) all of them.
        per[k]["bytes"] = kbytes.get(k, c5.product_bytes if k.startswith("mfma") else
                                     8 * n_out if k.endswith("-batch") else 8 * n_out // c5.Bt)
        per[k]["gbs_median"] = per[k]["bytes"] / (per[k]["median_us"] * 1e-6) / 1e9
        per[k]["hbm_frac_median"] = per[k]["gbs_median"] / PEAK_HBM_GBS
    # The chain's operands once: x read, B and the weight scales read, y written.
    chain_bytes = 4 * n_act + c5.Bt * c5.K * c5.N + 4 * c5.Bt * c5.N + 4 * n_out
    res = {"ops": c5.ops, "chain_bytes": chain_bytes, "wall_s": wall, "chain_mean_ms": region / steps * 1e3,
           "dispatches_per_step": len(times) // steps, "per_kernel": per}
    if check:
        res["check"] = "bit-exact (DQ and rescale whole, sums on sampled rows)" if c5.check(True) else "MISMATCH"
    return res, c5


def elementwise_c5(d, steps, warmup, which, check=True):
    """The element-wise passes alone at configuration 5's sizes, each one launch over 67,108,864 elements:
    'dequant' DequantizeLinear int32 [16384 x 4096] -> float32 with a per-column scale (axis 1); 'quant' QuantizeLinear
    float32 -> uint8 with one scale and zero point; 'dq' DynamicQuantizeLinear of N(0,1) float32 (its two passes).
    Bytes are every operand read or written once."""
    R, N = 32 * 512, 4096
    n = R * N
    if which == "dequant":
        x = synth(d, og.ElementType.Int32, n, 8, 70, -2**31, 2**31 - 1, 1)
        sc = d.CreateBuffer(np.random.default_rng(71).uniform(1e-6, 1e-4, N).astype(np.float32))
        out = d.CreateBufferOf(og.ElementType.Float32, n)
        k = og.DequantizeKernels(d)
        rec = lambda e, i: k.Encode(e, x, 0, [R, N], 1, True, sc, 0, None, 0, out, 0)  # noqa: E731
        bytes_ = 8 * n + 4 * N
    elif which == "quant":
        x = synth(d, og.ElementType.Float32, n, 8, 72, 0.0, 1.0, 2)
        sc = d.CreateBuffer(np.array([4.7 / 255], np.float32))
        zp = d.CreateBuffer(np.array([117, 0, 0, 0], np.uint8))
        out = d.CreateBufferOf(og.ElementType.UInt8, n)
        k = og.DequantizeKernels(d)
        rec = lambda e, i: k.EncodeQuantize(e, x, 0, [n], 0, False, sc, 0, zp, 0, out, 0)  # noqa: E731
        bytes_ = 5 * n + 5
    else:
        x = synth(d, og.ElementType.Float32, n, 8, 73, 0.0, 1.0, 2)
        out = d.CreateBufferOf(og.ElementType.UInt8, n)
        s, z = d.CreateBufferOf(og.ElementType.Float32, 1), d.CreateBufferOf(og.ElementType.UInt8, 4)
        k = og.DynamicQuantizeKernels(d)
        rec = lambda e, i: k.Encode(e, x, 0, n, out, 0, s, 0, z, 0)  # noqa: E731
        bytes_ = 9 * n + 5
    wall, region, times = timed(d, rec, steps, warmup)
    per = per_kernel_us(times)
    step_us = region / steps * 1e6
    res = {"elements": n, "bytes": bytes_, "wall_s": wall, "step_mean_us": step_us, "per_kernel": per,
           "gbs": bytes_ / (step_us * 1e-6) / 1e9}
    res["hbm_frac"] = res["gbs"] / PEAK_HBM_GBS
    res["traffic"] = {k: traffic_of(k, which) for k in per}
    if which == "dq":
        per["dq-minmax"]["bytes"], per["dq-quantize"]["bytes"] = 4 * n, 5 * n + 5
        for kk in per:
            per[kk]["gbs_median"] = per[kk]["bytes"] / (per[kk]["median_us"] * 1e-6) / 1e9
            per[kk]["hbm_frac_median"] = per[kk]["gbs_median"] / PEAK_HBM_GBS
    if check:
        import oracle
        X, got = x.Read(), out.Read()
        if which == "dequant":
            ok = np.array_equal(got.view(np.uint32), oracle.dequantize(X, sc.Read(), True, N, 1).view(np.uint32))
        elif which == "quant":
            ok = np.array_equal(got, oracle.quantize(X, np.array([4.7 / 255], np.float32), False,
                                                     zero=np.array([117], np.uint8)))
        else:
            wy, ws_, wz = oracle.dynamic_quantize(X)
            ok = np.array_equal(got, wy) and int(z.Read()[0]) == wz and np.float32(s.Read()[0]) == np.float32(ws_)
        res["check"] = "bit-exact (every element)" if ok else "MISMATCH"
    for b in (x, out):
        b.Dispose()
    return res


def host_cpu():
    """(threads to use, description): the threads this process may use (its CPU affinity, capped by OMP_NUM_THREADS
    where the host sets it: a GPU box's share of cores for one GPU), beside nproc and the CPU model."""
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    threads = affinity
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return threads, {"nproc": nproc, "affinity": affinity, "omp_num_threads": omp or None, "cpu_model": model}


def cpu_baseline_c4(host_operands, budget_s=12.0, runs=5):
    """The oracle (the reference's CPU definition restated in C, std::thread over rows) on the 4096^3 product's
    operands: `runs` timed runs, each over a fresh block of rows sized to about budget_s / runs seconds, reported as
    the median run's throughput."""
    import oracle
    A, B, Z = host_operands
    M = N = K = 4096
    threads, host = host_cpu()
    p = oracle.Gemm(M, N, K)

    def run_rows(start, count):
        rows = np.arange(start, start + count) % M
        t0 = time.perf_counter()
        oracle.int8_gemm_rows(p, A, False, B.view(np.uint8), True, rows, (Z, True, 0), threads=threads)
        return time.perf_counter() - t0

    chunk = threads
    while True:   # size one run's block of rows
        dt = run_rows(0, chunk)
        if dt >= budget_s / runs / 2 or chunk >= M:
            break
        chunk = min(M, chunk * 2)
    chunk = max(threads, min(M, int(chunk * (budget_s / runs) / max(dt, 1e-3))))
    times, start = [], 0
    for _ in range(runs):
        times.append(run_rows(start, chunk))
        start += chunk
    rates = sorted(2.0 * chunk * N * K / t / 1e12 for t in times)
    return {"value": rates[len(rates) // 2], "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"median of {runs} runs, each {chunk} rows of the 4096^3 product (u8 A with per-row zero point x "
                      f"int8 B), {sum(times):.1f} s in all; oracle/oracle.c ora_int8_gemm_rows on {threads} threads",
            "runs_tops": rates, **host}


def traffic_of(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE per
    dispatch, scaled by the same counters' reading for a device copy of known size), or None when not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    e = t.get("kernels", {}).get(f"{kernel} {workload}")
    return None if e is None else e.get("hbm_bytes_per_launch")


def clock_of(kernel, workload):
    """The clock the chip held and the MFMA-busy fraction for `kernel` on `workload`, from profiles/clock.json
    (rocprofv3 GRBM_GUI_ACTIVE and SQ_VALU_MFMA_BUSY_CYCLES per dispatch), or None when not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "clock.json")) as f:
            return json.load(f).get("kernels", {}).get(f"{kernel} {workload}")
    except (OSError, ValueError):
        return None


def c3_stream_floor(d, steps, warmup, copies=9):
    """The floor configuration 3 is measured against, in one launch: og_util_stream_tiles reads B int8 [4096 x 11008]
    (45 MB) in the one-launch few-rows kernel's own tiles, workgroups and loads and does nothing else; and a
    device-to-device copy of the same 45 MB (read and write). `copies` matrices rotate, 405 MB in all, past the 256 MiB
    Infinity Cache, as in configuration 3's leg."""
    K, N = 4096, 11008
    L = _abi()
    L.og_util_stream_tiles.argtypes = [ctypes.c_void_p, _Buf, ctypes.c_uint32, ctypes.c_uint32, _Buf]
    L.og_memcpy_d2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
    bs = [synth(d, og.ElementType.Int8, K * N, 3, 20 + i, -127, 127, 0) for i in range(copies)]
    sink = d.CreateBufferOf(og.ElementType.UInt32, 1)
    dsts = [d.CreateBufferOf(og.ElementType.UInt8, K * N) for _ in range(2)]

    def region(fn):
        for i in range(warmup):
            fn(i)
        d.WaitIdle()
        ms = ctypes.c_float(0.0)
        _ok(L.og_timing_region_begin(d.Context), d)
        for i in range(steps):
            fn(warmup + i)
        _ok(L.og_timing_region_end(d.Context, ctypes.byref(ms)), d)
        d.WaitIdle()
        return ms.value * 1e3 / steps

    stream_us = region(lambda i: _ok(L.og_util_stream_tiles(d.Context, _b(bs[i % copies]), K, N, _b(sink)), d))
    copy_us = region(lambda i: _ok(L.og_memcpy_d2d(d.Context, dsts[i % 2].DevicePointer, bs[i % copies].DevicePointer,
                                                   K * N), d))
    return {"bytes": K * N, "stream_tiles_us": stream_us, "stream_tiles_gbs": K * N / (stream_us * 1e-6) / 1e9,
            "stream_tiles_frac": K * N / (stream_us * 1e-6) / 1e9 / PEAK_HBM_GBS, "copy_us": copy_us,
            "copy_gbs_read_plus_write": 2 * K * N / (copy_us * 1e-6) / 1e9}


def copy_workload(d, steps, warmup, mib=256):
    """A device-to-device copy of a known size (the counters' calibration for the traffic figures)."""
    n = mib << 20
    src, dst = d.CreateBufferOf(og.ElementType.UInt8, n), d.CreateBufferOf(og.ElementType.UInt8, n)
    L = _abi()
    L.og_memcpy_d2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
    for _ in range(warmup + steps):
        _ok(L.og_memcpy_d2d(d.Context, dst.DevicePointer, src.DevicePointer, n), d)
    d.WaitIdle()
    return {"bytes_read": n, "bytes_written": n, "launches": warmup + steps}


def vendor_int8(steps, warmup):
    """The vendor library's int8 product at 4096^3 for comparison: torch._int_mm (hipBLASLt on ROCm), int8 x int8 ->
    int32 without zero points, B stored K x N (as configuration 4) and N x K, on random and on constant operands,
    timed with torch's events over `steps` back-to-back launches."""
    import torch
    dev = torch.device("cuda", 0)
    M = N = K = 4096
    torch.manual_seed(4)
    out = {}
    for kind in ("random", "constant"):
        if kind == "random":
            a = torch.randint(-128, 128, (M, K), dtype=torch.int8, device=dev)
            b = torch.randint(-128, 128, (K, N), dtype=torch.int8, device=dev)
        else:
            a = torch.full((M, K), 0x37, dtype=torch.int8, device=dev)
            b = torch.full((K, N), -13, dtype=torch.int8, device=dev)
        for layout, bb in (("B K x N", b), ("B N x K", b.t().contiguous().t())):
            for _ in range(warmup):
                torch._int_mm(a, bb)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                torch._int_mm(a, bb)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / steps * 1e3
            out[f"{kind}, {layout}"] = {"us": us, "tops": 2.0 * M * N * K / us / 1e6}
    return out


def qlinear_c2(d, steps, warmup, fused, check=True):
    """QLinearMatMul on configuration 2's product (1024 x 3072 x 768): u8 A with a zero point, int8 B symmetric per
    column (N(0, 0.02)), int bias and multiplier per column, u8 output with zero point 128. `fused`: one launch, the
    requantization in the product's store; else the reference's two passes (int32 sums into scratch, then the
    requantize pass)."""
    M, K, N = 1024, 768, 3072
    a = synth(d, og.ElementType.UInt8, M * K, 2, 50, 0, 255, 0)
    q, _ = sym_weights(d, K, N, 2, 51)
    za = d.CreateBuffer(np.array([131, 0, 0, 0], np.uint8))
    cols = np.arange(N)
    multv = ((cols % 97).astype(np.float32) * np.float32(1e-6) + np.float32(2.5e-4)).astype(np.float32)
    ibv = (((cols * 6007) % 4001) - 2000).astype(np.int32)
    mult, ib = d.CreateBuffer(multv), d.CreateBuffer(ibv)
    y = d.CreateBufferOf(og.ElementType.UInt8, M * N)
    scratch = d.CreateBufferOf(og.ElementType.Int32, M * N)
    gemm = og.Int8Gemm(d, og.Int8GemmOptions(FusedRequantize=fused))
    p = og.Int8GemmProblem(M, N, K)
    wall, region, times = timed(d, lambda e, i: gemm.EncodeRequantized(e, p, a, q, y, og.Int8Operand(mult, 0, True), 128,
                                                                       og.Int8Operand(za, 0), None,
                                                                       og.Int8Operand(ib, 0, True),
                                                                       og.Int8Scratch(scratch)),
                                steps, warmup)
    per = {}
    for t, k in times:
        per.setdefault(k, []).append(t)
    bytes_ = M * K + K * N + M * N + 8 * N + 1
    res = {"ops": 2.0 * M * N * K, "wall_s": wall, "step_mean_ms": region / steps * 1e3, "bytes": bytes_,
           "dispatch_mean_ms": {k: statistics.mean(v) for k, v in per.items()}}
    if check:
        import oracle
        A, Q = a.Read(), q.Read()
        rows = np.array([0, 7, 600, 1023])
        sums = oracle.int8_gemm_rows(oracle.Gemm(M, N, K), A, False, Q.view(np.uint8), True, rows,
                                     (np.array([131], np.uint8), False, 0))
        want = oracle.requant_array(sums.ravel(), N, multv, True, 128, True, ibv).reshape(len(rows), N)
        got = y.Read().reshape(M, N)[rows]
        res["check"] = "bit-exact" if np.array_equal(got, want) else "MISMATCH"
    return res


def embedding_gather(d, steps, warmup, tokens, check=True, vocab=250002, hidden=768):
    """The int8 embedding lookup in front of the first int8 product: Gather on axis 0 of an int8 table
    [vocab, hidden] (the largest vocabulary of the reference's embedding tests) with `tokens` int64 token ids.
    Bytes per step: the rows read and written once each, and the ids."""
    table = synth(d, og.ElementType.Int8, vocab * hidden, 6, 60, -128, 127, 0)
    ids_host = (np.random.default_rng(tokens).integers(0, vocab, tokens)).astype(np.int64)
    ids = d.CreateBuffer(ids_host)
    out = d.CreateBufferOf(og.ElementType.Int8, tokens * hidden)
    k = og.GatherKernels(d)
    wall, region, times = timed(d, lambda e, i: k.EncodeGather(e, table, 0, [vocab, hidden], 0, ids, 0, tokens, out, 0),
                                steps, warmup)
    res = {"tokens": tokens, "bytes": 2 * tokens * hidden + 8 * tokens, "wall_s": wall, "step_mean_ms": region / steps * 1e3,
           "kernel": times[0][1] if times else ""}
    if check:
        rows = np.array([0, 1, tokens // 2, tokens - 1])
        T = table.Read().reshape(vocab, hidden)
        got = out.Read().reshape(tokens, hidden)[rows]
        res["check"] = "bit-exact" if np.array_equal(got, T[ids_host[rows]]) else "MISMATCH"
    return res


def resnet50_convs() -> list:
    """The 53 convolutions of ResNet-50 (v1.5: the stride of a stage's first block in its 3 x 3) at 224 x 224, as
    (in channels, size, out channels, kernel, stride, pad)."""
    layers = [(3, 224, 64, 7, 2, 3)]
    cin, size = 64, 56
    for blocks, mid, out, stride in ((3, 64, 256, 1), (4, 128, 512, 2), (6, 256, 1024, 2), (3, 512, 2048, 2)):
        for b in range(blocks):
            s = stride if b == 0 else 1
            layers.append((cin, size, mid, 1, 1, 0))
            layers.append((mid, size, mid, 3, s, 1))
            osize = size // s
            layers.append((mid, osize, out, 1, 1, 0))
            if b == 0:
                layers.append((cin, size, out, 1, s, 0))   # the projection shortcut
            cin, size = out, osize
    return layers


def conv_workload(d, steps, warmup, which):
    """ConvInteger layers at batch 1, u8 activations with a zero point, int8 weights with a zero point per output
    channel, int32 out: 'resnet50' runs all 53 convolutions of ResNet-50 back to back as one step; 'whisper' the
    two convolutions of the Whisper-small stem; 'depthwise' MobileNet's 96-channel 3 x 3 depthwise layer at 28 x 28."""
    if which == "resnet50":
        layers = [(1, c, h, h, o, k, k, s, p, 1) for (c, h, o, k, s, p) in resnet50_convs()]
    elif which == "whisper":
        layers = [(1, 80, 1, 3000, 768, 1, 3, 1, 1, 1), (1, 768, 1, 3000, 768, 1, 3, 2, 1, 1)]
    else:
        layers = [(1, 96, 28, 28, 96, 3, 3, 1, 1, 96)]
    conv = og.ConvIntegerKernels(d)
    items, ops = [], 0.0
    for i, (b, c, h, w, o, kh, kw, st, pad, g) in enumerate(layers):
        q = og.ConvProblem(b, c, h, w, o, kh, kw)
        q.StrideWidth = st
        q.StrideHeight = st if h > 1 else 1
        q.PadLeft = q.PadRight = pad
        q.PadTop = q.PadBottom = pad if h > 1 else 0
        q.Groups = g
        x = synth(d, og.ElementType.UInt8, b * c * h * w, 7, 100 + 3 * i, 0, 255, 0)
        wt = synth(d, og.ElementType.Int8, o * (c // g) * kh * kw, 7, 101 + 3 * i, -127, 127, 0)
        wz = synth(d, og.ElementType.Int8, o, 7, 102 + 3 * i, -8, 8, 0)
        xz = d.CreateBuffer(np.array([128, 0, 0, 0], np.uint8))
        y = d.CreateBufferOf(og.ElementType.Int32, b * o * q.OutHeight * q.OutWidth)
        items.append((q, x, wt, y, xz, wz))
        ops += 2.0 * b * o * q.OutHeight * q.OutWidth * (c // g) * kh * kw

    def step(e, i):
        for q, x, wt, y, xz, wz in items:
            conv.Encode(e, q, x, wt, y, og.Int8Operand(xz, 0), og.Int8Operand(wz, 0, True))

    wall, region, times = timed(d, step, steps, warmup)
    per = {}
    for t, k in times:
        per.setdefault(k, []).append(t)
    return {"layers": len(layers), "ops": ops, "wall_s": wall, "step_mean_ms": region / steps * 1e3,
            "dispatches_per_step": len(times) // steps,
            "kernel_ms_per_step": {k: sum(v) / steps for k, v in per.items()}}


def only(d, name, steps, warmup):
    """One workload alone (for rocprofv3 runs of committed files); prints a one-line summary."""
    if name == "c4":
        r = c4_square(d, steps, warmup, check=False)
        r.pop("host_operands", None)
    elif name == "gemvshard":
        r = c3_gemv(d, 1, steps, warmup, copies=48, check=False, n=1376)
    elif name.startswith("gemv") and name.endswith("tiles"):
        r = c3_gemv(d, int(name[4:-5] or 1), steps, warmup, check=False, opts={"FewRowsOneLaunch": False})
    elif name.startswith("gemv"):
        r = c3_gemv(d, int(name[4:] or 1), steps, warmup, check=False)
    elif name == "c2":
        r = c2_bert_ffn(d, steps, warmup, check=False)
    elif name in ("c2ffn", "c2ffn2"):
        r = c2_two_layer(d, steps, warmup, ranged=name == "c2ffn", check=False)
    elif name == "c5":
        r = c5_batched(d, steps, warmup, check=False)[0]
    elif name == "c5chain":
        r = c5_chain(d, steps, warmup, check=False)[0]
    elif name in ("dequant", "quant", "dq"):
        r = elementwise_c5(d, steps, warmup, name, check=False)
    elif name in ("c2q", "c2q2"):
        r = qlinear_c2(d, steps, warmup, fused=name == "c2q", check=False)
    elif name in ("resnet50", "whisper", "depthwise"):
        r = conv_workload(d, steps, warmup, name)
    elif name.startswith("gather"):
        r = embedding_gather(d, steps, warmup, int(name[6:] or 4096), check=False)
    elif name == "copy":
        r = copy_workload(d, steps, warmup)
    elif name == "stream":
        r = c3_stream_floor(d, steps, warmup)
    elif name in ("c4const", "c4nt", "c4plain", "c4plainnt"):
        r = c4_square(d, steps, warmup, check=False, constant=name == "c4const", trans_b=name.endswith("nt"),
                      plain=name.startswith("c4plain"))
        r.pop("host_operands", None)
        r["tops_kernel"] = r["ops"] / (r["kernel_mean_ms"] * 1e-3) / 1e12
    else:
        raise SystemExit(f"unknown workload {name}")
    print(json.dumps({"workload": name, **{k: v for k, v in r.items() if isinstance(v, (int, float, str, list, dict))}}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline configuration only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["c4", "c4const", "c4nt", "c4plain", "c4plainnt", "gemv1", "gemv4", "gemv16", "gemvshard", "gemv1tiles", "gemv16tiles", "c2", "c2ffn", "c2ffn2", "c2q", "c2q2", "c5", "c5chain", "dequant", "quant", "dq", "gather4096", "gather65536", "resnet50", "whisper", "depthwise", "copy", "stream", "vendor"],
                    help="run one workload alone and print its summary (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported"}))
        sys.exit(2)
    if args.only == "vendor":
        # torch's bundled HIP runtime must own the device in this process: no context of this library is opened.
        print(json.dumps({"workload": "vendor", "hipblaslt_int_mm_4096": vendor_int8(args.steps, args.warmup)}))
        return
    d = og.GpuDevice.Create(0)
    log = lambda s: print(s, file=sys.stderr, flush=True)  # noqa: E731
    if args.only:
        only(d, args.only, args.steps, args.warmup)
        return

    log("config 4: 4096^3 MatMulInteger")
    c4 = c4_square(d, args.steps, args.warmup)
    tops = c4["ops"] * args.steps / c4["wall_s"] / 1e12
    kern_tops = c4["ops"] / (c4["kernel_mean_ms"] * 1e-3) / 1e12
    configs = {"c4_square_4096": {"tops_wall": tops, "tops_kernel": kern_tops, "kernel": c4["kernel"],
                                  "kernel_mean_us": c4["kernel_mean_ms"] * 1e3,
                                  "event_pair_mean_us": c4["event_pair_mean_ms"] * 1e3,
                                  "event_pair_median_us": c4["event_pair_median_ms"] * 1e3,
                                  "tops_event_pair_median": c4["ops"] / (c4["event_pair_median_ms"] * 1e-3) / 1e12,
                                  "check": c4["check"]}}
    log(json.dumps(configs["c4_square_4096"]))

    gemv = {}
    for m in ((1,) if args.quick else (1, 4, 16)):
        log(f"config 3: GEMV M={m}")
        r = c3_gemv(d, m, args.steps, args.warmup)
        gbs = r["bytes"] / (r["step_mean_ms"] * 1e-3) / 1e9
        gemv[m] = {"gbs": gbs, "frac": gbs / PEAK_HBM_GBS, "step_mean_us": r["step_mean_ms"] * 1e3,
                   "tops": r["ops"] / (r["step_mean_ms"] * 1e-3) / 1e12, "kernels": r["kernels"],
                   "dispatch_mean_us": [t * 1e3 for t in r["dispatch_mean_ms"]],
                   "event_pair_step_mean_us": r["event_pair_step_mean_ms"] * 1e3,
                   "event_pair_step_median_us": r["event_pair_step_median_ms"] * 1e3, "bytes": r["bytes"],
                   "check": r["check"]}
        configs[f"c3_gemv_m{m}"] = gemv[m]
        log(json.dumps(gemv[m]))
    if not args.quick:
        log("config 3 at one GPU's share of an 8-way column split: M=1, N=1376")
        r = c3_gemv(d, 1, args.steps, args.warmup, copies=48, n=1376)
        gbs = r["bytes"] / (r["step_mean_ms"] * 1e-3) / 1e9
        configs["c3_gemv_m1_shard8"] = {"n": 1376, "weight_copies": 48, "gbs": gbs, "frac": gbs / PEAK_HBM_GBS,
                                        "step_mean_us": r["step_mean_ms"] * 1e3, "kernels": r["kernels"],
                                        "dispatch_mean_us": [t * 1e3 for t in r["dispatch_mean_ms"]],
                                        "bytes": r["bytes"], "check": r["check"]}
        log(json.dumps(configs["c3_gemv_m1_shard8"]))
    log("config 3's floor: B read once in the one-launch kernel's tiles, and a 45 MB copy")
    configs["c3_stream_floor"] = c3_stream_floor(d, args.steps, args.warmup)
    log(json.dumps(configs["c3_stream_floor"]))
    if not args.quick:
        log("config 2: BERT FFN chain")
        r = c2_bert_ffn(d, args.steps, args.warmup)
        configs["c2_bert_ffn"] = {"chain_wall_us": r["wall_s"] / args.steps * 1e6,
                                  "chain_mean_us": r["chain_mean_ms"] * 1e3,
                                  "chain_gbs": r["chain_bytes"] / (r["chain_mean_ms"] * 1e-3) / 1e9,
                                  "tops": r["ops"] / (r["chain_mean_ms"] * 1e-3) / 1e12,
                                  "per_kernel": r["per_kernel"], "check": r["check"]}
        log(json.dumps(configs["c2_bert_ffn"]))
        log("config 2: BERT FFN chain with the scale product as its own dispatch (the reference's chain)")
        r = c2_bert_ffn(d, args.steps, args.warmup, fused_scale=False)
        configs["c2_bert_ffn_separate_scale"] = {"chain_mean_us": r["chain_mean_ms"] * 1e3,
                                                 "per_kernel": r["per_kernel"], "check": r["check"]}
        log(json.dumps(configs["c2_bert_ffn_separate_scale"]))
        for ranged, key in ((True, "c2_ffn_two_layers_ranged"), (False, "c2_ffn_two_layers_two_pass_dq")):
            log(f"config 2 as two FFN layers, DQ of the hidden layer {'from its recorded range' if ranged else 'in two passes'}")
            r = c2_two_layer(d, args.steps, args.warmup, ranged)
            configs[key] = {"chain_mean_us": r["chain_mean_ms"] * 1e3, "dispatches": r["dispatches"],
                            "tops": r["ops"] / (r["chain_mean_ms"] * 1e-3) / 1e12, "per_kernel": r["per_kernel"],
                            "range_groups": r["range_groups"], "check": r["check"]}
            log(json.dumps(configs[key]))
        for fused, key in ((True, "qlinear_c2_one_launch"), (False, "qlinear_c2_two_passes")):
            log(f"QLinearMatMul on configuration 2's product, {'one launch' if fused else 'two passes'}")
            r = qlinear_c2(d, args.steps, args.warmup, fused)
            configs[key] = {"step_mean_us": r["step_mean_ms"] * 1e3,
                            "gbs": r["bytes"] / (r["step_mean_ms"] * 1e-3) / 1e9,
                            "tops": r["ops"] / (r["step_mean_ms"] * 1e-3) / 1e12,
                            "dispatch_mean_us": {k: v * 1e3 for k, v in r["dispatch_mean_ms"].items()},
                            "check": r["check"]}
            log(json.dumps(configs[key]))
        for tokens in (4096, 65536):
            log(f"int8 embedding lookup: 250002 x 768 table, {tokens} token ids")
            r = embedding_gather(d, args.steps, args.warmup, tokens)
            gbs = r["bytes"] / (r["step_mean_ms"] * 1e-3) / 1e9
            configs[f"embedding_gather_{tokens}"] = {"step_mean_us": r["step_mean_ms"] * 1e3, "gbs": gbs,
                                                     "frac": gbs / PEAK_HBM_GBS, "kernel": r["kernel"],
                                                     "check": r["check"]}
            log(json.dumps(configs[f"embedding_gather_{tokens}"]))
        for which in ("resnet50", "whisper", "depthwise"):
            log(f"ConvInteger: {which} at batch 1")
            r = conv_workload(d, args.steps, args.warmup, which)
            configs[f"conv_{which}_b1"] = {"layers": r["layers"], "step_mean_us": r["step_mean_ms"] * 1e3,
                                            "tops": r["ops"] / (r["step_mean_ms"] * 1e-3) / 1e12,
                                            "dispatches_per_step": r["dispatches_per_step"],
                                            "kernel_us_per_step": {k: v * 1e3 for k, v in r["kernel_ms_per_step"].items()}}
            log(json.dumps(configs[f"conv_{which}_b1"]))
        log("config 5: batched 32 x 512 x 4096 x 4096, the product alone")
        c5_steps = max(3, args.steps // 5)
        r, c5 = c5_batched(d, c5_steps, 2)
        tops5 = r["ops"] / (r["kernel_mean_ms"] * 1e-3) / 1e12
        gbs5 = r["bytes"] / (r["kernel_mean_ms"] * 1e-3) / 1e9
        configs["c5_batched"] = {"tops_kernel": tops5, "mfma_frac": tops5 / PEAK_INT8_TOPS, "gbs": gbs5,
                                 "hbm_frac": gbs5 / PEAK_HBM_GBS, "kernel_mean_us": r["kernel_mean_ms"] * 1e3,
                                 "event_pair_median_us": r["event_pair_median_ms"] * 1e3, "kernel": r["kernel"],
                                 "bytes": r["bytes"], "check": r["check"]}
        log(json.dumps(configs["c5_batched"]))
        log("config 5 as a chain: DynamicQuantizeLinear -> batched product -> DequantizeLinear per batch")
        r, _ = c5_chain(d, c5_steps, 2, c5=c5)
        del c5
        us = r["chain_mean_ms"] * 1e3
        configs["c5_chain"] = {"chain_mean_us": us, "tops": r["ops"] / (us * 1e-6) / 1e12,
                               "mfma_frac": r["ops"] / (us * 1e-6) / 1e12 / PEAK_INT8_TOPS,
                               "chain_gbs": r["chain_bytes"] / (us * 1e-6) / 1e9,
                               "hbm_frac": r["chain_bytes"] / (us * 1e-6) / 1e9 / PEAK_HBM_GBS,
                               "chain_bytes": r["chain_bytes"], "dispatches_per_step": r["dispatches_per_step"],
                               "per_kernel": r["per_kernel"], "check": r["check"]}
        log(json.dumps(configs["c5_chain"]))
        for which in ("dequant", "quant", "dq"):
            log(f"element-wise at configuration 5's size: {which}")
            configs[f"{which}_c5_size"] = elementwise_c5(d, args.steps // 2 or 1, 2, which)
            log(json.dumps(configs[f"{which}_c5_size"]))

    roof = {"bound": "mfma", "achieved": kern_tops, "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
            "frac": kern_tops / PEAK_INT8_TOPS, "traffic": traffic_of(c4["kernel"], "c4"),
            "note": "int8 ops (a multiply-add counts 2), 2*M*N*K per launch over the average launch duration (one HIP "
                    "event pair on the library's stream around the back-to-back timed launches, / steps); unit is "
                    "tera-ops/s"}
    clk = clock_of(c4["kernel"], "c4")
    if clk:
        # The nominal peak assumes 2.4 GHz; on random int8 operands the chip's power limit holds a lower clock
        # (measured with rocprofv3 on the same kernel and workload), and the peak at that clock is the reachable one.
        peak_adj = PEAK_INT8_TOPS * clk["held_clock_ghz"] / 2.4
        roof["clock_adjusted"] = {"held_clock_ghz": round(clk["held_clock_ghz"], 3), "peak": round(peak_adj, 1),
                                  "frac": kern_tops / peak_adj, "mfma_busy_profiled": round(clk["mfma_busy"], 3),
                                  "source": "profiles/clock.json (GRBM_GUI_ACTIVE / duration; MfmaUtil)"}
    cpu = None if args.no_cpu else cpu_baseline_c4(c4["host_operands"])
    g1 = gemv.get(1)
    line = {
        "metric": METRIC, "value": round(tops, 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": c4["wall_s"] / args.steps * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic (device-side SplitMix64)",
        "config": {"workload": "MatMulInteger M=N=K=4096, uint8 A per-row zero point, int8 B (K x N), int32 out",
                   "global_batch": 1, "m": 4096, "n": 4096, "k": 4096, "parallelism": "single GPU"},
        "roofline": roof,
        "gemv_m1": None if g1 is None else {
            "metric": "GB/s at M=1 K=4096 N=11008 (MatMulIntegerToFloat, 9 rotating weight copies)",
            "value": round(g1["gbs"], 1), "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": g1["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": g1["frac"], "traffic": traffic_of(g1["kernels"][0], "gemv1")},
            "floor": configs.get("c3_stream_floor")},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
