#!/usr/bin/env python3
"""Benchmark of the MI355X ternary GEMV/GEMM library, one JSON line.

Headline workload (the decode GEMV sweep, M = 1): int2 upcvt GEMV, bf16
activations ~N(0,1), ternary weights p(-1,0,+1) = (.25,.5,.25) packed 2
bits/weight, per-128-group bf16 scales ~U[.005,.02], fused bias add (bias
~N(0,0.1)) + residual add (residual ~N(0,1)), shapes (K=4096, N=14336) and
(K=14336, N=4096).  A step = one GEMV per shape.  Every call reads its own
weight set out of a rotation of distinct sets totalling > 2 GiB per shape (the
reference's cache-defeat rule, int2_fp16_upcvt/main.cpp:218-228), so weights
stream from HBM, not from the 256 MB Infinity Cache.

The same line reports the metric's prefill half and the other workloads,
each timed the same way (> 2 GiB rotation, HIP-graph replays between events):
  prefill  int2 x int8 prefill M=1024 K=4096 N=14336 fp16, quant_a pre-kernel
           + s8 x s2 GEMM (TOPS, fraction of the 5.0 POPS int8 peak)
  c1       int2 GEMV M=1 K=N=4096 fp16, no epilogue
  c4       FWHT (HB 512, sign flip) + BITCOS GEMV M=1 K=5376 N=21504, z = .3/.5/.7
  c5       int2 MoE prefill layer T=2048 E=64 top-8 H=2048 I=1408 bf16
           (TFLOPS, fraction of the 2.5 PFLOPS bf16 peak)

Timing: the W warm-up steps and then exactly K timed steps are captured in HIP
graphs (host launch overhead stays off the GPU timeline) and replayed on one
stream between HIP events, after a device synchronize; every figure is the
median of 3 timed replays (the reference's median-of-3 re-measure,
int2_fp16_upcvt/bench.sh:52-63).  `value` and `roofline` come from the timed
step; per-kernel durations come from graphs of that kernel's launches alone,
and each headline shape is also timed with its decode removed (the same kernel
streaming the same bytes: the engine's memory ceiling, the reference's own
method, int2_fp16_upcvt/README.md:135-137).  Bytes follow the reference
byte models (int2_fp16_upcvt/main.cpp:331-333, bitcos_fp16_upcvt/main.cpp:289-293),
ops 2*M*N*K (int2_moe/prefill.cpp:350 for the MoE layer).  The CPU baseline is
the reference's own host golds (compiled from its sources into oracle/_ref)
timed on this machine's CPU cores, all of them and one, per config.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
I8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POPS
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA, 2.5 PFLOPS
METRIC = "GEMV weight-stream GB/s (%HBM peak) at M=1; prefill TOPS (%MFMA peak) at M=1024"
SHAPES = [(4096, 14336), (14336, 4096)]
WEIGHT_ROTATION_BYTES = 2 * 2**30
POSTOP_BIAS_RESIDUAL = 5


def gemv_bytes(M, K, N):
    """Reference byte model with Other (residual, DT) and Bias (DT)."""
    return M * K * 2 + K * N / 4 + M * N * 2 + (K // 128) * N * 2 + M * N * 2 + N * 2


class ShapeBench:
    """Device buffers of one shape: one input set copied into enough rotating
    weight sets to exceed 2 GiB (the reference uploads the same host data to
    every set too)."""

    def __init__(self, torch, T, synth, formats, M, K, N, seed, tile=None):
        self.torch, self.T, self.M, self.K, self.N, self.tile = torch, T, M, K, N, tile
        g = synth.rng(seed)
        bf16 = True
        self.A = synth.activations(g, (M, K), bf16)
        self.B = synth.int2_weights(g, K, N)
        self.S = synth.scales(g, K, N, bf16)
        self.other = synth.activations(g, (M, N), bf16)
        self.bias = formats.f32_to_dt(g.standard_normal(N).astype(np.float32) * np.float32(0.1), bf16)
        dev = torch.device("cuda:0")
        dt = torch.bfloat16
        self.dA = torch.from_numpy(self.A.view(np.int16)).to(dev).view(dt)
        self.dO = torch.from_numpy(self.other.view(np.int16)).to(dev).view(dt)
        self.dBias = torch.from_numpy(self.bias.view(np.int16)).to(dev).view(dt)
        B0 = torch.from_numpy(self.B.view(np.int32)).to(dev)
        S0 = torch.from_numpy(self.S.view(np.int16)).to(dev).view(dt)
        wbytes = self.B.nbytes + self.S.nbytes
        self.sets = max(1, math.ceil(WEIGHT_ROTATION_BYTES / wbytes))
        self.dB = [B0.clone() for _ in range(self.sets)]
        self.dS = [S0.clone() for _ in range(self.sets)]
        self.dC = torch.empty((M, N), dtype=dt, device=dev)
        wsb = T.int2_gemm_ws_bytes(M, N, K)  # the K split's slice sums and strip counters
        self.ws = torch.zeros(wsb, dtype=torch.uint8, device=dev) if wsb else None
        self.next = 0

    def launch(self):
        s = self.next % self.sets
        self.next += 1
        self.T.int2_fp16_upcvt_gemm(self.dA, self.dB[s], self.dS[s], self.dC, self.dO, self.dBias,
                                    self.M, self.N, self.K, POSTOP_BIAS_RESIDUAL, False, ws=self.ws,
                                    tile=self.tile)

    def bytes(self):
        return gemv_bytes(self.M, self.K, self.N)

    def output(self):
        return self.dC.view(self.torch.int16).cpu().numpy().view(np.uint16)


def graph_of(torch, fn, n):
    """Capture n calls of fn into a HIP graph (on a side stream)."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # one eager call on the capture stream before capture
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        for _ in range(n):
            fn()
    return g, s


def time_graph(torch, g, s):
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        e0.record(s)
        g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3  # seconds


REPEATS = 3  # every figure: the median of this many timed replays
_T0 = time.perf_counter()


def progress(msg):
    """One progress line on stderr per finished stage (the JSON line stays alone on stdout)."""
    print(f"[bench {time.perf_counter() - _T0:7.1f}s] {msg}", file=sys.stderr, flush=True)


def median_replays(torch, g, s, reps=REPEATS):
    """Median and all of reps timed replays of graph g (after one warm replay)."""
    time_graph(torch, g, s)
    ts = [time_graph(torch, g, s) for _ in range(reps)]
    return float(np.median(ts)), ts


def per_launch_us(torch, sb, n):
    """Duration of one launch of this shape: a graph of n launches, median of 3 replays."""
    g, s = graph_of(torch, sb.launch, n)
    t, _ = median_replays(torch, g, s)
    return t / n * 1e6


def check_parity(sb, orc, formats):
    """Set 0 output against the oracle (bias + residual epilogue, bf16)."""
    acc = orc.int2_gold(sb.A, sb.B, sb.S, sb.M, sb.K, sb.N, True)
    want = formats.dt_to_f32(orc.epilogue(acc, sb.other, sb.bias, POSTOP_BIAS_RESIDUAL, False, True), True)
    got = formats.dt_to_f32(sb.output(), True)
    d = np.abs(got - want)
    bad = int((d > 1e-3 + 1e-2 * np.abs(want)).sum())
    return bad, float(d.max())


def ceiling_us(torch, T, sb):
    """The shape's GEMV kernel with the decode removed (ternocl_int2_gemv_stream_probe):
    the same plan, weight and scale stream, reduction and stores, on the same
    rotated weight sets; graph of 200 launches, median of 3."""
    out = torch.empty((sb.M, sb.N), dtype=torch.float32, device="cuda")
    it = [0]

    def call():
        s = it[0] % sb.sets
        it[0] += 1
        T.int2_gemv_stream_probe(sb.dB[s], sb.dS[s], out, sb.M, sb.N, sb.K)
    return graph_time_us(torch, call, 200)


def wait_mode_us(torch, fn, n=50):
    """The reference's per-launch timing (int2_fp16_upcvt/main.cpp:303-328): each call between
    a pair of events on the launch stream, then a synchronize; median and mean over n calls
    (after 5 untimed ones)."""
    st = torch.cuda.current_stream()
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        fn()
        e1.record(st)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3)
    return float(np.median(ts)), float(np.mean(ts))


def plain_read_us(torch, T, nbytes, n=200):
    """One launch of the plain streaming read (ternocl_stream_read_probe) over nbytes, each
    launch on its own buffer of a > 2 GiB rotation: the per-launch ceiling of a kernel that
    must stream that many bytes (graph of n launches, median of 3)."""
    nb = (int(nbytes) + 15) // 16 * 16
    sets = max(1, math.ceil(WEIGHT_ROTATION_BYTES / nb))
    bufs = [torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(sets)]
    for b in bufs:
        b.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    it = [0]

    def call():
        T.stream_read_probe(bufs[it[0] % sets], nb, sink)
        it[0] += 1
    us = graph_time_us(torch, call, max(n, 2 * sets))
    del bufs
    torch.cuda.empty_cache()
    return us


# The reference's GEMV / prefill benchmark shapes (int2_fp16_upcvt/bench.sh:12) and its
# published Arc Pro B70 results at them (int2_fp16_upcvt/README.md:121-155: GEMV GiB/s at
# M=1, prefill TFLOPS at M=1024; fp16, >= 2 GiB rotating weights, median of 3).
REF_SHAPES = [("8B.qkv", 4096, 6144, 434, 137), ("8B.o_proj", 4096, 4096, 403, 130),
              ("8B.gate_up", 4096, 24576, 528, 139), ("8B.down", 12288, 4096, 496, 141),
              ("8B.lm_head", 4096, 151680, 552, 131), ("27B.gate_up", 5120, 34816, 509, 138),
              ("27B.down", 17408, 5120, 517, 132), ("27B.qkvz", 5120, 16384, 519, 138),
              ("27B.out_proj", 6144, 5120, 455, 133), ("27B.qkv", 5120, 14336, 512, 141),
              ("27B.lm_head", 5120, 248320, 550, 128)]


def bench_ref_shapes(torch, T, synth, formats, orc):
    """The reference's 11 benchmark shapes, fp16, no epilogue, >2 GiB rotating weight sets:
    the decode GEMV at M=1 (reference byte model, GB/s and GiB/s, fraction of 8 TB/s, the
    plain-read time of the same bytes, the wait-mode per-launch time) and the prefill GEMM
    at M=1024 (TFLOPS, fraction of the 2.5 PF fp16 peak), each parity-checked against the
    oracle (M=1: every column; M=1024: rows 0..3)."""
    out = {}
    for i, (name, K, N, ref_gibs, ref_tf) in enumerate(REF_SHAPES):
        bf16 = False
        g = synth.rng(900 + i)
        A = synth.activations(g, (1024, K), bf16)
        B, S = synth.int2_weights(g, K, N), synth.scales(g, K, N, bf16)
        sets, W = rotation(torch, [dev32(torch, B), dev16(torch, S, bf16)], B.nbytes + S.nbytes)
        e = {"K": K, "N": N, "weight_sets": sets}
        for M in (1, 1024):
            dA = dev16(torch, A[:M], bf16)
            dC = torch.empty((M, N), dtype=torch.float16, device="cuda")
            wsb = T.int2_gemm_ws_bytes(M, N, K)
            ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda") if wsb else None
            it = [0]

            def call():
                b, sc = W[it[0] % sets]
                it[0] += 1
                T.int2_fp16_upcvt_gemm(dA, b, sc, dC, None, None, M, N, K, ws=ws)
            call()
            torch.cuda.synchronize()
            rows = min(M, 4)
            want = formats.dt_to_f32(orc.epilogue(orc.int2_gold(np.ascontiguousarray(A[:rows]), B, S, rows, K, N,
                                                                bf16), None, None, 0, False, bf16), bf16)
            got = formats.dt_to_f32(dC[:rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16), bf16)
            bad = int((np.abs(got - want) > 1e-3 + 1e-2 * np.abs(want)).sum())
            if M == 1:
                us = graph_time_us(torch, call, max(100, 2 * sets))
                nbytes = K * 2 + K * N / 4 + N * 2 + (K // 128) * N * 2  # int2_fp16_upcvt/bench.sh:27
                w_med, w_mean = wait_mode_us(torch, call)
                pr = plain_read_us(torch, T, nbytes)
                e["gemv_m1"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                "GiB/s": round(nbytes / us * 1e6 / 2**30, 1),
                                "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": int(nbytes),
                                "plain_read_us": round(pr, 3), "of_plain_read": round(pr / us, 4),
                                "wait_mode_us": {"median": round(w_med, 3), "mean": round(w_mean, 3)},
                                "ref_b70_GiB/s": ref_gibs, "parity_bad": bad}
            else:
                us = graph_time_us(torch, call, 10)
                tf = 2.0 * M * N * K / us / 1e6
                e["prefill_m1024"] = {"us": round(us, 2), "TFLOPS": round(tf, 1),
                                      "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4), "ref_b70_TFLOPS": ref_tf,
                                      "parity_bad": bad, "parity_rows": rows}
            del dA, dC, ws
        out[name] = e
        del W
        torch.cuda.empty_cache()
        progress(f"ref shape {name} K={K} N={N}: GEMV {e['gemv_m1']['us']} us, prefill {e['prefill_m1024']['us']} us")
    return out


def _rate(fn, sample_s):
    """Calls of fn in about sample_s seconds (at least one, after one untimed call)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= sample_s or n >= 10000:
            return n, el


def cpu_baseline(sample_s: float):
    """The reference's host golds (compiled from the reference sources into
    oracle/_ref; where that was not built, the oracle's restatement) timed on
    this machine's CPU cores, on all cores (OpenMP over outputs, as the golds
    are written) and on one core.  The headline is the decode GEMV gold
    (compute_gold + epilogue_ref postop 3) at M=1 K=4096 N=14336 bf16, about
    sample_s seconds per core count; the other configs about sample_s / 4 each:
      c1  M=1 K=N=4096 fp16 int2 gold, no epilogue (full);
      c3  int8 gold (compute_scale_a + the s8 x s2 gold) on 8 of the 1024 rows:
          the work is linear in the rows, so the rate is the full problem's;
      c4  BITCOS gold M=1 K=5376 N=21504 fp16 z=.5 (full);
      c5  the MoE prefill check's double-precision layer for 4 of the 2048
          tokens (the oracle's restatement of int2_moe/prefill.cpp:289-318;
          that driver is not compiled), rate per token."""
    from oracle import binding as orc
    from ternocl_amd import formats, synth
    ref = orc.ref_available()
    kind = "reference" if ref else "port"
    cores = orc.max_threads()
    g = synth.rng(7)
    # c2: the headline shape
    M, K, N = 1, 4096, 14336
    A, B, S = synth.activations(g, (M, K), True), synth.int2_weights(g, K, N), synth.scales(g, K, N, True)
    bias = formats.f32_to_dt(g.standard_normal(N).astype(np.float32) * np.float32(0.1), True)
    if ref:
        c2 = lambda: orc.ref_epilogue(orc.ref_int2_gold(A, B, S, M, K, N, True), None, bias, 3, False, True)
    else:
        c2 = lambda: orc.epilogue(orc.int2_gold(A, B, S, M, K, N, True), None, bias, 3, False, True)
    # c1
    A1, B1, S1 = synth.activations(g, (1, 4096), False), synth.int2_weights(g, 4096, 4096), synth.scales(g, 4096, 4096, False)
    c1 = (lambda: orc.ref_int2_gold(A1, B1, S1, 1, 4096, 4096, False)) if ref else \
         (lambda: orc.int2_gold(A1, B1, S1, 1, 4096, 4096, False))
    # c3: 8 rows of the M=1024 prefill
    r3, K3, N3 = 8, 4096, 14336
    A3, B3, S3 = synth.activations(g, (r3, K3), False), synth.int2_weights(g, K3, N3), synth.scales(g, K3, N3, False)
    if ref:
        c3 = lambda: orc.ref_int8_gold(A3, B3, orc.ref_scale_a(A3, r3, K3, False), S3, r3, K3, N3, False)
    else:
        c3 = lambda: orc.int8_gold(A3, B3, orc.scale_a(A3, r3, K3, False), S3, r3, K3, N3, False)
    # c4
    K4, N4 = 5376, 21504
    A4 = synth.activations(g, (1, K4), False)
    buf4, _ = synth.bitcos_weights(g, K4, N4, 0.5)
    S4 = synth.scales(g, K4, N4, False)
    c4 = (lambda: orc.ref_bitcos_gold(A4, buf4, S4, 1, K4, N4, False)) if ref else \
         (lambda: orc.bitcos_gold(A4, buf4, S4, 1, K4, N4, False))
    bytes4 = formats.bitcos_bytes(buf4) + K4 * 2 + N4 * 2 + (K4 // 128) * N4 * 2
    # c5: 4 tokens of the MoE layer
    Tk, E, topk, H, I, t5 = 2048, 64, 8, 2048, 1408, 4
    X5 = synth.activations(g, (t5, H), True)
    ids5, RW5 = synth.moe_routing(g, t5, E, topk, True)
    w5 = []
    for K_, N_ in ((H, I), (H, I), (I, H)):
        w5.append(np.stack([synth.int2_weights(g, K_, N_) for _ in range(E)]))
        w5.append(np.stack([synth.scales(g, K_, N_, True) for _ in range(E)]))
    c5 = lambda: orc.moe_ref_tokens(X5, ids5, RW5, 0, t5, topk, H, I, *w5, True)
    flops5 = 2.0 * t5 * topk * (2 * H * I + I * H)

    configs = [
        ("c2", c2, sample_s, gemv_bytes(M, K, N), 1e9, "GB/s", f"M=1 K={K} N={N} bf16 compute_gold + epilogue_ref postop 3"),
        ("c1", c1, sample_s / 4, 1 * 4096 * 2 + 4096 * 4096 / 4 + 4096 * 2 + 32 * 4096 * 2, 1e9, "GB/s",
         "M=1 K=N=4096 fp16 compute_gold"),
        ("c3", c3, sample_s / 4, 2.0 * r3 * N3 * K3, 1e12, "TOPS",
         f"compute_scale_a + int8 compute_gold on {r3} of the 1024 rows, K={K3} N={N3} fp16 (rate = full problem's)"),
        ("c4", c4, sample_s / 4, bytes4, 1e9, "GB/s", f"BITCOS compute_gold M=1 K={K4} N={N4} fp16 z=.5"),
        ("c5", c5, sample_s / 4, flops5, 1e12, "TFLOPS",
         f"MoE prefill check layer (double) for {t5} of {Tk} tokens, E={E} top-{topk} H={H} I={I} (oracle restatement)"),
    ]
    per = {}
    for name, fn, secs, work, scale, unit, what in configs:
        e = {"unit": unit, "sample": what}
        for tag, nth in (("all_cores", cores), ("one_core", 1)):
            orc.set_threads(nth)
            n, el = _rate(fn, secs if tag == "all_cores" else secs / 2)
            e[tag] = {"value": round(work * n / el / scale, 4), "cores": nth, "calls": n,
                      "ms_per_call": round(el / n * 1e3, 3)}
        per[name] = e
    orc.set_threads(cores)
    head = per["c2"]["all_cores"]
    return {"value": head["value"], "unit": "GB/s", "cores": cores, "kind": kind,
            "sample": f"{head['calls']} calls of the host gold (compute_gold + epilogue_ref postop 3) for "
                      f"M=1 K={K} N={N} bf16 ({head['ms_per_call']} ms/call), OpenMP over outputs",
            "one_core": per["c2"]["one_core"], "per_config": per}


def rotation(torch, tensors, set_bytes):
    """Copies of the device tensors making > 2 GiB of distinct weight sets."""
    sets = max(1, math.ceil(WEIGHT_ROTATION_BYTES / set_bytes))
    return sets, [[t.clone() for t in tensors] for _ in range(sets)]


def graph_time_us(torch, fn, n):
    """Duration of one fn() call from a HIP graph of n calls (warm replay, then the median of 3)."""
    g, s = graph_of(torch, fn, n)
    t, _ = median_replays(torch, g, s)
    return t / n * 1e6


def dev16(torch, a, bf16):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(
        torch.bfloat16 if bf16 else torch.float16)


def dev32(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).cuda()


def bench_c1(torch, T, synth, formats, orc):
    """int2 GEMV M=1 K=N=4096 fp16, no epilogue."""
    M, K, N, bf16 = 1, 4096, 4096, False
    g = synth.rng(11)
    A, B, S = synth.activations(g, (M, K), bf16), synth.int2_weights(g, K, N), synth.scales(g, K, N, bf16)
    dA = dev16(torch, A, bf16)
    sets, W = rotation(torch, [dev32(torch, B), dev16(torch, S, bf16)], B.nbytes + S.nbytes)
    dC = torch.empty((M, N), dtype=torch.float16, device="cuda")
    it = [0]

    def call():
        b, sc = W[it[0] % sets]
        it[0] += 1
        T.int2_fp16_upcvt_gemm(dA, b, sc, dC, None, None, M, N, K)
    call()
    torch.cuda.synchronize()
    got = formats.dt_to_f32(dC.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    want = formats.dt_to_f32(orc.epilogue(orc.int2_gold(A, B, S, M, K, N, bf16), None, None, 0, False, bf16), bf16)
    bad = int((np.abs(got - want) > 1e-3 + 1e-2 * np.abs(want)).sum())
    us = graph_time_us(torch, call, 400)
    nbytes = M * K * 2 + K * N / 4 + M * N * 2 + (K // 128) * N * 2
    return {"workload": "int2 GEMV M=1 K=4096 N=4096 fp16, no epilogue", "us": round(us, 3),
            "GB/s": round(nbytes / us / 1e3, 1), "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "bytes": int(nbytes), "weight_sets": sets, "parity_bad": bad}


def bench_c3(torch, T, synth, formats, orc):
    """int2 x int8 prefill M=1024 K=4096 N=14336 fp16: quant_a + s8 x s2 GEMM."""
    M, K, N, bf16 = 1024, 4096, 14336, False
    g = synth.rng(33)
    A, B, SB = synth.activations(g, (M, K), bf16), synth.int2_weights(g, K, N), synth.scales(g, K, N, bf16)
    dA = dev16(torch, A, bf16)
    sets, W = rotation(torch, [dev32(torch, B), dev16(torch, SB, bf16)], B.nbytes + SB.nbytes)
    dSA = torch.empty((K // 128, T.ldsa(M)), dtype=torch.float16, device="cuda")
    dAq = torch.empty((M, K), dtype=torch.int8, device="cuda")
    dC = torch.empty((M, N), dtype=torch.float16, device="cuda")
    it = [0]

    def call():
        b, sb = W[it[0] % sets]
        it[0] += 1
        T.quant_a(dA, dSA, dAq, M, K)
        T.int2_int8_gemm(None, dAq, dSA, b, sb, dC, None, None, M, N, K)

    def quant():
        T.quant_a(dA, dSA, dAq, M, K)

    def gemm():
        b, sb = W[it[0] % sets]
        it[0] += 1
        T.int2_int8_gemm(None, dAq, dSA, b, sb, dC, None, None, M, N, K)

    def upcvt():
        b, sb = W[it[0] % sets]
        it[0] += 1
        T.int2_fp16_upcvt_gemm(dA, b, sb, dC, None, None, M, N, K)
    call()
    torch.cuda.synchronize()
    rows = 8  # parity on the first rows (quantization and dots are per row)
    SA = orc.scale_a(A[:rows], rows, K, bf16)
    want = formats.dt_to_f32(orc.epilogue(orc.int8_gold(A[:rows], B, SA, SB, rows, K, N, bf16), None, None, 0,
                                          False, bf16), bf16)
    got = formats.dt_to_f32(dC[:rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    bad = int((np.abs(got - want) > 1e-3 + 1e-2 * np.abs(want)).sum())
    Aq_ok = bool(np.array_equal(dAq[:rows].cpu().numpy(), orc.quant_a(A[:rows], SA, rows, K, bf16)))
    # the fp16 upcvt GEMM on the same operands, checked on the same rows
    it[0] = 0
    upcvt()
    torch.cuda.synchronize()
    want_u = formats.dt_to_f32(orc.epilogue(orc.int2_gold(A[:rows], B, SB, rows, K, N, bf16), None, None, 0,
                                            False, bf16), bf16)
    got_u = formats.dt_to_f32(dC[:rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    bad_u = int((np.abs(got_u - want_u) > 1e-3 + 1e-2 * np.abs(want_u)).sum())
    us = graph_time_us(torch, call, 40)
    q_us = graph_time_us(torch, quant, 40)
    g_us = graph_time_us(torch, gemm, 40)
    u_us = graph_time_us(torch, upcvt, 20)
    ops = 2.0 * M * N * K
    tops = ops / us / 1e6
    return {"workload": "int2_via_int2_x_int8 prefill M=1024 K=4096 N=14336 fp16, quant_a + s8 x s2 GEMM",
            "value": round(tops, 1), "unit": "TOPS", "us": round(us, 2), "mfma_frac": round(tops / I8_PEAK_TOPS, 4),
            "peak": I8_PEAK_TOPS, "quant_us": round(q_us, 2), "gemm_us": round(g_us, 2),
            "gemm_TOPS": round(ops / g_us / 1e6, 1), "weight_sets": sets,
            "parity_bad": bad, "parity_rows": rows, "quant_bit_exact": Aq_ok,
            "upcvt_fp16_gemm": {"us": round(u_us, 2), "TFLOPS": round(ops / u_us / 1e6, 1),
                                "mfma_frac": round(ops / u_us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                "parity_bad": bad_u, "parity_rows": rows}}


def bench_c4(torch, T, synth, formats, orc):
    """FWHT (HB 512) + BITCOS GEMV M=1 K=5376 N=21504 fp16 at z = .3 / .5 / .7."""
    M, K, N, HB, bf16 = 1, 5376, 21504, 512, False
    out = {"workload": "sign flip + FWHT HB=512, then BITCOS GEMV M=1 K=5376 N=21504 fp16; us = the transform "
                       "fused into the GEMV launch, two_launch_us = FWHT and GEMV as two launches"}
    for z in (0.3, 0.5, 0.7):
        g = synth.rng(44 + int(10 * z))
        x = synth.activations(g, (M, K), bf16)
        buf, _ = synth.bitcos_weights(g, K, N, z)
        S = synth.scales(g, K, N, bf16)
        sgn = (g.integers(0, 2, K, dtype=np.int8) * 2 - 1).astype(np.int8)
        ls = T.bitcos_pick_ls(M, N, K)
        dx, ds = dev16(torch, x, bf16), torch.from_numpy(sgn).cuda()
        dy = torch.empty_like(dx)
        dB = dev32(torch, buf)
        dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
        T.bitcos_slice_ranks(dB, dSR, K, N, ls)
        sets, W = rotation(torch, [dB, dev16(torch, S, bf16), dSR], buf.nbytes + S.nbytes)
        dC = torch.empty((M, N), dtype=torch.float16, device="cuda")
        wsb = T.bitcos_gemv_ws_bytes(N, ls)  # the split launch's sums and strip counters
        dws = torch.zeros(max(wsb, 16), dtype=torch.uint8, device="cuda")
        it = [0]

        def fwht():
            T.hadamard_fwht(dx, ds, dy, M, K, HB, True)

        def gemv(ws=dws):
            b, sc, sr = W[it[0] % sets]
            it[0] += 1
            T.bitcos_fp16_upcvt_gemm(dy, b, sc, sr, dC, None, None, M, N, K, ls, ws=ws)

        def call():  # the two launches, as the reference runs them
            fwht()
            gemv()

        def fused():  # the transform inside the GEMV (ternocl_bitcos_fwht_gemm_ws)
            b, sc, sr = W[it[0] % sets]
            it[0] += 1
            T.bitcos_fwht_gemm(dx, ds, HB, b, sc, sr, dC, None, None, M, N, K, ls, ws=dws)
        call()
        torch.cuda.synchronize()
        y = orc.fwht(x, sgn, M, K, HB, True, bf16)
        fwht_ok = bool(np.array_equal(dy.view(torch.int16).cpu().numpy().view(np.uint16), y))
        want = formats.dt_to_f32(orc.epilogue(orc.bitcos_gold(y, buf, S, M, K, N, bf16), None, None, 0, False,
                                              bf16), bf16)
        got = formats.dt_to_f32(dC.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
        bad = int((np.abs(got - want) > 1e-3 + 1e-2 * np.abs(want)).sum())
        two = dC.clone()
        it[0] = 0
        fused()
        torch.cuda.synchronize()
        fused_same = bool(torch.equal(dC, two))
        us2 = graph_time_us(torch, call, 200)
        us = graph_time_us(torch, fused, 200)
        g_us = graph_time_us(torch, gemv, 200)
        g1_us = graph_time_us(torch, lambda: gemv(None), 200)  # one workgroup per strip
        f_us = graph_time_us(torch, fwht, 200)
        nbytes = M * K * 2 + buf.nbytes + S.nbytes + M * N * 2  # bitcos_fp16_upcvt/main.cpp:289-291
        out[f"z{z}"] = {"us": round(us, 2), "two_launch_us": round(us2, 2), "fused_bits_equal_two_launch": fused_same,
                        "gemv_us": round(g_us, 2), "gemv_unsplit_us": round(g1_us, 2),
                        "fwht_us": round(f_us, 2),
                        "gemv_GB/s": round(nbytes / g_us / 1e3, 1),
                        "gemv_hbm_frac": round(nbytes / g_us / 1e3 / HBM_PEAK_GBS, 4),
                        "pipeline_GB/s": round((nbytes + 2 * M * K * 2 + K) / us / 1e3, 1),
                        "bytes": int(nbytes), "ls": ls, "weight_sets": sets, "parity_bad": bad,
                        "fwht_bit_exact": fwht_ok}
        del W, dB, dSR
        torch.cuda.empty_cache()
    # the M-tiled BITCOS path (bitcos_fp16_upcvt_gemm_mt) at a prefill M: re-pack + int2 GEMM
    Mp, z = 1024, 0.5
    g = synth.rng(77)
    A = synth.activations(g, (Mp, K), bf16)
    buf, _ = synth.bitcos_weights(g, K, N, z)
    S = synth.scales(g, K, N, bf16)
    ls = T.bitcos_pick_ls(1, N, K)
    dA, dB, dS = dev16(torch, A, bf16), dev32(torch, buf), dev16(torch, S, bf16)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    ws = torch.empty(T.bitcos_gemm_mt_ws_bytes(K, N), dtype=torch.uint8, device="cuda")
    dC = torch.empty((Mp, N), dtype=torch.float16, device="cuda")
    dW2 = ws[T.WS_HEADER_BYTES:].view(torch.int32).view(K // 16, N)  # the re-packed words follow the header

    def mt():
        T.bitcos_fp16_upcvt_gemm_mt(dA, dB, dS, dSR, dC, None, None, Mp, N, K, ls, ws)

    def repack():
        T.bitcos_to_int2(dB, dSR, ls, dW2, K, N)
    mt()
    torch.cuda.synchronize()
    rows = 4
    want = formats.dt_to_f32(orc.epilogue(orc.bitcos_gold(A[:rows], buf, S, rows, K, N, bf16), None, None, 0,
                                          False, bf16), bf16)
    got = formats.dt_to_f32(dC[:rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    bad = int((np.abs(got - want) > 1e-3 + 1e-2 * np.abs(want)).sum())
    us = graph_time_us(torch, mt, 10)
    r_us = graph_time_us(torch, repack, 20)
    flops = 2.0 * Mp * N * K
    out["prefill_m1024_z0.5"] = {"workload": "bitcos_fp16_upcvt_gemm_mt M=1024 K=5376 N=21504 fp16 z=.5: "
                                             "re-pack to int2 + int2 prefill GEMM",
                                 "us": round(us, 2), "TFLOPS": round(flops / us / 1e6, 1),
                                 "mfma_frac": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                 "repack_us": round(r_us, 2), "parity_bad": bad, "parity_rows": rows}

    def mt_in_tile():  # the reference's call: no workspace, the tiles decode BITCOS
        T.bitcos_fp16_upcvt_gemm_mt(dA, dB, dS, dSR, dC, None, None, Mp, N, K, ls, None)
    mt_in_tile()
    torch.cuda.synchronize()
    got = formats.dt_to_f32(dC[:rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    bad = int((np.abs(got - want) > 1e-3 + 1e-2 * np.abs(want)).sum())
    us = graph_time_us(torch, mt_in_tile, 10)
    out["prefill_m1024_z0.5"]["in_tile"] = {"us": round(us, 2), "TFLOPS": round(flops / us / 1e6, 1),
                                            "mfma_frac": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                            "parity_bad": bad, "parity_rows": rows}
    return out


def bench_c5(torch, T, synth, formats, orc):
    """int2 MoE prefill layer: T=2048 E=64 top-8, H=2048 I=1408, bf16, uniform routing."""
    Tk, E, topk, H, I, bf16 = 2048, 64, 8, 2048, 1408, True
    g = synth.rng(55)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)

    def experts(K, N):
        return (np.stack([synth.int2_weights(g, K, N) for _ in range(E)]),
                np.stack([synth.scales(g, K, N, bf16) for _ in range(E)]))
    (Bg, Sg), (Bu, Su), (Bd, Sd) = experts(H, I), experts(H, I), experts(I, H)
    layer_bytes = sum(a.nbytes for a in (Bg, Sg, Bu, Su, Bd, Sd))
    sets, W = rotation(torch, [dev32(torch, Bg), dev16(torch, Sg, bf16), dev32(torch, Bu), dev16(torch, Su, bf16),
                               dev32(torch, Bd), dev16(torch, Sd, bf16)], layer_bytes)
    dX, dRW = dev16(torch, X, bf16), dev16(torch, RW, bf16)
    dids = torch.from_numpy(ids).cuda()
    dO = torch.empty((Tk, H), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(T.int2_moe_prefill_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")
    it = [0]

    def call():
        bg, sg, bu, su, bd, sd = W[it[0] % sets]
        it[0] += 1
        T.int2_moe_prefill(dX, dids, dRW, Tk, E, topk, H, I, bg, sg, bu, su, bd, sd, dO, ws)
    call()
    torch.cuda.synchronize()
    got = formats.dt_to_f32(dO.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    # the reference's double-precision check (int2_moe/prefill.cpp:288-319) on the first four
    # tokens (the first rows of the experts' first tiles), the last four (the ends of the
    # expert segments, in the last tiles) and eight random ones
    rs = np.random.default_rng(505)
    tok = [(0, 4), (Tk - 4, Tk)] + [(int(t), int(t) + 1) for t in sorted(rs.choice(np.arange(4, Tk - 4), 8, replace=False))]
    refs = [(t0, t1, orc.moe_ref_tokens(X, ids, RW, t0, t1, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16)) for t0, t1 in tok]

    def check(out):
        return max(float(np.abs(out[t0:t1] - r).max() / np.abs(r).max()) for t0, t1, r in refs)
    rel = check(got)
    us = graph_time_us(torch, call, 10)
    flops = 2.0 * Tk * topk * (2.0 * H * I + I * H)  # int2_moe/prefill.cpp:350
    tf = flops / us / 1e6
    # the same layer on the s8 x s2 GEMM (int2_moe_prefill_int8.cl, QMODE 1)
    ws8 = torch.empty(T.int2_moe_prefill_int8_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")

    def call8():
        bg, sg, bu, su, bd, sd = W[it[0] % sets]
        it[0] += 1
        T.int2_moe_prefill_int8(dX, dids, dRW, Tk, E, topk, H, I, bg, sg, bu, su, bd, sd, dO, ws8)
    call8()
    torch.cuda.synchronize()
    got8 = formats.dt_to_f32(dO.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    rel8 = check(got8)
    us8 = graph_time_us(torch, call8, 10)
    # the route alone at this layer's G and at a long prefill's (T = 32768 tokens, G = 262144,
    # where each route workgroup ranks its chunk in four passes), checked against the oracle
    route = {}
    for gT in (Tk, 32768):
        G = gT * topk
        rid = ids if gT == Tk else np.random.default_rng(506).integers(0, E, G, dtype=np.int32)
        drid = torch.from_numpy(rid).cuda()
        meta = torch.zeros(2 * E + 2, dtype=torch.int32, device="cuda")
        perm = torch.empty(G, dtype=torch.int32, device="cuda")
        inv = torch.empty(G, dtype=torch.int32, device="cuda")

        def rcall():
            T.int2_moe_route(drid, meta, perm, inv, G, E)
        rcall()
        torch.cuda.synchronize()
        m, pm, iv = orc.moe_route(rid, E, T.moe_tile_rows())
        exact = bool(np.array_equal(meta.cpu().numpy(), m) and np.array_equal(perm.cpu().numpy(), pm)
                     and np.array_equal(inv.cpu().numpy(), iv))
        route[f"G{G}"] = {"us": round(graph_time_us(torch, rcall, 20), 2), "exact": exact}
        if gT == Tk:
            # the combine alone on this layer's inv (Y: fp32 [G][H] as the down GEMM writes it)
            dY = torch.randn((G, H), dtype=torch.float32, device="cuda")

            def ccall():
                T.int2_moe_combine(dY, inv, dRW, dO, Tk, topk, H)
            combine_us = graph_time_us(torch, ccall, 20)
            del dY
    route_us = route[f"G{Tk * topk}"]["us"]
    # the reference reports each phase (int2_moe/prefill.cpp:323-350); here the layer is one
    # call, so its grouped GEMMs are the layer minus its route and combine, each timed alone
    phases = {"route_us": route_us, "combine_us": round(combine_us, 2),
              "gemm_us": round(us - route_us - combine_us, 2),
              "gemm_TFLOPS": round(flops / (us - route_us - combine_us) / 1e6, 1),
              "measured": "route and combine graph-timed alone; gemm_us = us - route_us - combine_us "
                          "(gate/up in one launch, then down)"}
    return {"workload": "int2 MoE prefill layer T=2048 E=64 top-8 H=2048 I=1408 bf16 (route, up, gate, down, combine)",
            "value": round(tf, 1), "unit": "TFLOPS", "us": round(us, 2), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
            "peak": BF16_PEAK_TFLOPS, "layers_rotated": sets, "layer_weight_bytes": int(layer_bytes),
            "check_tokens": [list(t[:2]) for t in refs], "check_rel_err": rel, "check_pass": rel < 1e-2,
            "int8": {"us": round(us8, 2), "TOPS": round(flops / us8 / 1e6, 1),
                     "mfma_frac": round(flops / us8 / 1e6 / I8_PEAK_TOPS, 4), "peak": I8_PEAK_TOPS,
                     "check_rel_err": rel8, "check_pass": rel8 < 5e-2},
            "phases": phases, "route": route}


def bench_c6(torch, T, synth, formats, orc):
    """int2 MoE decode layer at the reference driver's default problem (int2_moe/main.cpp:6):
    T=1 E=128 top-8, H=2048 I=768, bf16.  Rate = the weight bytes the layer must stream (the
    topk experts' gate, up and down B and S) / time; weight sets rotated past the caches like
    the reference's --sets."""
    Tk, E, topk, H, I, bf16 = 1, 128, 8, 2048, 768, True
    g = synth.rng(66)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)

    def experts(K, N):
        return (np.stack([synth.int2_weights(g, K, N) for _ in range(E)]),
                np.stack([synth.scales(g, K, N, bf16) for _ in range(E)]))
    (Bg, Sg), (Bu, Su), (Bd, Sd) = experts(H, I), experts(H, I), experts(I, H)
    layer_bytes = sum(a.nbytes for a in (Bg, Sg, Bu, Su, Bd, Sd))
    streamed = layer_bytes * len(np.unique(ids)) // E  # the distinct experts touched (int2_moe/main.cpp:322-328)
    sets, W = rotation(torch, [dev32(torch, Bg), dev16(torch, Sg, bf16), dev32(torch, Bu), dev16(torch, Su, bf16),
                               dev32(torch, Bd), dev16(torch, Sd, bf16)], layer_bytes)
    dX, dRW = dev16(torch, X, bf16), dev16(torch, RW, bf16)
    dids = torch.from_numpy(ids).cuda()
    dO = torch.empty((Tk, H), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(T.int2_moe_decode_ws_bytes(Tk, topk, H, I), dtype=torch.uint8, device="cuda")
    it = [0]

    def call():
        bg, sg, bu, su, bd, sd = W[it[0] % sets]
        it[0] += 1
        T.int2_moe_decode(dX, dids, dRW, Tk, E, topk, H, I, bg, sg, bu, su, bd, sd, dO, ws)
    call()
    torch.cuda.synchronize()
    got = formats.dt_to_f32(dO.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    ref = orc.moe_ref_tokens(X, ids, RW, 0, Tk, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16, round_up=False)
    rel = float(np.abs(got - ref).max() / np.abs(ref).max())
    us = graph_time_us(torch, call, 2 * sets)
    gbs = streamed / us / 1e3
    return {"workload": "int2 MoE decode layer T=1 E=128 top-8 H=2048 I=768 bf16 (gate/up, silu*up, down, combine)",
            "value": round(gbs, 1), "unit": "GB/s", "us": round(us, 2), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "streamed_weight_bytes": int(streamed), "layers_rotated": sets,
            "check_rel_err": rel, "check_pass": rel < 1e-2}


def bench_c7(torch, T, synth, formats, orc):
    """s8 x s2 decode GEMV (int2_int8_gemv, QMODE 0 and 1) at M=1 on the GEMV workload shapes,
    bf16, weight sets rotated: quant_a on its own and the GEMV, rates on the reference
    byte model with the int8 activations and their scales in place of the DT activations."""
    out = {}
    for i, (K, N) in enumerate(SHAPES):
        M, bf16 = 1, True
        g = synth.rng(700 + i)
        A = synth.activations(g, (M, K), bf16)
        B, SB = synth.int2_weights(g, K, N), synth.scales(g, K, N, bf16)
        set_bytes = B.nbytes + SB.nbytes
        sets, W = rotation(torch, [dev32(torch, B), dev16(torch, SB, bf16)], set_bytes)
        dA = dev16(torch, A, bf16)
        dSA = torch.empty((K // 128, T.ldsa(M)), dtype=torch.bfloat16, device="cuda")
        dAq = torch.empty((M, K), dtype=torch.int8, device="cuda")
        dC = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        T.quant_a(dA, dSA, dAq, M, K)
        wsb = T.int2_int8_gemm_ws_bytes(M, N, K)  # the K split's strip counters and slice sums
        ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda") if wsb else None
        it = [0]

        def upfront():
            b, sb = W[it[0] % sets]
            it[0] += 1
            T.int2_int8_gemm(None, dAq, dSA, b, sb, dC, None, None, M, N, K, ws=ws)

        def in_gemv():
            b, sb = W[it[0] % sets]
            it[0] += 1
            T.int2_int8_gemm(dA, None, dSA, b, sb, dC, None, None, M, N, K, ws=ws)
        upfront()
        torch.cuda.synchronize()
        want = orc.int8_gold(A, B, orc.scale_a(A, M, K, bf16), SB, M, K, N, bf16)
        got = formats.dt_to_f32(dC.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
        d = np.abs(got - want)
        bad = int((d > 1e-3 + 1e-2 * np.abs(want)).sum())
        q_us = graph_time_us(torch, lambda: T.quant_a(dA, dSA, None, M, K), 50)
        u_us = graph_time_us(torch, upfront, 2 * sets)
        i_us = graph_time_us(torch, in_gemv, 2 * sets)
        nbytes = M * K + (K // 128) * M * 2 + K * N / 4 + (K // 128) * N * 2 + M * N * 2
        out[f"m1_k{K}_n{N}"] = {"gemv_us": round(u_us, 2), "gemv_GB/s": round(nbytes / u_us / 1e3, 1),
                                "hbm_frac": round(nbytes / u_us / 1e3 / HBM_PEAK_GBS, 4),
                                "in_gemv_quant_us": round(i_us, 2), "quant_a_scales_only_us": round(q_us, 2),
                                "ws_bytes": wsb, "parity_bad": bad, "layers_rotated": sets}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-sample-s", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-sweep", action="store_true", help="skip the M = 2, 4, 8 sweep and the VALU and bf16-MFMA engines")
    ap.add_argument("--only-headline", action="store_true", help="skip the prefill, C1, C4 and C5 workloads")
    ap.add_argument("--no-ref-shapes", action="store_true",
                    help="skip the reference's 11 benchmark shapes (GEMV at M=1, prefill at M=1024)")
    ap.add_argument("--probe", type=int, default=0, metavar="N",
                    help="counter-collection mode for rocprofv3 --pmc: N eager launches per GEMV shape, "
                         "a 64 MiB device copy (the calibration kernel of known size), N calls each of the "
                         "int8 prefill (quant_a + s8 x s2 GEMM) and the fp16 upcvt prefill GEMM (M=1024 "
                         "K=4096 N=14336), of the BITCOS GEMV (K=5376 N=21504, z = .5; alone and with the "
                         "FWHT fused in), of the LM head GEMV (M=1 K=4096 N=151680) and of one MoE "
                         "prefill layer (T=2048 E=64 top-8 H=2048 I=1408); prints one line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Each GEMV would shard by output columns with no exchange; run --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import ternocl_amd as T
    from ternocl_amd import formats, synth
    from oracle import binding as orc
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    T.lib()

    sbs = [ShapeBench(torch, T, synth, formats, 1, K, N, 100 + i) for i, (K, N) in enumerate(SHAPES)]

    if args.probe:
        src = torch.ones(16 << 20, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.probe):
            for sb in sbs:
                sb.launch()
        for _ in range(4):  # an elementwise kernel reading 64 MiB and writing 64 MiB: the
            torch.add(src, 1, out=dst)  # calibration of the FETCH_SIZE / WRITE_SIZE counters
        del src, dst
        M, K, N = 1024, 4096, 14336  # the prefill workload, one weight set (counters, not timing)
        g = synth.rng(33)
        A, B, SB = synth.activations(g, (M, K), False), synth.int2_weights(g, K, N), synth.scales(g, K, N, False)
        dA, dB, dSB = dev16(torch, A, False), dev32(torch, B), dev16(torch, SB, False)
        dSA = torch.empty((K // 128, T.ldsa(M)), dtype=torch.float16, device="cuda")
        dAq = torch.empty((M, K), dtype=torch.int8, device="cuda")
        dC = torch.empty((M, N), dtype=torch.float16, device="cuda")
        for _ in range(args.probe):
            T.quant_a(dA, dSA, dAq, M, K)
            T.int2_int8_gemm(None, dAq, dSA, dB, dSB, dC, None, None, M, N, K)
        for _ in range(args.probe):  # the fp16 upcvt prefill GEMM on the same operands
            T.int2_fp16_upcvt_gemm(dA, dB, dSB, dC, None, None, M, N, K)
        del dA, dB, dSB, dSA, dAq, dC
        # BITCOS GEMV M=1 K=5376 N=21504 fp16 at z = .5, one weight set
        Kb, Nb = 5376, 21504
        g = synth.rng(49)
        x = dev16(torch, synth.activations(g, (1, Kb), False), False)
        buf, _ = synth.bitcos_weights(g, Kb, Nb, 0.5)
        dBc, dSc = dev32(torch, buf), dev16(torch, synth.scales(g, Kb, Nb, False), False)
        ls = T.bitcos_pick_ls(1, Nb, Kb)
        dSR = torch.zeros(max(ls - 1, 1) * Nb, dtype=torch.int32, device="cuda")
        T.bitcos_slice_ranks(dBc, dSR, Kb, Nb, ls)
        dCb = torch.empty((1, Nb), dtype=torch.float16, device="cuda")
        wsb = T.bitcos_gemv_ws_bytes(Nb, ls)  # the split launch, as the c4 leg runs it
        dws = torch.zeros(max(wsb, 16), dtype=torch.uint8, device="cuda")
        for _ in range(args.probe):
            T.bitcos_fp16_upcvt_gemm(x, dBc, dSc, dSR, dCb, None, None, 1, Nb, Kb, ls, ws=dws)
        sgn = torch.ones(Kb, dtype=torch.int8, device="cuda")
        for _ in range(args.probe):  # the same GEMV with the sign flip + FWHT (HB 512) fused in
            T.bitcos_fwht_gemm(x, sgn, 512, dBc, dSc, dSR, dCb, None, None, 1, Nb, Kb, ls, ws=dws)
        del x, dBc, dSc, dSR, dCb, dws, sgn
        # the reference's 8B LM head GEMV, M=1 K=4096 N=151680 fp16 (the multi-strip kernel)
        Kl, Nl = 4096, 151680
        g = synth.rng(901)
        xl = dev16(torch, synth.activations(g, (1, Kl), False), False)
        dBl, dSl = dev32(torch, synth.int2_weights(g, Kl, Nl)), dev16(torch, synth.scales(g, Kl, Nl, False), False)
        dCl = torch.empty((1, Nl), dtype=torch.float16, device="cuda")
        for _ in range(args.probe):
            T.int2_fp16_upcvt_gemm(xl, dBl, dSl, dCl, None, None, 1, Nl, Kl)
        del xl, dBl, dSl, dCl
        # one int2 MoE prefill layer, T=2048 E=64 top-8 H=2048 I=1408 bf16
        Tk, E, topk, H, I = 2048, 64, 8, 2048, 1408
        g = synth.rng(55)
        X = dev16(torch, synth.activations(g, (Tk, H), True), True)
        ids, RW = synth.moe_routing(g, Tk, E, topk, True)
        dids, dRW = torch.from_numpy(ids).cuda(), dev16(torch, RW, True)
        wts = []
        for K_, N_ in ((H, I), (H, I), (I, H)):
            wts.append(dev32(torch, np.stack([synth.int2_weights(g, K_, N_) for _ in range(E)])))
            wts.append(dev16(torch, np.stack([synth.scales(g, K_, N_, True) for _ in range(E)]), True))
        dO = torch.empty((Tk, H), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(T.int2_moe_prefill_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")
        for _ in range(args.probe):
            T.int2_moe_prefill(X, dids, dRW, Tk, E, topk, H, I, *wts, dO, ws)
        torch.cuda.synchronize()
        print(json.dumps({"probe": args.probe, "bytes_per_launch": {f"K{sb.K}_N{sb.N}": sb.bytes() for sb in sbs},
                          "copy_bytes": 64 << 20}), flush=True)
        return

    def step():
        for sb in sbs:
            sb.launch()

    # eager check of one call per shape against the oracle
    parity = []
    for sb in sbs:
        sb.launch()
    torch.cuda.synchronize()
    eager = [sb.output().copy() for sb in sbs]
    for sb in sbs:
        parity.append(check_parity(sb, orc, formats))

    # warm-up steps, then exactly K timed steps, each a graph replay; the K-step
    # graph is replayed REPEATS times and the median is the value
    gw, sw = graph_of(torch, step, max(args.warmup, 1))
    gt, st = graph_of(torch, step, args.steps)
    torch.cuda.synchronize()
    time_graph(torch, gw, sw)
    ts = [time_graph(torch, gt, st) for _ in range(REPEATS)]
    t = float(np.median(ts))
    replay_same = all(np.array_equal(sb.output(), e) for sb, e in zip(sbs, eager))
    progress(f"headline step timed: {t / args.steps * 1e6:.2f} us per step")
    step_bytes = sum(sb.bytes() for sb in sbs)
    value = step_bytes * args.steps / t / 1e9

    # per-shape launch durations (graph of that shape alone), and the same
    # kernel with the decode removed (the memory ceiling of its structure)
    shapes = {}
    tot_b, tot_t = 0.0, 0.0
    for sb, (bad, dmax) in zip(sbs, parity):
        us = per_launch_us(torch, sb, 200)
        gbs = sb.bytes() / (us * 1e-6) / 1e9
        tot_b += sb.bytes()
        tot_t += us
        c_us = ceiling_us(torch, T, sb)
        w_med, w_mean = wait_mode_us(torch, sb.launch)
        pr = plain_read_us(torch, T, sb.bytes())
        shapes[f"K{sb.K}_N{sb.N}"] = {"us_per_launch": round(us, 3), "GB/s": round(gbs, 1),
                                      "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": int(sb.bytes()),
                                      "decode_removed_us": round(c_us, 3),
                                      "of_decode_removed": round(c_us / us, 4),
                                      "plain_read_us": round(pr, 3), "of_plain_read": round(pr / us, 4),
                                      "wait_mode_us": {"median": round(w_med, 3), "mean": round(w_mean, 3),
                                                       "measured": "event pair + synchronize per launch"},
                                      "weight_sets": sb.sets, "parity_bad": bad, "max_abs_diff": dmax}
    isolated = tot_b / (tot_t * 1e-6) / 1e9
    progress("headline shapes: per-launch, decode-removed, wait-mode and plain-read times done")

    extra = {}
    if not args.no_sweep:
        sweep = {}
        for M in (2, 4, 8):
            for K, N in SHAPES:
                sb = ShapeBench(torch, T, synth, formats, M, K, N, 300 + M)
                us = per_launch_us(torch, sb, 100)
                sweep[f"M{M}_K{K}_N{N}"] = {"us": round(us, 3),
                                            "GB/s": round(sb.bytes() / (us * 1e-6) / 1e9, 1)}
                del sb
                torch.cuda.empty_cache()
        extra["m_sweep"] = sweep
        valu = {}
        for K, N in SHAPES:
            sb = ShapeBench(torch, T, synth, formats, 1, K, N, 500, tile=T.gemv_tile(T.VALU))
            us = per_launch_us(torch, sb, 100)
            valu[f"K{K}_N{N}"] = {"us": round(us, 3), "GB/s": round(sb.bytes() / (us * 1e-6) / 1e9, 1)}
            del sb
            torch.cuda.empty_cache()
        extra["valu_engine_m1"] = valu
        bf = {}
        for K, N in SHAPES:
            sb = ShapeBench(torch, T, synth, formats, 1, K, N, 600, tile=T.gemv_tile(T.MFMA))
            us = per_launch_us(torch, sb, 100)
            bf[f"K{K}_N{N}"] = {"us": round(us, 3), "GB/s": round(sb.bytes() / (us * 1e-6) / 1e9, 1)}
            del sb
            torch.cuda.empty_cache()
        extra["bf16_mfma_engine_m1"] = bf
        progress("M sweep and the other GEMV engines done")

    if not args.only_headline:
        for key, fn in (("prefill", bench_c3), ("c1", bench_c1), ("c4", bench_c4), ("c5", bench_c5),
                        ("c6", bench_c6), ("int8_gemv", bench_c7)):
            extra[key] = fn(torch, T, synth, formats, orc)
            torch.cuda.empty_cache()
            progress(f"{key} done")
    if not args.no_ref_shapes:
        extra["ref_shapes"] = bench_ref_shapes(torch, T, synth, formats, orc)
        torch.cuda.empty_cache()

    traffic = None
    tf = ROOT / "profiles" / "int2_gemv_m1_bf16_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_step")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations, int2 weights, fp32 accumulate",
        "data": "synthetic (seeded): A~N(0,1), ternary p=(.25,.5,.25), scales~U[.005,.02], "
                "bias~N(0,.1), residual~N(0,1); >2 GiB rotating weight sets per shape",
        "config": {"workload": "int2_fp16_upcvt decode GEMV, M=1, bf16, bias+residual epilogue, "
                               "step = (K=4096,N=14336) + (K=14336,N=4096)",
                   "M": 1, "shapes": [list(s) for s in SHAPES], "epilogue": "acc + bias[n] + residual",
                   "engine": "fp8 x fp4 block-scaled MFMA (engine 4)"},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "measured": "the timed step (value): algorithmic bytes of its two GEMV launches / "
                                 "their time, median of 3 replays of the K-step graph",
                     "isolated_per_shape": {"achieved": round(isolated, 1),
                                            "frac": round(isolated / HBM_PEAK_GBS, 4),
                                            "measured": "each shape's launches alone in a graph of 200"}},
        "repeats": {"n": REPEATS, "step_ms": [round(x / args.steps * 1e3, 5) for x in ts]},
        "shapes": shapes,
        "parity": {"ok": all(b == 0 for b, _ in parity) and replay_same,
                   "graph_replay_bit_identical": replay_same,
                   "rule": "|got-ref| <= 1e-3 + 1e-2|ref| vs the oracle"},
        **extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_sample_s)
        progress("cpu baseline done")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
