#!/usr/bin/env python3
"""Benchmark of the MI355X ternary GEMV (the int2 decode path), one JSON line.

Workload (the decode GEMV sweep): int2 upcvt GEMV, bf16 activations ~N(0,1),
ternary weights p(-1,0,+1) = (.25,.5,.25) packed 2 bits/weight, per-128-group
bf16 scales ~U[.005,.02], fused bias add (bias ~N(0,0.1)) + residual add
(residual ~N(0,1)), shapes (K=4096, N=14336) and (K=14336, N=4096), M = 1.
A step = one GEMV per shape.  Every call reads its own weight set out of a
rotation of distinct sets totalling > 2 GiB per shape (the reference's
cache-defeat rule, int2_fp16_upcvt/main.cpp:218-228), so weights stream from
HBM, not from the 256 MB Infinity Cache.

Timing: the W warm-up steps and then exactly K timed steps are captured in HIP
graphs (so host launch overhead stays off the GPU timeline) and replayed on one
stream between HIP events, after a device synchronize; the per-shape launch
duration comes from a graph of that shape's launches alone.  Bytes follow the
reference byte model (int2_fp16_upcvt/main.cpp:331-333): A + B + S + C + Other
+ Bias.  Also reported: M = 2, 4, 8 of the sweep, the VALU engine, and the
reference's own host gold (compiled from its sources into oracle/_ref) timed on
this machine's CPU cores as the cpu_baseline.
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
        self.next = 0

    def launch(self):
        s = self.next % self.sets
        self.next += 1
        self.T.int2_fp16_upcvt_gemm(self.dA, self.dB[s], self.dS[s], self.dC, self.dO, self.dBias,
                                    self.M, self.N, self.K, POSTOP_BIAS_RESIDUAL, False, tile=self.tile)

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


def per_launch_us(torch, sb, n):
    """Average duration of one launch of this shape (graph of n launches)."""
    g, s = graph_of(torch, sb.launch, n)
    time_graph(torch, g, s)  # warm replay
    t = time_graph(torch, g, s)
    return t / n * 1e6


def check_parity(sb, orc, formats):
    """Set 0 output against the oracle (bias + residual epilogue, bf16)."""
    acc = orc.int2_gold(sb.A, sb.B, sb.S, sb.M, sb.K, sb.N, True)
    want = formats.dt_to_f32(orc.epilogue(acc, sb.other, sb.bias, POSTOP_BIAS_RESIDUAL, False, True), True)
    got = formats.dt_to_f32(sb.output(), True)
    d = np.abs(got - want)
    bad = int((d > 1e-3 + 1e-2 * np.abs(want)).sum())
    return bad, float(d.max())


def cpu_baseline(sample_s: float):
    """The reference's host gold (compute_gold + epilogue_ref, compiled from the
    reference sources into oracle/_ref) or, where that was not built, the
    oracle's restatement of it, timed on this machine's CPU cores on the
    (K=4096, N=14336) M = 1 shape, repeated for about sample_s seconds."""
    from oracle import binding as orc
    from ternocl_amd import formats, synth
    M, K, N = 1, 4096, 14336
    g = synth.rng(7)
    A = synth.activations(g, (M, K), True)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, True)
    bias = formats.f32_to_dt(g.standard_normal(N).astype(np.float32) * np.float32(0.1), True)
    kind = "reference" if orc.ref_available() else "port"
    if kind == "reference":
        gold = lambda: orc.ref_epilogue(orc.ref_int2_gold(A, B, S, M, K, N, True), None, bias, 3, False, True)
    else:
        gold = lambda: orc.epilogue(orc.int2_gold(A, B, S, M, K, N, True), None, bias, 3, False, True)
    gold()
    n, t0 = 0, time.perf_counter()
    while True:
        gold()
        n += 1
        el = time.perf_counter() - t0
        if el >= sample_s or n >= 10000:
            break
    per = el / n
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    return {"value": round(gemv_bytes(M, K, N) / per / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": kind,
            "sample": f"{n} calls of the host gold (compute_gold + epilogue_ref postop 3) for "
                      f"M=1 K={K} N={N} bf16 in {el:.1f} s ({per * 1e3:.2f} ms/call), OpenMP over outputs"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-sample-s", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-sweep", action="store_true", help="skip the M = 2, 4, 8 sweep")
    ap.add_argument("--probe", type=int, default=0, metavar="N",
                    help="counter-collection mode for rocprofv3 --pmc: N eager launches per shape plus "
                         "a 64 MiB device copy (the calibration kernel of known size); prints one line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
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

    # warm-up steps, then exactly K timed steps, each a graph replay
    gw, sw = graph_of(torch, step, max(args.warmup, 1))
    gt, st = graph_of(torch, step, args.steps)
    torch.cuda.synchronize()
    time_graph(torch, gw, sw)
    t = time_graph(torch, gt, st)
    replay_same = all(np.array_equal(sb.output(), e) for sb, e in zip(sbs, eager))
    step_bytes = sum(sb.bytes() for sb in sbs)
    value = step_bytes * args.steps / t / 1e9

    # per-shape launch durations (graph of that shape alone)
    shapes = {}
    tot_b, tot_t = 0.0, 0.0
    for sb, (bad, dmax) in zip(sbs, parity):
        us = per_launch_us(torch, sb, 200)
        gbs = sb.bytes() / (us * 1e-6) / 1e9
        tot_b += sb.bytes()
        tot_t += us
        shapes[f"K{sb.K}_N{sb.N}"] = {"us_per_launch": round(us, 3), "GB/s": round(gbs, 1),
                                      "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": int(sb.bytes()),
                                      "weight_sets": sb.sets, "parity_bad": bad, "max_abs_diff": dmax}
    achieved = tot_b / (tot_t * 1e-6) / 1e9

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

    traffic = None
    tf = ROOT / "profiles" / "int2_gemv_m1_bf16_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_step")

    line = {
        "metric": "GEMV weight-stream GB/s (%HBM peak) at M=1",
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
                   "engine": "mfma"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "shapes": shapes,
        "parity": {"ok": all(b == 0 for b, _ in parity) and replay_same,
                   "graph_replay_bit_identical": replay_same,
                   "rule": "|got-ref| <= 1e-3 + 1e-2|ref| vs the oracle"},
        **extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_sample_s)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
