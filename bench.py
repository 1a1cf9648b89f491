#!/usr/bin/env python3
"""Benchmark of the quantized-dot hot path on one MI355X.

Workload "matvec": one routed-expert decode pass for one
token — Q8_K-quantize x[4096] -> IQ2_S gate matvec 1536x4096 -> Q8_K-quantize
h[1536] -> IQ3_S down matvec 4096x1536.  Weights are random-from-seed
(synthetic data, no checkpoint).  Inputs are resident in HBM before timing;
every step reads a different copy of the weights (> 512 MB of copies in
rotation, twice the 256 MB Infinity Cache) so the bytes come from HBM.
Launches are captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

Prints ONE JSON line (rank 0).  `value` = algorithmic bytes moved per step /
step time, in GB/s.  `roofline` reports the dominant kernel measured alone.
`cpu_baseline` times the oracle's AVX2 restatement of the reference CPU path on
this host's cores for a bounded sample of the same step.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "lightbridge-engine_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
HIDDEN, FFN = 4096, 1536
# Algorithmic bytes (weights + Q8_K activation + f32 output) per matvec.
GATE_BYTES = FFN * (HIDDEN // 256) * 82 + (HIDDEN // 256) * 292 + FFN * 4     # 2,026,048
DOWN_BYTES = HIDDEN * (FFN // 256) * 110 + (FFN // 256) * 292 + HIDDEN * 4     # 2,721,496
STEP_BYTES = GATE_BYTES + DOWN_BYTES


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=0, help="weight copies in rotation (0 = enough for 512 MB)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--lpu", type=int, default=0, help="lanes per (row, block) unit (0 = library default)")
    return ap.parse_args()


def cpu_baseline(w_gate, w_down, x, seconds: float):
    """Oracle AVX2 path (restating the reference's vec_dot_q8_k_cpu + rayon rows):
    the same step on host cores, bounded to ~`seconds` of work."""
    import numpy as np
    from oracle import lb_oracle as orc

    threads = min(orc.default_threads(), 16)
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, threads, True)
    mg = orc.make_matrix(22, FFN, HIDDEN, w_gate)
    md = orc.make_matrix(21, HIDDEN, FFN, w_down)
    h = np.random.default_rng(5).standard_normal(FFN).astype(np.float32)
    orc.gemv(ex, mg, x)
    n, t0 = 0, time.perf_counter()
    while True:
        orc.gemv(ex, mg, x)          # quantize x + gate rows
        orc.gemv(ex, md, h)          # quantize h + down rows
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 3:
            break
    gbs = STEP_BYTES * n / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} steps of the same workload (quantize+IQ2_S gate+quantize+IQ3_S down) in {el:.1f} s, "
                      f"oracle AVX2 restatement, {threads} threads of {os.cpu_count()} logical CPUs",
            "ms_per_step": round(el / n * 1e3, 4)}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build runs on a "
              f"single MI355X; see DESIGN.md for how the path shards)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import lbhip
    from lbhip import synth

    be = lbhip.HipBackend(0)
    be.set_tuning(be.TUNE_GEMV_LPU, args.lpu)
    w_gate = synth.random_matrix(synth.IQ2_S, FFN, HIDDEN, seed=101)
    w_down = synth.random_matrix(synth.IQ3_S, HIDDEN, FFN, seed=102)
    copies = args.copies or max(2, math.ceil(512e6 / (w_gate.nbytes + w_down.nbytes)) + 4)
    gate_dev = torch.from_numpy(w_gate.reshape(-1)).cuda()
    down_dev = torch.from_numpy(w_down.reshape(-1)).cuda()
    gates = [be.upload(synth.IQ2_S, FFN, HIDDEN, gate_dev) for _ in range(copies)]
    downs = [be.upload(synth.IQ3_S, HIDDEN, FFN, down_dev) for _ in range(copies)]
    del gate_dev, down_dev

    x = synth.random_activations(HIDDEN, seed=103)
    xs = torch.from_numpy(np.stack([synth.random_activations(HIDDEN, seed=200 + i) for i in range(copies)])).cuda()
    q8x = torch.zeros((copies, HIDDEN // 256 * 292), dtype=torch.uint8, device="cuda")
    hs = torch.zeros((copies, FFN), dtype=torch.float32, device="cuda")
    q8h = torch.zeros((copies, FFN // 256 * 292), dtype=torch.uint8, device="cuda")
    ys = torch.zeros((copies, HIDDEN), dtype=torch.float32, device="cuda")

    def step(i):
        c = i % copies
        be.gemv_f32(gates[c], xs[c], hs[c], q8x[c])      # Q8_K(x) + IQ2_S gate, one launch
        be.gemv_f32(downs[c], hs[c], ys[c], q8h[c])      # Q8_K(h) + IQ3_S down, one launch

    # Capture one rotation (copies steps) per graph; replay it.
    per_graph = copies
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        be.set_stream(stream)
        for i in range(per_graph):   # eager warm-up on the capture stream
            step(i)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(per_graph):
                step(i)
        # dominant kernel alone: the IQ3_S down matvec over every copy
        g_down = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_down, stream=stream):
            for i in range(per_graph):
                be.gemv_f32(downs[i], hs[i], ys[i])
        g_gate = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_gate, stream=stream):
            for i in range(per_graph):
                be.gemv_f32(gates[i], xs[i], hs[i])

        reps_w = max(1, args.warmup // per_graph)
        reps = max(1, math.ceil(args.steps / per_graph))
        for _ in range(reps_w):
            g.replay()
        stream.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(reps):
            g.replay()
        t1.record(stream)
        t1.synchronize()
        ms_total = t0.elapsed_time(t1)
        steps = reps * per_graph
        ms_per_step = ms_total / steps

        def kernel_avg_us(graph):
            graph.replay()
            stream.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            n_rep = max(1, 2000 // per_graph)
            e0.record(stream)
            for _ in range(n_rep):
                graph.replay()
            e1.record(stream)
            e1.synchronize()
            return e0.elapsed_time(e1) * 1e3 / (n_rep * per_graph)

        down_us = kernel_avg_us(g_down)
        gate_us = kernel_avg_us(g_gate)

    # parity spot check of the last step against the oracle (not timed)
    from oracle import lb_oracle as orc
    c = (steps - 1) % copies
    q8h_last = q8h[c].cpu().numpy()
    y_ref = orc.gemv_prequantized(orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, 8, True),
                                  orc.make_matrix(synth.IQ3_S, HIDDEN, FFN, w_down), q8h_last)
    parity = bool(np.array_equal(ys[c].cpu().numpy().view(np.uint32), y_ref.view(np.uint32)))

    value = STEP_BYTES / (ms_per_step * 1e-3) / 1e9
    down_gbs = DOWN_BYTES / (down_us * 1e-6) / 1e9
    line = {
        "metric": "quant matvec HBM GB/s (% of MI355X peak); MoE-block decode tokens/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * per_graph,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi8->i32, f32 fold",
        "data": "synthetic (random-from-seed weights and activations)",
        "config": {"workload": "configs[1]: IQ2_S gate 1536x4096 + IQ3_S down 4096x1536, batch 1 (1 token)",
                   "weight_copies_in_rotation": copies,
                   "rotation_bytes": copies * (w_gate.nbytes + w_down.nbytes),
                   "step": "Q8_K(x)+IQ2_S gate -> Q8_K(h)+IQ3_S down (2 fused kernels, HIP graph)", "lpu": args.lpu,
                   "algorithmic_bytes_per_step": STEP_BYTES},
        "roofline": {"bound": "hbm", "kernel": "k_gemv<IQ3_S, fused Q8_K> (down 4096x1536)",
                     "achieved": round(down_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(down_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "avg_launch_us": round(down_us, 3), "algorithmic_bytes_per_launch": DOWN_BYTES},
        "kernels_us": {"iq2s_gate": round(gate_us, 3), "iq3s_down": round(down_us, 3)},
        "parity_last_step_bit_exact": parity,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(w_gate, w_down, x, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
