#!/usr/bin/env python3
"""Benchmark of the quantized-dot hot path on one MI355X.

Headline workload: one routed expert's decode pass for
one token -- Q8_K(x[4096]) + IQ2_S gate matvec 1536x4096, then Q8_K(h[1536]) +
IQ3_S down matvec 4096x1536, each a single fused kernel.  `value` is the
algorithmic bytes of that step (weights + Q8_K activations + f32 outputs)
divided by the step time, in GB/s.

Secondary workloads in the same JSON line:
  configs[0]  Q4_K x Q8_K matvec 4096x4096 (the reference's CPU-runnable case);
  model_matvecs  the same fused matvec at the Hy3 model's attention, dense-FFN and
              output-head shapes (up to the 340 MB Q5_K output head);
  configs[2]  the full MoE FFN block of one token: 192 routed experts (IQ2_S
              gate/up 1536x4096, IQ3_S down 4096x1536), top-8 of an F32 4096x192
              router with softmax weights, a Q4_K/Q5_K shared expert with ffn
              4096; reported with the routing given (moe_routed_by_id_into's
              boundary) and with the device router in the step.

Weights are random-from-seed (synthetic; no checkpoint).  Inputs are resident
in HBM before timing; launches are captured in HIP graphs and replayed; every
matvec step reads a different copy of the weights (> 512 MB in rotation, twice
the 256 MB Infinity Cache) and the MoE steps cycle through 1.3 GB of experts,
so weight bytes come from HBM.  `roofline` is the dominant kernel of the
headline step, timed alone with HIP events on the stream it runs on.
`cpu_baseline` times the CPU oracle (a C restatement of the reference's AVX2
path, rows over a thread pool as the reference's rayon pool) on this host for a
bounded sample of the same work.
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
HIDDEN, FFN, N_EXPERTS, TOP_K = 4096, 1536, 192, 8
Q8 = lambda k: k // 256 * 292  # noqa: E731
GATE_BYTES = FFN * (HIDDEN // 256) * 82 + Q8(HIDDEN) + FFN * 4          # 2,026,048
DOWN_BYTES = HIDDEN * (FFN // 256) * 110 + Q8(FFN) + HIDDEN * 4         # 2,721,496
STEP_BYTES = GATE_BYTES + DOWN_BYTES
Q4K_BYTES = HIDDEN * (HIDDEN // 256) * 144 + Q8(HIDDEN) + HIDDEN * 4    # 9,458,240
MOE_WEIGHT_BYTES = (TOP_K * (2 * FFN * 16 * 82 + HIDDEN * 6 * 110) + 2 * HIDDEN * 16 * 144
                    + HIDDEN * 16 * 176 + N_EXPERTS * HIDDEN * 4)      # 87,425,024 per token
EXPERT_BYTES = 2 * FFN * 16 * 82 + HIDDEN * 6 * 110                    # 6,733,824 per routed expert
SHARED_BYTES = 2 * HIDDEN * 16 * 144 + HIDDEN * 16 * 176               # 30,408,704
BATCH_TOKENS = 64
COLD_COPIES = 8
# Bytes per launch (read from beyond L2 + written) measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over `bench.py --pmc-workloads`, each scaled by the same counter's reading for a plain
# copy of known size (profiles/pmc_hot_kernels_traffic_and_valu.md).
MEASURED_TRAFFIC = {"gate": 2363569 + 6144, "down": 2987388 + 19648, "prefill": 193234918 + 25644960}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="timed steps of the headline workload")
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--moe-tokens", type=int, default=256, help="timed tokens of the MoE block workloads")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE block workload")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="bound on each CPU baseline sample")
    ap.add_argument("--lpu", type=int, default=0, help="matvec lanes per (row, block) unit (0 = library default)")
    ap.add_argument("--batch-reps", type=int, default=8, help="timed replays of the 8-step configs[3] graph")
    ap.add_argument("--stream-tokens", type=int, default=48,
                    help="tokens of the expert-streaming leg (sidecar -> HBM cache); 0 skips it")
    ap.add_argument("--pmc-workloads", action="store_true",
                    help="run a few dispatches of each workload for rocprofv3 --pmc passes and exit")
    return ap.parse_args()


class Timer:
    """HIP-graph replay timing on one stream (events recorded on that stream)."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def graph(self, fn):
        torch, s = self.torch, self.stream
        with torch.cuda.stream(s):
            fn()
            s.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                fn()
        return g

    def time(self, g, reps):
        torch, s = self.torch, self.stream
        with torch.cuda.stream(s):
            g.replay()
            s.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
            e1.synchronize()
        return e0.elapsed_time(e1) * 1e-3   # seconds

    def spread(self, g, replays, per):
        """Median, p10 and p90 in us per unit over `replays` replays, each bracketed by its own
        event pair on the stream (one replay = `per` units: steps, launches or tokens)."""
        torch, s = self.torch, self.stream
        with torch.cuda.stream(s):
            g.replay()
            s.synchronize()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(replays)]
            for a, b in ev:
                a.record(s)
                g.replay()
                b.record(s)
            ev[-1][1].synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 / per for a, b in ev)
        q = lambda f: us[min(len(us) - 1, int(round(f * (len(us) - 1))))]  # noqa: E731
        return {"median_us": round(q(0.5), 3), "p10_us": round(q(0.1), 3), "p90_us": round(q(0.9), 3),
                "replays": replays, "units_per_replay": per}


def logical_cpus():
    """Logical CPUs this process may run on (the box's share, not the machine's count)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_threads():
    """recommended_thread_count (crates/bridge-kernels-cpu/src/lib.rs:121-126): ceil(logical / 2)."""
    return max(1, (logical_cpus() + 1) // 2)


def host_cpu():
    """lscpu-style facts of the host the CPU baselines ran on: model name, physical
    cores (distinct (package, core) pairs among the CPUs this process may use) and
    logical CPUs."""
    model, cores = "unknown", set()
    allowed = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else None
    try:
        cpu, phys = None, None
        for line in Path("/proc/cpuinfo").read_text().splitlines() + [""]:
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                cpu = int(v)
            elif k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id" and cpu is not None and (allowed is None or cpu in allowed):
                cores.add((phys, v))
    except OSError:
        pass
    return {"cpu_model": model, "physical_cores": len(cores) or None, "logical_cpus": logical_cpus()}


def _cpu_fields(threads):
    d = {"threads": threads}
    d.update(host_cpu())
    d["cores"] = min(threads, d["physical_cores"] or threads)
    d["cores_note"] = ("physical cores the timed threads can occupy: min(threads, physical cores in this "
                       "process's CPU affinity); threads are not pinned")
    return d


def cpu_matvec_step(w_gate, w_down, seconds, threads=None):
    """Oracle AVX2 path for the headline step: gemv_into (quantize + row dots) of
    the gate, then of the down projection on its output."""
    import numpy as np
    from oracle import lb_oracle as orc
    threads = threads or cpu_threads()
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, threads, True)
    mg = orc.make_matrix(22, FFN, HIDDEN, w_gate)
    md = orc.make_matrix(21, HIDDEN, FFN, w_down)
    x = np.random.default_rng(5).standard_normal(HIDDEN).astype(np.float32)
    h = orc.gemv(ex, mg, x)
    n, t0 = 0, time.perf_counter()
    while True:
        h = orc.gemv(ex, mg, x)
        orc.gemv(ex, md, h)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 3) or el >= 4 * seconds:
            break
    return {"value": round(STEP_BYTES * n / el / 1e9, 3), "unit": "GB/s", **_cpu_fields(threads), "kind": "port",
            "ms_per_step": round(el / n * 1e3, 4),
            "sample": f"{n} steps of the headline step (Q8_K + IQ2_S gate 1536x4096, Q8_K + IQ3_S down "
                      f"4096x1536) in {el:.2f} s; oracle AVX2 restatement, rows over {threads} threads "
                      f"of {logical_cpus()} logical CPUs"}


def cpu_q4k(w, seconds):
    import numpy as np
    from oracle import lb_oracle as orc
    threads = cpu_threads()
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, threads, True)
    m = orc.make_matrix(12, HIDDEN, HIDDEN, w)
    x = np.random.default_rng(6).standard_normal(HIDDEN).astype(np.float32)
    orc.gemv(ex, m, x)
    n, t0 = 0, time.perf_counter()
    while True:
        orc.gemv(ex, m, x)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 3) or el >= 4 * seconds:
            break
    return {"value": round(Q4K_BYTES * n / el / 1e9, 3), "unit": "GB/s", **_cpu_fields(threads), "kind": "port",
            "sample": f"{n} Q4_K 4096x4096 gemv_into calls in {el:.2f} s, {threads} threads"}


def cpu_moe(experts_np, shared_np, router_w, xs, seconds):
    """Oracle MoE block per token: router logits + softmax top-8, then
    moe_routed_by_id_into with its preflight pass (the reference's structure) and
    the single-pass variant."""
    import numpy as np
    from oracle import lb_oracle as orc
    threads = cpu_threads()
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, threads, True)
    orc_exp, orc_sh = _oracle_layer(experts_np, shared_np)
    out = {}
    for preflight in (True, False):
        n, t0 = 0, time.perf_counter()
        while True:
            x = xs[n % len(xs)]
            ids, coefs = orc.route_softmax_topk(orc.router_logits_f32(router_w, x), TOP_K)
            orc.moe_routed_by_id(ex, ids, coefs, orc_exp, orc_sh, x, preflight=preflight)
            n += 1
            el = time.perf_counter() - t0
            if (el >= seconds / 2 and n >= 2) or el >= 2 * seconds:
                break
        out["preflight" if preflight else "single_pass"] = (n / el, n, el)
    best = max(v[0] for v in out.values())
    return {"value": round(best, 3), "unit": "tokens/s", **_cpu_fields(threads), "kind": "port",
            "faithful_with_preflight_tokens_per_s": round(out["preflight"][0], 3),
            "single_pass_tokens_per_s": round(out["single_pass"][0], 3),
            "sample": f"{out['preflight'][1]} + {out['single_pass'][1]} tokens through the 192-expert block "
                      f"(router + top-8 + experts + shared) in {out['preflight'][2] + out['single_pass'][2]:.2f} s, "
                      f"{threads} threads; value is the faster (single-pass) variant"}


def empty_kernel_us(be, timer):
    """Launch floor: one empty kernel per graph node, averaged over 400 nodes."""
    g = timer.graph(lambda: [be.empty_kernel() for _ in range(400)])
    timer.time(g, 2)
    return timer.time(g, 20) / (20 * 400) * 1e6


def read_floor_us(be, timer, torch, mats, nbytes):
    """Memory floor of a matvec: the fastest plain read of its weight bytes (16-byte non-temporal
    loads, every lane's loads issued before any is used) over a sweep of launch shapes, each
    timed in the same rotation of weight copies as the matvec.  Returns (us, shape)."""
    cus = be.cu_count()
    sink = torch.zeros(4 * be.READ_MAX_GRID, dtype=torch.int32, device="cuda")
    best = (float("inf"), None)
    copies = len(mats)
    reps = max(2, min(100, int(0.05 / (copies * nbytes / 5e12))))
    for unroll in (1, 4, 8):
        fit = max(1, min(be.READ_MAX_GRID, math.ceil(nbytes / (4096 * unroll))))
        for grid in sorted({fit, cus, 2 * cus, 4 * cus, 8 * cus}):
            if grid > fit:
                continue
            for slab in (False, True):
                g = timer.graph(lambda: [be.read_matrix(m, sink, grid, unroll, slab) for m in mats])
                timer.time(g, 1)
                us = timer.time(g, reps) / (reps * copies) * 1e6
                if us < best[0]:
                    best = (us, {"grid": grid, "loads_per_lane_in_flight": unroll, "slab": slab})
                del g
    return best


def floor_fields(kernel_us, empty_us, read):
    """Floors beside a kernel time: frac_of_floor = best plain read / kernel time."""
    return {"empty_kernel_us": round(empty_us, 3), "read_floor_us": round(read[0], 3),
            "read_floor_shape": read[1], "frac_of_floor": round(read[0] / kernel_us, 4)}


def bench_matvec_step(args, be, timer, torch, np, synth):
    w_gate = synth.random_matrix(synth.IQ2_S, FFN, HIDDEN, seed=101)
    w_down = synth.random_matrix(synth.IQ3_S, HIDDEN, FFN, seed=102)
    copies = max(2, math.ceil(512e6 / (w_gate.nbytes + w_down.nbytes)) + 4)
    gate_dev = torch.from_numpy(w_gate.reshape(-1)).cuda()
    down_dev = torch.from_numpy(w_down.reshape(-1)).cuda()
    gates = [be.upload(synth.IQ2_S, FFN, HIDDEN, gate_dev) for _ in range(copies)]
    downs = [be.upload(synth.IQ3_S, HIDDEN, FFN, down_dev) for _ in range(copies)]
    del gate_dev, down_dev
    xs = torch.from_numpy(np.stack([synth.random_activations(HIDDEN, seed=200 + i) for i in range(copies)])).cuda()
    q8x = torch.zeros((copies, Q8(HIDDEN)), dtype=torch.uint8, device="cuda")
    hs = torch.zeros((copies, FFN), dtype=torch.float32, device="cuda")
    q8h = torch.zeros((copies, Q8(FFN)), dtype=torch.uint8, device="cuda")
    ys = torch.zeros((copies, HIDDEN), dtype=torch.float32, device="cuda")

    def step_all():
        for c in range(copies):
            be.gemv_f32(gates[c], xs[c], hs[c], q8x[c])      # Q8_K(x) + IQ2_S gate, one launch
            be.gemv_f32(downs[c], hs[c], ys[c], q8h[c])      # Q8_K(h) + IQ3_S down, one launch

    g = timer.graph(step_all)
    reps_w = max(1, args.warmup // copies)
    reps = max(1, math.ceil(args.steps / copies))
    timer.time(g, reps_w)
    t = timer.time(g, reps)
    steps = reps * copies
    ms_per_step = t / steps * 1e3
    step_spread = timer.spread(g, 100, copies)
    g_gate = timer.graph(lambda: [be.gemv_f32(gates[c], xs[c], hs[c]) for c in range(copies)])
    g_down = timer.graph(lambda: [be.gemv_f32(downs[c], hs[c], ys[c]) for c in range(copies)])
    n_k = max(1, 2000 // copies)
    gate_us = timer.time(g_gate, n_k) / (n_k * copies) * 1e6
    down_us = timer.time(g_down, n_k) / (n_k * copies) * 1e6
    kernel_spread = {"iq2s_gate": timer.spread(g_gate, 100, copies), "iq3s_down": timer.spread(g_down, 100, copies)}
    del g, g_gate, g_down
    empty_us = empty_kernel_us(be, timer)
    gate_floor = read_floor_us(be, timer, torch, gates, w_gate.nbytes)
    down_floor = read_floor_us(be, timer, torch, downs, w_down.nbytes)

    c = (steps - 1) % copies
    torch.cuda.synchronize()
    check = (q8h[c].cpu().numpy(), ys[c].cpu().numpy())
    for m in gates + downs:
        m.close()
    return dict(w_gate=w_gate, w_down=w_down, copies=copies, steps=steps, warmup=reps_w * copies,
                ms_per_step=ms_per_step, gate_us=gate_us, down_us=down_us, check=check, empty_us=empty_us,
                gate_floor=gate_floor, down_floor=down_floor, step_spread=step_spread, kernel_spread=kernel_spread)


def bench_q4k(args, be, timer, torch, np, synth):
    w = synth.random_matrix(synth.Q4_K, HIDDEN, HIDDEN, seed=111)
    copies = math.ceil(600e6 / w.nbytes)
    wd = torch.from_numpy(w.reshape(-1)).cuda()
    ms = [be.upload(synth.Q4_K, HIDDEN, HIDDEN, wd) for _ in range(copies)]
    del wd
    xs = torch.randn(copies, HIDDEN, device="cuda")
    ys = torch.zeros(copies, HIDDEN, device="cuda")
    g = timer.graph(lambda: [be.gemv_f32(ms[c], xs[c], ys[c]) for c in range(copies)])
    timer.time(g, 3)
    reps = max(3, 1000 // copies)
    us = timer.time(g, reps) / (reps * copies) * 1e6
    spread = timer.spread(g, 100, copies)
    del g
    floors = floor_fields(us, empty_kernel_us(be, timer), read_floor_us(be, timer, torch, ms, w.nbytes))
    for m in ms:
        m.close()
    return w, {"workload": "configs[0]: Q4_K x Q8_K matvec 4096x4096, batch 1 (fused Q8_K + matvec kernel)",
               "us_per_matvec": round(us, 3), "GB/s": round(Q4K_BYTES / us / 1e3, 2),
               "roofline_frac": round(Q4K_BYTES / us / 1e3 / HBM_PEAK_GBS, 4), "weight_copies": copies,
               "per_replay_spread": spread, **floors}


# Decode matvecs of the Hy3 model's own tensors (crates/bridge-model-hy3/src/schema.rs:96-201,
# sizes from profile.rs:17-44): (name, type, rows, K).
MODEL_SHAPES = [("attn_q IQ2_S 8192x4096", 22, 8192, 4096), ("attn_k IQ2_S 1024x4096", 22, 1024, 4096),
                ("attn_v Q4_K 1024x4096", 12, 1024, 4096), ("attn_output IQ3_S 4096x8192", 21, 4096, 8192),
                ("dense_gate IQ2_S 13312x4096", 22, 13312, 4096), ("dense_down IQ3_S 4096x13312", 21, 4096, 13312),
                ("output Q5_K 120832x4096", 13, 120832, 4096)]


def bench_model_shapes(args, be, timer, torch, np, synth):
    """One fused Q8_K + matvec launch per shape, > 600 MB of weight copies in rotation."""
    out = {}
    empty_us = empty_kernel_us(be, timer)
    for name, ty, rows, k in MODEL_SHAPES:
        w = synth.random_matrix(ty, rows, k, seed=rows + k)
        copies = max(2, math.ceil(600e6 / w.nbytes))
        wd = torch.from_numpy(w.reshape(-1)).cuda()
        ms = [be.upload(ty, rows, k, wd) for _ in range(copies)]
        del wd
        xs = torch.randn(copies, k, device="cuda")
        ys = torch.zeros(copies, rows, device="cuda")
        g = timer.graph(lambda: [be.gemv_f32(ms[c], xs[c], ys[c]) for c in range(copies)])
        reps = max(3, min(400, int(0.25 / (copies * w.nbytes / 5e12))))
        timer.time(g, 2)
        us = timer.time(g, reps) / (reps * copies) * 1e6
        del g
        alg = w.nbytes + Q8(k) + 4 * rows
        out[name] = {"us": round(us, 3), "algorithmic_bytes": alg, "GB/s": round(alg / us / 1e3, 1),
                     "roofline_frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4), "weight_copies": copies,
                     **floor_fields(us, empty_us, read_floor_us(be, timer, torch, ms, w.nbytes))}
        for m in ms:
            m.close()
        del ms, xs, ys
        torch.cuda.empty_cache()
    return out


def bench_moe(args, be, timer, torch, np, synth, lbhip):
    # 192 experts, every matrix random from its own seed.
    experts_np = [(synth.random_matrix(synth.IQ2_S, FFN, HIDDEN, 3000 + 3 * e),
                   synth.random_matrix(synth.IQ2_S, FFN, HIDDEN, 3001 + 3 * e),
                   synth.random_matrix(synth.IQ3_S, HIDDEN, FFN, 3002 + 3 * e)) for e in range(N_EXPERTS)]
    experts = [(be.upload(synth.IQ2_S, FFN, HIDDEN, g), be.upload(synth.IQ2_S, FFN, HIDDEN, u),
                be.upload(synth.IQ3_S, HIDDEN, FFN, d)) for g, u, d in experts_np]
    shared_np = (synth.random_matrix(synth.Q4_K, HIDDEN, HIDDEN, 304), synth.random_matrix(synth.Q4_K, HIDDEN, HIDDEN, 305),
                 synth.random_matrix(synth.Q5_K, HIDDEN, HIDDEN, 306))
    shared = (be.upload(synth.Q4_K, HIDDEN, HIDDEN, shared_np[0]), be.upload(synth.Q4_K, HIDDEN, HIDDEN, shared_np[1]),
              be.upload(synth.Q5_K, HIDDEN, HIDDEN, shared_np[2]))
    moe = be.moe_create(experts, shared)
    router_w = synth.router_weights(N_EXPERTS, HIDDEN, 307)
    router = lbhip.Router(be, router_w)
    T = args.moe_tokens
    xs_np = [synth.random_activations(HIDDEN, seed=400 + i) for i in range(T)]
    xs = torch.from_numpy(np.stack(xs_np)).cuda()
    ys = torch.zeros(T, HIDDEN, device="cuda")
    routes = [router.route_into(xs[i], TOP_K) for i in range(T)]   # device router, before timing
    hit = len({int(e) for r in routes for e in r[0]})

    g_host = timer.graph(lambda: [be.moe_forward(moe, routes[i][0], routes[i][1], xs[i], ys[i]) for i in range(T)])
    timer.time(g_host, 1)
    reps = 3
    us_host = timer.time(g_host, reps) / (reps * T) * 1e6
    g_dev = timer.graph(lambda: [lbhip.moe_block_forward(be, moe, router, xs[i], ys[i], TOP_K) for i in range(T)])
    timer.time(g_dev, 1)
    us_dev = timer.time(g_dev, reps) / (reps * T) * 1e6
    spread_host, spread_dev = timer.spread(g_host, 11, T), timer.spread(g_dev, 11, T)
    del g_host, g_dev

    # Cold figure: token i reads shared expert and router copy i % COLD_COPIES
    # (8 x 33.5 MB in rotation, beyond the 256 MB Infinity Cache), so neither is
    # served from a cache that a single copy re-read every token would hit.
    cold_layers = [(be.moe_create(experts, tuple(be.upload(ty, HIDDEN, HIDDEN, w)
                                                 for ty, w in zip((synth.Q4_K, synth.Q4_K, synth.Q5_K), shared_np))),
                    lbhip.Router(be, router_w)) for _ in range(COLD_COPIES)]
    cold = lambda i: cold_layers[i % COLD_COPIES]  # noqa: E731
    g_host_c = timer.graph(lambda: [be.moe_forward(cold(i)[0], routes[i][0], routes[i][1], xs[i], ys[i])
                                    for i in range(T)])
    timer.time(g_host_c, 1)
    us_host_c = timer.time(g_host_c, reps) / (reps * T) * 1e6
    g_dev_c = timer.graph(lambda: [lbhip.moe_block_forward(be, cold(i)[0], cold(i)[1], xs[i], ys[i], TOP_K)
                                   for i in range(T)])
    timer.time(g_dev_c, 1)
    us_dev_c = timer.time(g_dev_c, reps) / (reps * T) * 1e6
    del g_host_c, g_dev_c
    torch.cuda.synchronize()
    for layer, r in cold_layers:
        shared_c = layer._keep[1]
        layer.close()
        r.close()
        for m in shared_c:
            m.close()

    torch.cuda.synchronize()
    host = lambda t: t.cpu().numpy()  # noqa: E731
    res = {"workload": "configs[2]: MoE FFN block, 1 token: 192 experts (IQ2_S gate/up 1536x4096, IQ3_S down "
                       "4096x1536), top-8 softmax of an F32 4096x192 router, Q4_K/Q5_K shared expert ffn 4096",
           "tokens_timed": T * reps, "distinct_experts_hit": hit,
           "routing_given": {"us_per_token": round(us_host, 2), "tokens_per_s": round(1e6 / us_host, 1),
                             "GB/s": round((MOE_WEIGHT_BYTES - N_EXPERTS * HIDDEN * 4) / us_host / 1e3, 1),
                             "per_replay_spread": spread_host},
           "with_device_router": {"us_per_token": round(us_dev, 2), "tokens_per_s": round(1e6 / us_dev, 1),
                                  "GB/s": round(MOE_WEIGHT_BYTES / us_dev / 1e3, 1),
                                  "per_replay_spread": spread_dev},
           "cold_shared_and_router": {
               "what": f"token i reads shared-expert and router copy i % {COLD_COPIES} "
                       f"({COLD_COPIES} x {(SHARED_BYTES + N_EXPERTS * HIDDEN * 4) / 1e6:.1f} MB in rotation); "
                       "the figures above re-read one copy every token",
               "routing_given_us_per_token": round(us_host_c, 2),
               "routing_given_GB/s": round((MOE_WEIGHT_BYTES - N_EXPERTS * HIDDEN * 4) / us_host_c / 1e3, 1),
               "with_device_router_us_per_token": round(us_dev_c, 2),
               "with_device_router_GB/s": round(MOE_WEIGHT_BYTES / us_dev_c / 1e3, 1),
               "with_device_router_roofline_frac": round(MOE_WEIGHT_BYTES / us_dev_c / 1e3 / HBM_PEAK_GBS, 4)},
           "algorithmic_weight_bytes_per_token": MOE_WEIGHT_BYTES}
    state = dict(experts_np=experts_np, shared_np=shared_np, router_w=router_w, xs_np=xs_np,
                 last_y=host(ys[T - 1]), moe=moe, router=router, experts=experts, shared=shared)
    return res, state


def bench_batch(args, be, timer, torch, np, synth, state):
    """64 tokens per step, each token's top-8 from seeded Zipf(1.1)
    router logits (softmax top-8 selected on the device), grouped per-expert decode
    after the device token-by-expert sort, on the same 192-expert layer."""
    T, R = BATCH_TOKENS, 8
    moe = state["moe"]
    moe.reserve_batch(T, TOP_K)
    logits = torch.from_numpy(np.stack([synth.zipf_routes(T, N_EXPERTS, TOP_K, 1.1, seed=500 + r)
                                        for r in range(R)])).cuda()
    xs = torch.from_numpy(np.stack([np.stack([synth.random_activations(HIDDEN, seed=600 + 64 * r + t)
                                              for t in range(T)]) for r in range(R)])).cuda()
    ids = torch.zeros((R, T, TOP_K), dtype=torch.int32, device="cuda")
    coefs = torch.zeros((R, T, TOP_K), dtype=torch.float32, device="cuda")
    ys = torch.zeros((R, T, HIDDEN), dtype=torch.float32, device="cuda")

    def step(r):
        be.route_experts_batch(logits[r], TOP_K, ids[r], coefs[r])
        be.moe_forward_batch(moe, ids[r], coefs[r], xs[r], ys[r])

    reps = max(2, args.batch_reps)

    def timed():
        g = timer.graph(lambda: [step(r) for r in range(R)])
        timer.time(g, 2)
        t_us = timer.time(g, reps) / (reps * R) * 1e6
        sp = timer.spread(g, 20, R)
        del g
        return t_us, sp

    # The layer's matrices as uploaded, then with the 16-row tile copies of every
    # routed expert that the matrix-core streams read (lbh_moe_make_batch_tile_copies).
    us_plain, _ = timed()
    moe.make_batch_tile_copies()
    tile_bytes = moe.batch_tile_copy_bytes
    us, spread = timed()
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy().view(np.uint32)
    hits = [len(np.unique(ids_h[r])) for r in range(R)]
    u = float(np.mean(hits))
    bytes_step = u * EXPERT_BYTES + SHARED_BYTES + T * (2 * HIDDEN * 4 + N_EXPERTS * 4)
    res = {"workload": "configs[3]: batched decode, 64 tokens: the configs[2] MoE block, per-token top-8 of seeded "
                       "Zipf(s=1.1) router logits (softmax top-8 on the device), token-by-expert sort, grouped "
                       "per-expert gate/up + SwiGLU + down, ordered combine",
           "tokens_per_step": T, "steps_timed": reps * R, "us_per_step": round(us, 2), "per_replay_spread": spread,
           "tokens_per_s": round(T / us * 1e6, 1),
           "us_per_step_without_tile_copies": round(us_plain, 2),
           "tile_copy_hbm_bytes": int(tile_bytes),
           "distinct_experts_hit_per_step": hits,
           "algorithmic_bytes_per_step": int(bytes_step),
           "GB/s": round(bytes_step / us / 1e3, 1), "roofline_frac": round(bytes_step / us / 1e3 / HBM_PEAK_GBS, 4),
           "note": "the 33.5 MB shared expert is read once per step (K-quant GEMM on the f16 matrix cores); routed "
                   "experts once per chunk of up to 16 tokens, chunks of 4+ tokens on the f16 matrix cores (exact "
                   "integer block sums), smaller ones on the VALU integer dots; us_per_step is timed with a second "
                   "copy of every routed expert's matrices with the 16 rows of each block adjacent (read by the "
                   "matrix-core streams only; tile_copy_hbm_bytes of HBM), us_per_step_without_tile_copies on the "
                   "matrices as uploaded"}
    check = dict(ids=ids_h[0].copy(), coefs=coefs[0].cpu().numpy(), xs=xs[0].cpu().numpy(), ys=ys[0].cpu().numpy())
    moe.make_batch_tile_copies([])
    return res, check


def bench_streaming(args, be, torch, np, synth, lbhip, state):
    """configs[2] decode with the routed experts streamed through the HBM expert
    cache from an expert-major sidecar file (the reference runtime's streaming
    MoE, crates/bridge-runtime/src/hy3_scalar.rs:561-626): per token, lease the
    8 routed experts (a miss reads the record from the sidecar into pinned
    staging, DMAs and repacks it on the copy stream), queue the leased forward,
    release.  Wall clock over the tokens, host work and PCIe included."""
    import shutil
    import tempfile

    from lbhip import sidecar as sc
    from lbhip.cache import CachedMoeLayer, ExpertCache

    tmp = Path(tempfile.mkdtemp(prefix="lbh_sidecar_"))
    try:
        names = ("IQ2_S", "IQ2_S", "IQ3_S")
        sc.write_sidecar(tmp / "experts.sidecar", tmp / "experts.json",
                         [(sc.ExpertKey(1, e), tuple(m.reshape(-1) for m in state["experts_np"][e]), names)
                          for e in range(N_EXPERTS)], sc.FUSED_GATE_UP, 4096)
        side = sc.Sidecar(tmp / "experts.sidecar", tmp / "experts.json")
        logits = synth.zipf_routes(args.stream_tokens, N_EXPERTS, TOP_K, 1.1, seed=909)
        routes = [np.sort(np.argsort(-logits[t], kind="stable")[:TOP_K]).astype(np.uint32)
                  for t in range(args.stream_tokens)]
        coefs = np.full(TOP_K, 1.0 / TOP_K, np.float32)
        xs = torch.from_numpy(np.stack([synth.random_activations(HIDDEN, seed=950 + t)
                                        for t in range(args.stream_tokens)])).cuda()
        ys = torch.zeros(args.stream_tokens, HIDDEN, device="cuda")
        out = {"workload": "configs[2] MoE block decode with the 192 routed experts streamed from an expert-major "
                           "sidecar file through the HBM expert cache (Zipf(s=1.1) top-8 routes)",
               "sidecar_bytes": side.manifest.sidecar["length"]}
        for name, entries, admit, warm in (("cold_8_entries", 8, 1, False), ("zipf_32_entries", 32, 2, False),
                                           ("warm_all_resident", N_EXPERTS, 1, True)):
            cache = ExpertCache(be, entries * EXPERT_BYTES, admit, HIDDEN, FFN, synth.IQ2_S, synth.IQ3_S)
            layer = CachedMoeLayer(be, cache, state["shared"])
            load = lambda e: (lambda dst: side.read_into(sc.ExpertKey(1, e), dst))  # noqa: E731
            if warm:
                for e in range(N_EXPERTS):
                    cache.get_or_try_insert(sc.ExpertKey(1, e), load(e), into=True).release()
            torch.cuda.synchronize()
            s0 = cache.stats()
            t0 = time.perf_counter()
            for t, ids in enumerate(routes):
                leases = [cache.get_or_try_insert(sc.ExpertKey(1, int(e)), load(int(e)), into=True) for e in ids]
                layer.forward_leased(leases, coefs, xs[t], ys[t])
                for lease in leases:
                    lease.release()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            s1 = cache.stats()
            hits, misses = s1["hits"] - s0["hits"], s1["misses"] - s0["misses"]
            up = s1["bytes_uploaded"] - s0["bytes_uploaded"]
            out[name] = {"cache_entries": entries, "admit_after_requests": admit, "tokens": len(routes),
                         "ms_per_token": round(dt / len(routes) * 1e3, 3), "tokens_per_s": round(len(routes) / dt, 1),
                         "hit_rate": round(hits / max(1, hits + misses), 3), "bytes_uploaded": up,
                         "upload_GB/s": round(up / dt / 1e9, 2)}
            layer.close()
            cache.close()
        side.close()
        return out
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def bench_ingest(args, be, torch, np, synth, lbhip):
    """GGUF payload ingestion straight to HBM (crates/bridge-gguf/src/reader.rs:194-341 locates the
    tensor; the bytes go to the device without a whole-file host copy): the
    Hy3 output head (Q5_K 120832x4096, 340 MB) in a GGUF file (page cache),
    located by the directory reader and streamed through pinned 32 MiB chunks
    with lbh_matrix_create_streamed, against lbh_matrix_create from host memory."""
    import shutil
    import tempfile

    from lbhip import gguf as gg
    rows, k = 120832, HIDDEN
    w = synth.random_matrix(synth.Q5_K, rows, k, seed=77)
    tmp = Path(tempfile.mkdtemp(prefix="lbh_gguf_"))
    try:
        path = tmp / "head.gguf"
        gg.write_gguf(path, [("general.architecture", gg.STRING, "hy3")],
                      [("output.weight", (k, rows), synth.Q5_K, w.tobytes())], alignment=4096)
        gg.ingest(be, path)["output.weight"].close()   # warm the page cache and the code paths
        t0 = time.perf_counter()
        m = gg.ingest(be, path)["output.weight"]
        t_stream = time.perf_counter() - t0
        exact = bool(np.array_equal(m.read_ggml(), w.reshape(-1)))
        m.close()
        t0 = time.perf_counter()
        m2 = be.upload(synth.Q5_K, rows, k, w)
        t_host = time.perf_counter() - t0
        m2.close()
        return {"workload": "GGUF ingestion: Q5_K output head 120832x4096 (340 MB) from a GGUF file in the page "
                            "cache to HBM (directory parse, positioned reads into pinned chunks, DMA, repack)",
                "bytes": int(w.nbytes), "streamed_s": round(t_stream, 4),
                "streamed_GB/s": round(w.nbytes / t_stream / 1e9, 2),
                "from_host_memory_s": round(t_host, 4), "from_host_memory_GB/s": round(w.nbytes / t_host / 1e9, 2),
                "read_back_bit_exact": exact}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def cpu_batch(experts_np, shared_np, check, seconds):
    """Oracle per token (the reference's token-serial loop) over the configs[3]
    batch's tokens and routes: moe_routed_by_id_into single pass."""
    import numpy as np
    from oracle import lb_oracle as orc
    threads = cpu_threads()
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, threads, True)
    orc_exp, orc_sh = _oracle_layer(experts_np, shared_np)
    n, t0 = 0, time.perf_counter()
    while True:
        t = n % BATCH_TOKENS
        orc.moe_routed_by_id(ex, check["ids"][t], check["coefs"][t], orc_exp, orc_sh, check["xs"][t], preflight=False)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or el >= 2 * seconds:
            break
    return {"value": round(n / el, 3), "unit": "tokens/s", **_cpu_fields(threads), "kind": "port",
            "sample": f"{n} tokens of the configs[3] batch (its Zipf routes) through moe_routed_by_id_into, single "
                      f"pass, one token at a time as the reference decodes, in {el:.2f} s, {threads} threads"}


def _oracle_layer(experts_np, shared_np):
    from oracle import lb_oracle as orc
    orc_exp = [orc.make_expert(orc.make_matrix(22, FFN, HIDDEN, g), orc.make_matrix(22, FFN, HIDDEN, u),
                               orc.make_matrix(21, HIDDEN, FFN, d)) for g, u, d in experts_np]
    sg, su, sd = shared_np
    orc_sh = orc.make_expert(orc.make_matrix(12, HIDDEN, HIDDEN, sg), orc.make_matrix(12, HIDDEN, HIDDEN, su),
                             orc.make_matrix(13, HIDDEN, HIDDEN, sd))
    return orc_exp, orc_sh


def _prefill_parity(check):
    import numpy as np
    from oracle import lb_oracle as orc
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, cpu_threads(), True)
    om = orc.make_matrix(13, PF_ROWS, HIDDEN, check["w"])
    return all(bool(np.array_equal(check["y"][t].view(np.uint32), orc.gemv_prequantized(ex, om, check["q8"][t]).view(np.uint32)))
               for t in range(8))


def cpu_parity(mv, moe_state, batch_check):
    """Spot checks of the timed GPU outputs against the CPU oracle (not timed)."""
    import numpy as np
    from oracle import lb_oracle as orc
    same = lambda a, b: bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))  # noqa: E731
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, cpu_threads(), True)
    q8h, y = mv["check"]
    out = {"configs[1]_last_step": same(y, orc.gemv_prequantized(ex, orc.make_matrix(21, HIDDEN, FFN, mv["w_down"]),
                                                                  q8h))}
    if moe_state is not None:
        orc_exp, orc_sh = _oracle_layer(moe_state["experts_np"], moe_state["shared_np"])
        x = moe_state["xs_np"][-1]
        ids, coefs = orc.route_softmax_topk(orc.router_logits_f32(moe_state["router_w"], x), TOP_K)
        out["configs[2]_last_token"] = same(moe_state["last_y"],
                                             orc.moe_routed_by_id(ex, ids, coefs, orc_exp, orc_sh, x))
        if batch_check is not None:
            bc = batch_check
            ok = True
            for t in range(0, BATCH_TOKENS, 9):
                want = orc.moe_routed_by_id(ex, bc["ids"][t], bc["coefs"][t], orc_exp, orc_sh, bc["xs"][t],
                                            preflight=False)
                ok = ok and same(bc["ys"][t], want)
            out["configs[3]_tokens_0_9_18_.._63"] = ok
    return out


PF_TOKENS, PF_ROWS = 512, 12288
PF_OPS = 2 * PF_TOKENS * PF_ROWS * HIDDEN                                 # 51,539,607,552
PF_BYTES = PF_ROWS * 16 * 176 + PF_TOKENS * Q8(HIDDEN) + PF_TOKENS * PF_ROWS * 4   # 62,160,896
MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense f16 matrix-core peak (the GEMM's instruction)
MFMA_I8_PEAK_TOPS = 5000.0      # MI355X dense int8 matrix-core peak (the roofline the i8 path is priced on)


def bench_prefill(args, be, timer, torch, np, synth):
    """Q8_K activations [512 x 4096] x Q5_K [12288 x 4096] -> f32
    [512 x 12288] on the f16 matrix cores with exact integer sums (lbh_gemm_q8_k: activation
    tiles + GEMM)."""
    w = synth.random_matrix(synth.Q5_K, PF_ROWS, HIDDEN, seed=801)
    copies = 4   # 4 x (34.6 MB packed + 110.1 MB MFMA-ready) in rotation: > the 256 MB Infinity Cache
    wd = torch.from_numpy(w.reshape(-1)).cuda()
    ms = [be.upload(synth.Q5_K, PF_ROWS, HIDDEN, wd) for _ in range(copies)]
    for m in ms:
        m.prepare_gemm()
    del wd
    x = torch.from_numpy(np.random.default_rng(802).standard_normal((PF_TOKENS, HIDDEN)).astype(np.float32)).cuda()
    q8 = torch.zeros((PF_TOKENS, Q8(HIDDEN)), dtype=torch.uint8, device="cuda")
    be.quantize_q8_k_rows(x, q8, PF_TOKENS, HIDDEN)
    ws = torch.zeros(be.gemm_workspace_bytes(PF_TOKENS, HIDDEN), dtype=torch.uint8, device="cuda")
    ys = torch.zeros((copies, PF_TOKENS, PF_ROWS), dtype=torch.float32, device="cuda")
    g = timer.graph(lambda: [be.gemm_q8_k(ms[c], q8, PF_TOKENS, ys[c], ws) for c in range(copies)])
    # Warm-up of 20 replays (80 calls, ~15 ms): the first ~10 ms of sustained matrix-core work run
    # ~10% slower (measured: 195 us per call after 2 warm-up replays, 178 us after 20, unchanged from
    # there up to 100), so the timed replays start in the steady state.
    timer.time(g, 20)
    reps = 30
    us = timer.time(g, reps) / (reps * copies) * 1e6
    spread = timer.spread(g, 50, copies)
    torch.cuda.synchronize()
    tops = PF_OPS / us / 1e6
    footprint = ms[0].device_bytes
    res = {"workload": "configs[4]: prefill 512 tokens, Q8_K activations [512 x 4096] x Q5_K [12288 x 4096] -> f32 "
                       "[512 x 12288], f16 MFMA (v_mfma_f32_32x32x16_f16) on integer operands: exact "
                       "per-(block, lane residue) sums",
           "us_per_step": round(us, 2), "calls_timed": reps * copies, "warmup_calls": 20 * copies,
           "per_replay_spread": spread, "dot_TOPS": round(tops, 2),
           "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": MFMA_I8_PEAK_TOPS, "unit": "TOP/s",
                        "frac": round(tops / MFMA_I8_PEAK_TOPS, 4), "traffic": MEASURED_TRAFFIC["prefill"],
                        "peak_note": "priced on the dense int8 peak (5.0 POP/s) of the integer contraction; the "
                                     "kernel issues f16 MFMA on exact small-integer operands (measured faster than "
                                     "the i8 instruction at this shape), whose own peak is 2.5 PFLOP/s",
                        "frac_of_f16_instruction_peak": round(tops / MFMA_F16_PEAK_TFLOPS, 4)},
           "hbm_GB/s_algorithmic": round(PF_BYTES / us / 1e3, 1),
           "prepared_matrix_hbm_bytes": {"total": footprint, "packed": ms[0].nbytes,
                                         "mfma_ready_copy": footprint - ms[0].nbytes,
                                         "vs_ggml_bytes": round(footprint / (PF_ROWS * HIDDEN // 256 * 176), 2)},
           "note": "the exact per-block f32 folds (9 chains x 16 blocks per output, separately rounded) run on the "
                   "VALU at ~20 ops per (row, token, block); they and the LDS operand reads bound the kernel, not "
                   "the matrix cores or HBM"}
    check = dict(w=w, q8=q8[:8].cpu().numpy(), y=ys[copies - 1, :8].cpu().numpy())
    for m in ms:
        m.close()
    return res, check


def cpu_prefill(check, seconds):
    """Oracle per-row dots (the reference's only path: vec_dot_q8_k row by row,
    token by token) for a bounded sample of the prefill's tokens."""
    import numpy as np
    from oracle import lb_oracle as orc
    threads = cpu_threads()
    ex = orc.make_exec(orc.MODE_CPU_PARALLEL_Q8K, threads, True)
    om = orc.make_matrix(13, PF_ROWS, HIDDEN, check["w"])
    n, t0 = 0, time.perf_counter()
    while True:
        orc.gemv_prequantized(ex, om, check["q8"][n % 8])
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or el >= 2 * seconds:
            break
    ops = 2.0 * PF_ROWS * HIDDEN * n
    return {"value": round(ops / el / 1e12, 5), "unit": "TOP/s", **_cpu_fields(threads), "kind": "port",
            "sample": f"{n} tokens x 12288 rows of Q5_K dots (gemv over pre-quantized Q8_K) in {el:.2f} s, "
                      f"{threads} threads; the full 512-token step would take {512 * el / n:.2f} s"}


def _progress(msg):
    """One line on stderr per finished leg (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def pmc_workloads():
    """A few dispatches of every hot-path kernel at the bench shapes, for the
    rocprofv3 --pmc passes (one counter set per run), plus a plain 64 MiB copy
    that calibrates FETCH_SIZE / WRITE_SIZE."""
    import torch
    import lbhip
    from lbhip import synth
    be = lbhip.HipBackend(0)
    H, F = HIDDEN, FFN
    # calibration copy: 64 MiB read + 64 MiB written
    a = torch.empty(64 << 20, dtype=torch.uint8, device='cuda').fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    # configs[1] matvecs on distinct weight copies
    wg = torch.from_numpy(synth.random_matrix(22, F, H, 101).reshape(-1)).cuda()
    wd = torch.from_numpy(synth.random_matrix(21, H, F, 102).reshape(-1)).cuda()
    gates = [be.upload(22, F, H, wg) for _ in range(16)]
    downs = [be.upload(21, H, F, wd) for _ in range(16)]
    x = torch.randn(H, device='cuda'); h = torch.zeros(F, device='cuda'); y = torch.zeros(H, device='cuda')
    torch.cuda.synchronize()
    for c in range(16):
        be.gemv_f32(gates[c], x, h)
        be.gemv_f32(downs[c], h, y)
    torch.cuda.synchronize()
    # the Hy3 dense FFN matvecs (IQ2_S gate 13312x4096, IQ3_S down 4096x13312), 4 copies each
    for ty, rows, k, seed in ((22, 13312, H, 121), (21, H, 13312, 122)):
        wl = torch.from_numpy(synth.random_matrix(ty, rows, k, seed).reshape(-1)).cuda()
        ml = [be.upload(ty, rows, k, wl) for _ in range(4)]
        xl, yl = torch.randn(k, device='cuda'), torch.zeros(rows, device='cuda')
        torch.cuda.synchronize()
        for c in range(4):
            be.gemv_f32(ml[c], xl, yl)
        torch.cuda.synchronize()
        for m_ in ml:
            m_.close()
        del wl, ml
    # configs[0] Q4_K matvec
    wq = torch.from_numpy(synth.random_matrix(12, H, H, 111).reshape(-1)).cuda()
    qs = [be.upload(12, H, H, wq) for _ in range(8)]
    torch.cuda.synchronize()
    for c in range(8):
        be.gemv_f32(qs[c], x, y)
    torch.cuda.synchronize()
    # configs[2] MoE block (48 experts, top-8) and configs[3] batch
    NE = 48
    wu = torch.from_numpy(synth.random_matrix(22, F, H, 103).reshape(-1)).cuda()
    experts = [(be.upload(22, F, H, torch.roll(wg, 82 * e)), be.upload(22, F, H, torch.roll(wu, 82 * e)),
                be.upload(21, H, F, torch.roll(wd, 110 * e))) for e in range(NE)]
    shared = (be.upload(12, H, H, synth.random_matrix(12, H, H, 304)), be.upload(12, H, H, synth.random_matrix(12, H, H, 305)),
              be.upload(13, H, H, synth.random_matrix(13, H, H, 306)))
    moe = be.moe_create(experts, shared)
    router = lbhip.Router(be, synth.router_weights(NE, H, 307))
    xs = torch.randn(8, H, device='cuda'); ys = torch.zeros(8, H, device='cuda')
    torch.cuda.synchronize()
    for t in range(8):
        lbhip.moe_block_forward(be, moe, router, xs[t], ys[t], 8)
    torch.cuda.synchronize()
    moe.reserve_batch(64, 8)
    logits = torch.from_numpy(synth.zipf_routes(64, NE, 8, 1.1, seed=500)).cuda()
    ids = torch.zeros((64, 8), dtype=torch.int32, device='cuda'); coefs = torch.zeros((64, 8), device='cuda')
    xb = torch.randn(64, H, device='cuda'); yb = torch.zeros(64, H, device='cuda')
    for _ in range(2):
        be.route_experts_batch(logits, 8, ids, coefs)
        be.moe_forward_batch(moe, ids, coefs, xb, yb)
    torch.cuda.synchronize()
    # the same batch over the 16-row tile copies (the bench's configs[3] setting)
    moe.make_batch_tile_copies()
    for _ in range(2):
        be.route_experts_batch(logits, 8, ids, coefs)
        be.moe_forward_batch(moe, ids, coefs, xb, yb)
    torch.cuda.synchronize()
    # configs[4] prefill GEMM
    R, T = 12288, 512
    m5 = be.upload(13, R, H, synth.random_matrix(13, R, H, 801)); m5.prepare_gemm()
    q8 = torch.zeros((T, 16 * 292), dtype=torch.uint8, device='cuda')
    be.quantize_q8_k_rows(torch.randn(T, H, device='cuda'), q8, T, H)
    ws = torch.zeros(be.gemm_workspace_bytes(T, H), dtype=torch.uint8, device='cuda')
    yp = torch.zeros((T, R), device='cuda')
    for _ in range(2):
        be.gemm_q8_k(m5, q8, T, yp, ws)
    torch.cuda.synchronize()
    print("pmc workloads done", flush=True)


def main():
    args = parse()
    if args.pmc_workloads:
        pmc_workloads()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this build runs on a "
              f"single MI355X (the multi-GPU sharding of the path is a design, not built)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import lbhip
    from lbhip import synth

    be = lbhip.HipBackend(0)
    be.set_tuning(be.TUNE_GEMV_LPU, args.lpu)
    stream = torch.cuda.Stream()
    be.set_stream(stream)
    timer = Timer(torch, stream)

    mv = bench_matvec_step(args, be, timer, torch, np, synth)
    _progress(f"configs[1] step {mv['ms_per_step'] * 1e3:.2f} us")
    w_q4k, q4k = bench_q4k(args, be, timer, torch, np, synth)
    _progress(f"configs[0] {q4k['us_per_matvec']} us")
    model_mv = bench_model_shapes(args, be, timer, torch, np, synth)
    _progress("model shapes done")
    ingest = bench_ingest(args, be, torch, np, synth, lbhip)
    _progress("gguf ingest done")
    moe = state = batch = batch_check = streaming = None
    prefill, pf_check = bench_prefill(args, be, timer, torch, np, synth)
    _progress(f"configs[4] {prefill['us_per_step']} us")
    if not args.no_moe:
        moe, state = bench_moe(args, be, timer, torch, np, synth, lbhip)
        _progress("configs[2] done")
        batch, batch_check = bench_batch(args, be, timer, torch, np, synth, state)
        _progress(f"configs[3] {batch['us_per_step']} us")
        if args.stream_tokens > 0:
            streaming = bench_streaming(args, be, torch, np, synth, lbhip, state)
            _progress("expert streaming done")

    value = STEP_BYTES / (mv["ms_per_step"] * 1e-3) / 1e9
    if mv["down_us"] >= mv["gate_us"]:
        dom = ("k_gemv<IQ3_S, fused Q8_K> (down 4096x1536)", mv["down_us"], DOWN_BYTES, MEASURED_TRAFFIC["down"],
               mv["down_floor"])
    else:
        dom = ("k_gemv<IQ2_S, fused Q8_K> (gate 1536x4096)", mv["gate_us"], GATE_BYTES, MEASURED_TRAFFIC["gate"],
               mv["gate_floor"])
    step_floor_us = mv["gate_floor"][0] + mv["down_floor"][0]
    achieved = dom[2] / (dom[1] * 1e-6) / 1e9
    line = {
        "metric": "quant matvec HBM GB/s (% of MI355X peak); MoE-block decode tokens/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": mv["steps"],
        "warmup": mv["warmup"],
        "ms_per_step": round(mv["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi8->i32 integer dots, f32 scale fold",
        "data": "synthetic (random-from-seed weights and activations; no checkpoint)",
        "config": {"workload": "configs[1]: IQ2_S gate 1536x4096 + IQ3_S down 4096x1536 matvecs, batch 1 "
                               "(one routed expert's decode pass, one token)",
                   "step": "Q8_K(x)+IQ2_S gate -> Q8_K(h)+IQ3_S down: 2 fused kernels per step, HIP graph",
                   "weight_copies_in_rotation": mv["copies"],
                   "steps_note": "the timed steps are rounded up to whole rotations of the weight copies, so "
                                 "`steps` can exceed --steps",
                   "rotation_bytes": mv["copies"] * (mv["w_gate"].nbytes + mv["w_down"].nbytes),
                   "algorithmic_bytes_per_step": STEP_BYTES, "lpu": args.lpu},
        "roofline": {"bound": "hbm", "kernel": dom[0], "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": dom[3],
                     "avg_launch_us": round(dom[1], 3), "algorithmic_bytes_per_launch": dom[2],
                     **floor_fields(dom[1], mv["empty_us"], dom[4])},
        "kernels_us": {"iq2s_gate": round(mv["gate_us"], 3), "iq3s_down": round(mv["down_us"], 3)},
        "timing": {"what": "value, ms_per_step and kernels_us are totals over back-to-back HIP-graph replays "
                           "(one event pair around all of them); the spreads time each replay with its own "
                           "event pair and give median / p10 / p90 per step or per launch",
                   "step": mv["step_spread"], **mv["kernel_spread"]},
        "floors": {"what": "launch floor (an empty kernel) and memory floor (the fastest plain read of the same "
                           "weight bytes over a sweep of launch shapes, same rotation of copies) per kernel of the "
                           "step; frac_of_floor = floor / measured",
                   "gate": floor_fields(mv["gate_us"], mv["empty_us"], mv["gate_floor"]),
                   "down": floor_fields(mv["down_us"], mv["empty_us"], mv["down_floor"]),
                   "step_read_floor_us": round(step_floor_us, 3),
                   "step_frac_of_floor": round(step_floor_us / (mv["ms_per_step"] * 1e3), 4)},
        "q4k_matvec": q4k,
        "model_matvecs": {"workload": "decode matvecs (fused Q8_K + matvec, batch 1) at the Hy3 model's tensor shapes "
                                      "and types (schema.rs:96-201)", "shapes": model_mv},
        "gguf_ingest": ingest,
        "prefill_gemm": prefill,
    }
    if moe is not None:
        line["moe_block"] = moe
        line["moe_batch"] = batch
    if streaming is not None:
        line["expert_streaming"] = streaming
    if not args.no_cpu:
        _progress("CPU baselines")
        line["cpu_baseline"] = cpu_matvec_step(mv["w_gate"], mv["w_down"], args.cpu_seconds / 2)
        allc = cpu_matvec_step(mv["w_gate"], mv["w_down"], args.cpu_seconds / 2, threads=logical_cpus())
        line["cpu_baseline"]["all_cores"] = {k: allc[k] for k in ("value", "unit", "threads", "ms_per_step", "sample")}
        line["cpu_baseline"]["threads_rule"] = ("ceil(logical CPUs / 2), recommended_thread_count "
                                                "(crates/bridge-kernels-cpu/src/lib.rs:121-126); all_cores beside it")
        _progress("CPU configs[1] done")
        cq = cpu_q4k(w_q4k, args.cpu_seconds / 2)
        q4k["cpu_baseline"] = cq
        q4k["speedup_vs_cpu"] = round(q4k["GB/s"] / cq["value"], 1)
        if moe is not None:
            cm = cpu_moe(state["experts_np"], state["shared_np"], state["router_w"], state["xs_np"], args.cpu_seconds)
            moe["cpu_baseline"] = cm
            moe["speedup_vs_cpu"] = round(moe["with_device_router"]["tokens_per_s"] / cm["value"], 1)
            moe["speedup_vs_cpu_routing_given"] = round(moe["routing_given"]["tokens_per_s"] / cm["value"], 1)
            _progress("CPU configs[2] done")
            cb = cpu_batch(state["experts_np"], state["shared_np"], batch_check, args.cpu_seconds / 2)
            batch["cpu_baseline"] = cb
            batch["speedup_vs_cpu"] = round(batch["tokens_per_s"] / cb["value"], 1)
        _progress("CPU configs[3] done")
        cp = cpu_prefill(pf_check, args.cpu_seconds / 2)
        prefill["cpu_baseline"] = cp
        prefill["speedup_vs_cpu"] = round(prefill["dot_TOPS"] / cp["value"], 1)
        line["parity_spot_checks_bit_exact"] = cpu_parity(mv, state, batch_check)
        line["parity_spot_checks_bit_exact"]["configs[4]_tokens_0_7"] = _prefill_parity(pf_check)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
