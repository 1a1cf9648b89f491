"""Per-wave timeline of the fused Q8_K matvec kernels (k_gemv) from the profiling
build of the library (`make -C lightbridge-engine_amd/csrc timeline` ->
liblightbridge_hip_timeline.so, whose matvec kernels stamp s_memrealtime, a
100 MHz clock, at fixed points of every wave).

Steady state (default): a HIP graph of back-to-back launches, each on its own
copy of the matrix (the copies together exceed the 256 MB Infinity Cache, so
every launch reads its weights from HBM), is replayed; the stamps read after a
replay are those of its last launch, preceded by the others as in the bench's
timed graphs.  --single: one launch after a synchronization instead (the
dispatch ramp of an idle GPU).  Stamps are relative to the launch's earliest
wave start.  Phases per wave:

  start     the wave's first instruction (the dispatch ramp across the grid)
  prologue  start -> end of the prologue's LDS stores (codebook, Q8_K of x)
  barrier   the workgroup barrier after the prologue
  landed    the first row step's weights in registers
  step      landed -> that step's rows folded and stored
  end       the wave's last instruction

Usage: python3 lightbridge-engine_amd/wave_timeline.py [--launches N] [--shapes configs1|all] [--single]
"""
from __future__ import annotations

import argparse
import ctypes as C
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
sys.path.insert(0, str(PKG))

import lbhip  # noqa: E402
from lbhip import synth  # noqa: E402

TL_LIB = PKG / "liblightbridge_hip_timeline.so"
WORDS = 16384 * 8
SHAPES = {
    "configs1": [("configs[1] IQ2_S gate 1536x4096", synth.IQ2_S, 1536, 4096),
                 ("configs[1] IQ3_S down 4096x1536", synth.IQ3_S, 4096, 1536)],
    "dense": [("dense FFN IQ2_S gate 13312x4096", synth.IQ2_S, 13312, 4096),
              ("dense FFN IQ3_S down 4096x13312", synth.IQ3_S, 4096, 13312)],
}


def pct(a: np.ndarray) -> str:
    return " / ".join(f"{np.percentile(a, q):.2f}" for q in (0, 50, 90, 100))


def run_shape(be, lib, torch, stream, name: str, ty: int, rows: int, k: int, launches: int,
              single: bool) -> list[str]:
    w = torch.from_numpy(synth.random_matrix(ty, rows, k, seed=rows + k).reshape(-1)).cuda()
    n = max(8, -(-600_000_000 // w.numel()))    # copies: > 600 MB in rotation
    copies = [be.upload(ty, rows, k, w) for _ in range(n)]
    del w
    x = torch.randn(k, device="cuda")
    y = torch.zeros(rows, device="cuda")
    buf = np.zeros(WORDS, np.uint64)
    phases = {p: [] for p in ("start", "prologue", "barrier", "landed", "step", "end")}
    event_us, waves = [], 0
    graph = None
    if not single:
        with torch.cuda.stream(stream):
            for m in copies:
                be.gemv_f32(m, x, y)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for m in copies:
                    be.gemv_f32(m, x, y)
    for i in range(launches):
        with torch.cuda.stream(stream):
            if single:
                for m in copies[launches:]:      # warm-up on copies the measured launch does not read
                    be.gemv_f32(m, x, y)
            stream.synchronize()
            lib.lbh_wave_timeline_clear()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            if single:
                be.gemv_f32(copies[i], x, y)
            else:
                graph.replay()
            e1.record(stream)
            stream.synchronize()
        event_us.append(e0.elapsed_time(e1) * 1e3 / (1 if single else n))
        lib.lbh_wave_timeline_read(buf.ctypes.data_as(C.c_void_p), C.c_size_t(buf.nbytes))
        t = buf.reshape(-1, 8).astype(np.int64)
        t = t[t[:, 0] > 0]
        waves = len(t)
        rel = (t[:, :6] - t[:, 0].min()) * 0.01          # microseconds
        phases["start"].append(rel[:, 0])
        phases["prologue"].append(rel[:, 1] - rel[:, 0])
        phases["barrier"].append(rel[:, 2])
        phases["landed"].append(rel[:, 3])
        phases["step"].append(rel[:, 4] - rel[:, 3])
        phases["end"].append(rel[:, 5])
    del graph
    for m in copies:
        m.close()
    how = ("single launches after a synchronization; event-timed launch" if single else
           f"last launch of a graph of {n} back-to-back launches on distinct copies; graph time per launch")
    out = [f"### {name}", "",
           f"{launches} replays, {waves} waves per launch; {how}: median {np.median(event_us):.2f} us", "",
           "| phase (us from the launch's first wave start) | min / median / p90 / max over all waves |",
           "|---|---|"]
    labels = {"start": "wave start", "prologue": "prologue duration (start -> LDS stores done)",
              "barrier": "prologue barrier passed", "landed": "first step's weights landed",
              "step": "first step: decode + fold duration", "end": "wave end"}
    for p, lab in labels.items():
        out.append(f"| {lab} | {pct(np.concatenate(phases[p]))} |")
    out.append("")
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--launches", type=int, default=8)
    ap.add_argument("--shapes", choices=("configs1", "all"), default="configs1")
    ap.add_argument("--single", action="store_true", help="single launches instead of graph replays")
    args = ap.parse_args()
    if not TL_LIB.exists():
        raise SystemExit(f"{TL_LIB} is missing: build it with `make -C {PKG / 'csrc'} timeline`")
    lbhip.LIB_PATH = TL_LIB
    import torch

    lib = lbhip.lib()
    lib.lbh_wave_timeline_read.argtypes = [C.c_void_p, C.c_size_t]
    be = lbhip.HipBackend(0)
    stream = torch.cuda.Stream()
    be.set_stream(stream)
    shapes = SHAPES["configs1"] + (SHAPES["dense"] if args.shapes == "all" else [])
    lines = []
    for name, ty, rows, k in shapes:
        lines += run_shape(be, lib, torch, stream, name, ty, rows, k, args.launches, args.single)
        print(f"[timeline] {name} done", file=sys.stderr, flush=True)
    print("\n".join(lines))


if __name__ == "__main__":
    main()
