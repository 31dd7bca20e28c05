#!/usr/bin/env python3
"""Benchmark of the MRML decode hot path on one MI355X.

Workload: batch-1 Q4_0 matvecs at Gemma-2-2B FFN
shapes.  One step = one FFN pass over synthetic data:
    quantize x (2304)  ->  fused gate+up GeGLU matvec (2 x 9216x2304)
    quantize act (9216) ->  down matvec (2304x9216)
`value` is whole-step throughput in GB/s of algorithmic bytes (weights +
vectors), with weights resident in HBM and rotated over enough copies to
exceed the 256 MB MALL, timed with HIP events around a graph of the steps.
The JSON line also carries the per-matrix GB/s (gate, up, down, fused
gate+up), the dominant kernel's roofline, and the host-CPU baseline (the C
oracle restating the reference CPU path, timed on this box's cores).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import ctypes
import ctypes.util
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "qt_llama.cpp_amd"

DIM, FFN = 2304, 9216
Q4_ROW = lambda k: k // 32 * 18                       # GGUF Q4_0 bytes per row
W_BYTES = FFN * Q4_ROW(DIM)                            # 11,943,936 per matrix
# algorithmic bytes per launch: weights + f32 input + f32 output
BYTES_GATE = W_BYTES + DIM * 4 + FFN * 4
BYTES_DOWN = W_BYTES + FFN * 4 + DIM * 4
BYTES_GEGLU = 2 * W_BYTES + DIM * 4 + FFN * 4          # 23,887,872 + 9,216 + 36,864
BYTES_STEP = BYTES_GEGLU + BYTES_DOWN
PEAK_HBM_GBS = 8000.0
MALL_BYTES = 256 << 20


def load_backend():
    name = "qt_llama_cpp_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG / "__init__.py", submodule_search_locations=[str(PKG)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


class HipEvents:
    """hipEvent timing on a given stream (the library's own stream)."""

    def __init__(self):
        path = ctypes.util.find_library("amdhip64") or "/opt/rocm/lib/libamdhip64.so"
        self.hip = ctypes.CDLL(path)
        for n in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipEventDestroy"):
            getattr(self.hip, n).restype = ctypes.c_int

    def new(self):
        e = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream: int):
        assert self.hip.hipEventRecord(e, ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.hip.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return float(ms.value)


def time_graph(dev, ev, graph, launches: int) -> float:
    """Seconds for `launches` replays of `graph`, events on the device stream."""
    a, b = ev.new(), ev.new()
    dev.sync()
    ev.record(a, dev.stream)
    for _ in range(launches):
        graph.launch()
    ev.record(b, dev.stream)
    return ev.elapsed_ms(a, b) / 1e3


def cpu_baseline(orc, synth, budget_s: float) -> dict:
    """The oracle (reference CPU algorithm, VNNI path where the host has it,
    row-parallel like parallel.rs) on one FFN step, best of N wall-clock
    rounds (benches/hot_paths.rs:21-30)."""
    threads = len(os.sched_getaffinity(0))
    rng = synth.rng_for(2)
    wg = synth.q4_0_matrix(rng, FFN, DIM)
    wu = synth.q4_0_matrix(rng, FFN, DIM)
    wd = synth.q4_0_matrix(rng, DIM, FFN)
    x = synth.rms_normalised(synth.normal_vector(rng, DIM))

    def step():
        xq = orc.quantize_q8_0(x)
        g = orc.mat_vec_mul_q4_0_q8_0(wg, xq, FFN, DIM, threads=threads)
        u = orc.mat_vec_mul_q4_0_q8_0(wu, xq, FFN, DIM, threads=threads)
        act = orc.geglu(g, u)
        return orc.mat_vec_mul_q4_0(wd, act, DIM, FFN, threads=threads)

    step()
    best, rounds, t_end = float("inf"), 0, time.perf_counter() + budget_s
    while time.perf_counter() < t_end or rounds < 3:
        t0 = time.perf_counter()
        step()
        best = min(best, time.perf_counter() - t0)
        rounds += 1
    isa = {2: "avx-vnni", 1: "avx2", 0: "scalar"}[orc.host_isa()]
    return {"value": round(BYTES_STEP / best / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{rounds} FFN steps (quantize, gate, up, GeGLU, quantize, down at 2304/9216), "
                      f"best-of wall clock over ~{budget_s:.0f} s, {threads} threads, {isa} dot path",
            "ms_per_step": round(best * 1e3, 3)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--sets", type=int, default=0, help="rotating weight sets (default: > 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-loop", type=int, default=0,
                    help="only replay the GeGLU kernel graph this many times (for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "collectives and multi-GPU sharding are out of scope", file=sys.stderr)
        return 2

    be = load_backend()
    import qt_llama_cpp_amd.synth as synth
    dev = be.HipDevice.new(0)
    info = dev.device_info()
    ev = HipEvents()

    # ---- synthetic config-2 data, rotated over > 2x MALL of distinct copies
    rng = synth.rng_for(2)
    host = {"g": synth.q4_0_matrix(rng, FFN, DIM), "u": synth.q4_0_matrix(rng, FFN, DIM),
            "d": synth.q4_0_matrix(rng, DIM, FFN)}
    x = synth.rms_normalised(synth.normal_vector(rng, DIM))
    sets = args.sets or int(np.ceil(2 * MALL_BYTES / (3 * W_BYTES))) + 1
    first = {"g": be.HipBuffer.from_gguf(dev, host["g"], be.Q4_0, FFN, DIM),
             "u": be.HipBuffer.from_gguf(dev, host["u"], be.Q4_0, FFN, DIM),
             "d": be.HipBuffer.from_gguf(dev, host["d"], be.Q4_0, DIM, FFN)}
    rot = [first]
    for _ in range(sets - 1):
        s = {k: be.HipBuffer(dev, v.nbytes) for k, v in first.items()}
        for k in s:
            dev.copy_kernel(s[k], first[k], first[k].nbytes)
        rot.append(s)
    bx = be.HipBuffer.from_host(dev, x)
    act = be.HipBuffer.alloc(dev, FFN)
    y = be.HipBuffer.alloc(dev, DIM)
    dev.reserve_workspace(1 << 20)
    dev.sync()

    # one FFN step = mrml_hip_ffn_geglu_q4_0: two launches (GeGLU quantising x
    # itself and emitting the activation pack, then the down projection)
    def ffn_step(s):
        dev.ffn_geglu_q4_0(s["g"], s["u"], s["d"], bx, None, y, DIM, FFN)

    # one graph = one step over every rotating set
    for s in rot:
        ffn_step(s)
    dev.sync()
    g_step = dev.capture(lambda: [ffn_step(s) for s in rot])
    q_pack = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(DIM), np.uint8)
    dev.quantize_q8_0(bx, None, q_pack, DIM)
    a_pack = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(FFN), np.uint8)
    g_geglu = dev.capture(lambda: [dev.gemv_q4_0_geglu_pack(s["g"], s["u"], bx, None, a_pack, FFN, DIM) for s in rot])

    if args.profile_loop:
        for _ in range(args.profile_loop):
            g_geglu.launch()
        dev.sync()
        print(json.dumps({"profile_loop": args.profile_loop, "launches": args.profile_loop * sets}))
        return 0

    # ---- warmup, then exactly K steps between events
    reps_w = max(1, args.warmup // sets)
    reps = max(1, args.steps // sets)
    steps = reps * sets
    time_graph(dev, ev, g_step, reps_w)
    t = time_graph(dev, ev, g_step, reps)
    ms_per_step = t / steps * 1e3
    value = BYTES_STEP * steps / t / 1e9

    # ---- per-kernel rates (each timed alone over the rotating sets)
    def rate(fn, nbytes, per_graph):
        g = dev.capture(lambda: [fn(s) for s in rot])
        time_graph(dev, ev, g, 3)
        launches = max(5, 400 // per_graph)
        secs = time_graph(dev, ev, g, launches) / (launches * per_graph)
        g.close()
        return secs, nbytes / secs / 1e9

    out_f = be.HipBuffer.alloc(dev, FFN)
    # the step's first launch (f32 x in, activation pack out)
    k_geglu, gbs_geglu = rate(lambda s: dev.gemv_q4_0_geglu_pack(s["g"], s["u"], bx, None, a_pack, FFN, DIM),
                              BYTES_GEGLU, sets)
    k_gate, gbs_gate = rate(lambda s: dev.gemv_q4_0_q8(s["g"], q_pack, out_f, FFN, DIM), BYTES_GATE, sets)
    k_up, gbs_up = rate(lambda s: dev.gemv_q4_0_q8(s["u"], q_pack, out_f, FFN, DIM), BYTES_GATE, sets)
    # the step's second launch (activation pack in)
    k_down, gbs_down = rate(lambda s: dev.gemv_q4_0_q8(s["d"], a_pack, y, DIM, FFN), BYTES_DOWN, sets)
    # stream-copy ceiling on a buffer well above the MALL
    cbytes = 1 << 30
    src, dst = be.HipBuffer(dev, cbytes), be.HipBuffer(dev, cbytes)
    gc = dev.capture(lambda: dev.copy_kernel(dst, src, cbytes))
    time_graph(dev, ev, gc, 2)
    tc = time_graph(dev, ev, gc, 10) / 10
    copy_gbs = 2 * cbytes / tc / 1e9
    dev.sync()

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT))
        from oracle import orc
        cpu = cpu_baseline(orc, synth, args.cpu_seconds)

    line = {
        "metric": "Q4_0 matvec GB/s (Gemma-2-2B FFN: fused gate+up GeGLU + down, batch 1)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * sets,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 -> int32, f32 fold",
        "data": "synthetic (seeded GGUF Q4_0 bytes, N(0,1) RMS-normalised x)",
        "config": {"workload": "BASELINE configs[1]: Q4_0 gate/up 9216x2304 + down 2304x9216, batch 1",
                   "bytes_per_step": BYTES_STEP, "rotating_weight_sets": sets,
                   "rotating_bytes": sets * 3 * W_BYTES, "timing": "hipEvent around graph replays"},
        "pct_of_hbm_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "per_matrix_gbs": {"gate": round(gbs_gate, 1), "up": round(gbs_up, 1), "down": round(gbs_down, 1),
                           "fused_gate_up_geglu": round(gbs_geglu, 1)},
        "per_kernel_us": {"geglu": round(k_geglu * 1e6, 3), "gate": round(k_gate * 1e6, 3),
                          "up": round(k_up * 1e6, 3), "down": round(k_down * 1e6, 3)},
        "stream_copy_gbs": round(copy_gbs, 1),
        "roofline": {"bound": "hbm", "kernel": "gemv_q4_0_geglu_kernel", "achieved": round(gbs_geglu, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs_geglu / PEAK_HBM_GBS, 4),
                     "traffic": None, "bytes_per_launch": BYTES_GEGLU,
                     "avg_launch_us": round(k_geglu * 1e6, 3)},
        "cpu_baseline": cpu,
        "device": {"name": info["name"], "compute_units": info["compute_units"]},
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
