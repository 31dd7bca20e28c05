#!/usr/bin/env python3
"""Benchmark of the MRML decode hot path on one MI355X.

Headline workload: batch-1 Q4_0 matvecs at
Gemma-2-2B FFN shapes.  One step = one FFN pass over synthetic data:
    quantize x (2304)  ->  fused gate+up GeGLU matvec (2 x 9216x2304)
    quantize act (9216) ->  down matvec (2304x9216)
`value` is whole-step throughput in GB/s of algorithmic bytes (weights +
vectors), with weights resident in HBM and rotated over 15 weight sets
(45 matrices, 537 MB, more than twice the 256 MB MALL), timed with HIP events
around graph replays: W warm-up steps, then timed regions of exactly K steps
each (as many regions as it takes to time at least 100 launches, at least 5);
`value` is the median region, the minimum is reported beside it.  The JSON
line also carries the per-matrix GB/s (gate, up, down, fused gate+up, each
rotated over the whole pool), the dominant kernel's roofline, and the
host-CPU baseline (the C oracle restating the reference CPU path, timed on
this box's cores).

BASELINE configs[0] (Q8_0 2048x2048) and configs[2] (Q4_K 256000x2304 and
its greedy argmax) are in "q8_0" and "q4_k", each with GB/s, % of peak and
its own CPU baseline.

The second half of the metric is in "decode": greedy decode tok/s
of a random-init Gemma-2-2B-shape Q4_0 model (512-token prefill, 256 decode
tokens, f16 KV cache of 4096), each token one replay of the captured step,
beside the CPU oracle's tok/s for the same step ("decode_cpu_baseline").

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
PEAK_INT8_TOPS = 5000.0                                # dense int8 MFMA, MI355X
MALL_BYTES = 256 << 20
PREFILL_CHUNK = 512                                    # tokens per chunk of mrml_hip_gemma2_prefill (model.hip)
# the dominant kernel of the step (the fused GeGLU that quantises x and emits the act pack)
GEGLU_KERNEL = "gemv_q4_0_geglu_split_kernel<72, 9>"


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


def sample_launches(dev, ev, graph, per_graph: int, samples: int = 7, min_launches: int = 100) -> dict:
    """`samples` timings, each of enough replays of `graph` (per_graph launches
    of one kernel each) for at least min_launches launches; median and min
    seconds per launch."""
    reps = max(1, -(-min_launches // per_graph))
    time_graph(dev, ev, graph, 1)
    t = sorted(time_graph(dev, ev, graph, reps) / (reps * per_graph) for _ in range(samples))
    return {"median_s": t[len(t) // 2], "min_s": t[0], "launches_per_sample": reps * per_graph,
            "samples": samples}


# Streaming-read floors: the bytes of each matvec here read by the product's
# plain read kernel (mrml_hip_read_kernel: 16-byte non-temporal loads, nothing
# written), one launch per slice of a 700 MB buffer, so no launch finds its
# bytes in the MALL -- what one launch of that size cannot beat on this GPU.
READ_FLOOR_SIZES = {"q8_0_2048x2048": 2048 * 2048 // 32 * 34, "qkv_4096x2304": 4096 * Q4_ROW(DIM),
                    "gate_9216x2304": W_BYTES, "geglu_2x9216x2304": 2 * W_BYTES,
                    "lm_head_256000x2304": 256000 * Q4_ROW(DIM)}


def read_floors(be, dev, ev) -> dict:
    """Median and min µs per launch of the read kernel at each size."""
    span = 700 << 20
    buf = be.HipBuffer(dev, span)
    sink = be.HipBuffer(dev, 1024)
    dev.zero(buf, span)
    out = {}
    for name, nbytes in READ_FLOOR_SIZES.items():
        nb16 = (nbytes + 15) // 16 * 16
        step = (nbytes + 4095) // 4096 * 4096
        n = max(2, min(128, span // step))
        g = dev.capture(lambda: [dev.read_kernel(buf.ptr + i * step, nb16, sink) for i in range(n)])
        st = sample_launches(dev, ev, g, n)
        g.close()
        out[name] = {"bytes": nbytes, "us": round(st["median_s"] * 1e6, 3), "us_min": round(st["min_s"] * 1e6, 3),
                     "gb_s": round(nbytes / st["median_s"] / 1e9, 1),
                     "pct_of_hbm_peak": round(100 * nbytes / st["median_s"] / 1e9 / PEAK_HBM_GBS, 2),
                     "slices": n}
    buf.close()
    sink.close()
    return out


def kernel_source_hash(files=("gemv_q4_0.hip", "device.h", "exact_sum.h", "norm_block.h", "libm_f32.h")) -> str:
    """sha256 (16 hex digits) of the sources the Q4_0 matvec kernels' code is
    generated from: a committed counter reading applies only to the kernels
    it measured."""
    import hashlib
    h = hashlib.sha256()
    for f in files:
        h.update(f.encode())
        h.update((PKG / "csrc" / f).read_bytes())
    return h.hexdigest()[:16]


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


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by what the
    counter reads for the copy kernel of known size in the same run), or None
    when no summary for this kernel exists."""
    path = ROOT / "profiles" / "gemv_q4_0_geglu_traffic.json"
    try:
        d = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if d.get("kernel") != kernel or d.get("source_sha256_16") != kernel_source_hash():
        return None
    return d.get("traffic_bytes")


def decode_bytes_per_token(cfg: dict, pos: int) -> int:
    """Algorithmic HBM bytes of one token step at position `pos`: every layer's
    Q4_0 weights, the tied Q4_0 head, the f16 K and V rows read by attention
    (pos + 1 of them per layer) and written (one), the embedding row and the
    norm weights."""
    d, f, V, L = cfg["dim"], cfg["ffn_dim"], cfg["vocab"], cfg["n_layers"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    layer_w = Q4_ROW(d) * (qd + 2 * kvd + 2 * f) + Q4_ROW(qd) * d + Q4_ROW(f) * d
    kv = 2 * (pos + 2) * kvd * 2
    return L * (layer_w + kv + 4 * d * 4) + V * Q4_ROW(d) + Q4_ROW(d) + d * 4


def decode_fast_bench(be, synth, dev, ev, n_prefill: int, n_decode: int, exact_hist) -> dict:
    """The same configs[3] workload under the FAST numerics
    (MRML_HIP_NUMERICS_FAST: tree-order norm sums, split-K attention): tok/s,
    and how its greedy picks compare with the EXACT run's (the prompt steps
    are teacher-forced, so each of their picks is compared on the same
    context; decode steps follow the model's own tokens)."""
    cfg = dict(synth.GEMMA2_2B)
    model = synth.gemma2_model(cfg, seed=1)
    m = be.Gemma2Model.from_host(dev, model, numerics=be.NUMERICS_FAST)
    m.set_sampler(temperature=0.0, top_k=40)
    prompt = synth.prompt_tokens(n_prefill, cfg["vocab"], seed=1)
    total = n_prefill + n_decode
    state = be.HipBuffer.from_host(dev, np.array([prompt[0], 0], np.int32))
    hist = be.HipBuffer.from_host(dev, np.full(total, -1, np.int32))
    pr = be.HipBuffer.from_host(dev, prompt)
    kc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    vc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    graph = dev.capture(lambda: m.step(state, kc, vc, hist=hist, hist_cap=total, prompt=pr, prompt_len=n_prefill))
    t_pre = time_graph(dev, ev, graph, n_prefill)
    t_dec = time_graph(dev, ev, graph, n_decode)
    dev.sync()
    h = hist.numpy()
    graph.close()
    m.close()
    nbytes = sum(decode_bytes_per_token(cfg, p) for p in range(n_prefill, total))
    same_prompt = int(np.sum(h[:n_prefill] == exact_hist[:n_prefill]))
    dec_same = np.flatnonzero(h[n_prefill:] != exact_hist[n_prefill:])
    return {"tok_s": round(n_decode / t_dec, 2), "ms_per_token": round(t_dec / n_decode * 1e3, 4),
            "gb_s": round(nbytes / t_dec / 1e9, 1), "pct_of_hbm_peak": round(100 * nbytes / t_dec / 1e9 / PEAK_HBM_GBS, 2),
            "prefill_ms_per_token": round(t_pre / n_prefill * 1e3, 4),
            "prompt_picks_equal_to_exact": f"{same_prompt}/{n_prefill}",
            "decode_tokens_equal_to_exact_until": int(dec_same[0]) if dec_same.size else n_decode,
            "numerics": "FAST: tree-order RMSNorm sums, split-K (flash-decoding) attention, tree-order row sums "
                        "in the output and down projections; the other matvecs bit-exact given their inputs"}


def decode_bench(be, synth, dev, ev, n_prefill: int, n_decode: int, cpu_steps: int) -> tuple[dict, dict | None]:
    """random-init Gemma-2-2B-shape Q4_0 model, f16 KV cache
    of 4096, prefill a seeded random prompt token by token, then greedy decode;
    every step is one replay of a captured token-step graph."""
    cfg = dict(synth.GEMMA2_2B)
    model = synth.gemma2_model(cfg, seed=1)
    m = be.Gemma2Model.from_host(dev, model)
    m.set_sampler(temperature=0.0, top_k=40)  # step_generation's greedy: masks, softcap, recent-token penalty
    prompt = synth.prompt_tokens(n_prefill, cfg["vocab"], seed=1)
    total = n_prefill + n_decode
    state = be.HipBuffer.from_host(dev, np.array([prompt[0], 0], np.int32))
    hist = be.HipBuffer.from_host(dev, np.full(total, -1, np.int32))
    pr = be.HipBuffer.from_host(dev, prompt)
    kc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    vc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    graph = dev.capture(lambda: m.step(state, kc, vc, hist=hist, hist_cap=total, prompt=pr, prompt_len=n_prefill))
    t_pre = time_graph(dev, ev, graph, n_prefill)
    t_dec = time_graph(dev, ev, graph, n_decode)
    dev.sync()
    exact_hist = hist.numpy()
    toks = exact_hist[n_prefill:]
    nbytes = sum(decode_bytes_per_token(cfg, p) for p in range(n_prefill, total))
    out = {"tok_s": round(n_decode / t_dec, 2), "ms_per_token": round(t_dec / n_decode * 1e3, 4),
           "gb_s": round(nbytes / t_dec / 1e9, 1), "pct_of_hbm_peak": round(100 * nbytes / t_dec / 1e9 / PEAK_HBM_GBS, 2),
           "bytes_per_token_avg": nbytes // n_decode, "prefill_tokens": n_prefill, "decode_tokens": n_decode,
           "prefill_ms_per_token": round(t_pre / n_prefill * 1e3, 4),
           "workload": "BASELINE configs[3]: 26 layers, 2304, 8/4 heads x 256, GeGLU 9216, tied 256000 Q4_0 "
                       "head, f16 KV cache 4096, token step captured once and replayed",
           "pick": "step_generation's greedy: early-id mask, 30*tanh softcap, -3.5 for the last 32 tokens",
           "first_tokens": toks[:4].tolist(), "distinct_prompt_picks": int(len(set(exact_hist[:n_prefill].tolist()))),
           "numerics": "EXACT: every op in the CPU path's order (logits bit-identical to the oracle)"}
    graph.close()
    # the same prompt through the chunked prefill (batched MFMA products) on
    # fresh caches: throughput, and its caches and last-position argmax
    # against the token steps above
    kc_ref, vc_ref, first_ref = kc.numpy(), vc.numpy(), int(hist.numpy()[n_prefill - 1])
    kc.copy_from_host(np.zeros(m.cache_elems(), np.uint16))
    vc.copy_from_host(np.zeros(m.cache_elems(), np.uint16))
    am = be.HipBuffer.from_host(dev, np.array([-1], np.int32))
    m.prefill(pr, 1, 0, kc, vc, argmax=am)  # allocates the chunk buffers
    dev.sync()
    a, b = ev.new(), ev.new()
    ev.record(a, dev.stream)
    m.prefill(pr, n_prefill, 0, kc, vc, argmax=am)
    ev.record(b, dev.stream)
    t_pf = ev.elapsed_ms(a, b) / 1e3
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    shape = (cfg["n_layers"], cfg["ctx_len"], kvd)
    same = (int(am.numpy()[0]) == first_ref and
            np.array_equal(kc.numpy().reshape(shape)[:, :n_prefill], kc_ref.reshape(shape)[:, :n_prefill]) and
            np.array_equal(vc.numpy().reshape(shape)[:, :n_prefill], vc_ref.reshape(shape)[:, :n_prefill]))
    out["prefill_batched"] = {"tok_s": round(n_prefill / t_pf, 1), "ms_per_token": round(t_pf / n_prefill * 1e3, 4),
                              "chunk": PREFILL_CHUNK, "bit_identical_to_token_steps": bool(same),
                              "how": "mrml_hip_gemma2_prefill, eager (host launch time included), "
                                     "events around one call over the whole prompt"}
    m.close()
    cpu = None
    if cpu_steps > 0:
        sys.path.insert(0, str(ROOT))
        from oracle import orc
        threads = len(os.sched_getaffinity(0))
        o = orc.OracleGemma2(model)
        # a filled cache: positions < n_prefill hold random f16 rows (the
        # attention work per step depends only on the position)
        fill = np.random.default_rng(7).standard_normal(o.k_cache.size, dtype=np.float32).astype(np.float16)
        o.k_cache[:] = fill.view(np.uint16)
        o.v_cache[:] = fill.view(np.uint16)[::-1]
        tok, t0 = int(prompt[-1]), time.perf_counter()
        for i in range(cpu_steps):
            tok = o.step(tok, n_prefill + i, threads=threads)
        t_cpu = time.perf_counter() - t0
        cbytes = sum(decode_bytes_per_token(cfg, p) for p in range(n_prefill, n_prefill + cpu_steps))
        cpu = {"value": round(cpu_steps / t_cpu, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "gb_s": round(cbytes / t_cpu / 1e9, 2),
               "sample": f"{cpu_steps} decode steps of the oracle token step (orc_gemma2_step) at positions "
                         f"{n_prefill}..{n_prefill + cpu_steps - 1}, {threads} threads"}
    out["_exact_hist"] = exact_hist
    return out, cpu


def prefill_profile(be, synth, dev, n_prefill: int) -> dict:
    """Profiling aid for the chunked prefill of the C4 model: one warm-up
    call of one token, then one prefill of n_prefill tokens from position 0."""
    cfg = dict(synth.GEMMA2_2B)
    model = synth.gemma2_model(cfg, seed=1)
    m = be.Gemma2Model.from_host(dev, model)
    prompt = synth.prompt_tokens(n_prefill, cfg["vocab"], seed=1)
    pr = be.HipBuffer.from_host(dev, prompt)
    kc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    vc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    am = be.HipBuffer.from_host(dev, np.array([-1], np.int32))
    m.prefill(pr, 1, 0, kc, vc, argmax=am)
    dev.sync()
    m.prefill(pr, n_prefill, 0, kc, vc, argmax=am)
    dev.sync()
    m.close()
    return {"profile_prefill": n_prefill, "first_token": int(am.numpy()[0])}


def decode_profile(be, synth, dev, n_prefill: int, n_steps: int, numerics: int = 0, prefilled: bool = False) -> dict:
    """Profiling aid for the C4 model: n_prefill + n_steps token steps issued
    eagerly (no graph: the kernel trace then sees every launch; rocprofv3's
    kernel trace of many graph replays crashed in the runtime's graph-launch
    path on this image); the last n_steps are the decode steps at positions
    n_prefill..  With prefilled, the prompt goes through one batched prefill
    call instead of token steps (few dispatches: counter passes serialise
    every one).  Progress goes to stderr every 64 steps."""
    cfg = dict(synth.GEMMA2_2B)
    model = synth.gemma2_model(cfg, seed=1)
    m = be.Gemma2Model.from_host(dev, model, numerics=numerics)
    m.set_sampler(temperature=0.0, top_k=40)
    prompt = synth.prompt_tokens(n_prefill, cfg["vocab"], seed=1)
    total = n_prefill + n_steps
    state = be.HipBuffer.from_host(dev, np.array([prompt[0], 0], np.int32))
    hist = be.HipBuffer.from_host(dev, np.full(total, -1, np.int32))
    pr = be.HipBuffer.from_host(dev, prompt)
    kc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    vc = be.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    first = 0
    if prefilled:
        am = be.HipBuffer.from_host(dev, np.array([-1], np.int32))
        m.prefill(pr, n_prefill, 0, kc, vc, argmax=am)
        dev.sync()
        state.copy_from_host(np.array([int(am.numpy()[0]), n_prefill], np.int32))
        first = n_prefill
    for i in range(first, total):
        m.step(state, kc, vc, hist=hist, hist_cap=total, prompt=pr, prompt_len=n_prefill)
        if i % 64 == 63:
            dev.sync()
            print(f"[profile-decode] step {i + 1}/{total}", file=sys.stderr, flush=True)
    dev.sync()
    m.close()
    return {"profile_decode": n_steps, "prefill_tokens": n_prefill, "numerics": numerics, "prefilled": prefilled}


def gemm_bench(be, synth, dev, ev, batch: int, cpu_tokens: int, profile: int = 0) -> dict:
    """M prefill tokens x K, quantised to Q8_0, times the
    Q4_0 gate/up (9216x2304) and down (2304x9216) matrices on int8 MFMA.
    Ops = 2*M*rows*cols per matrix (the int8 multiply-adds of the block dots);
    utilisation is against MI355X's dense int8 MFMA peak."""
    rng = synth.rng_for(5)
    mats = {"gate": (FFN, DIM), "up": (FFN, DIM), "down": (DIM, FFN)}
    w = {k: be.HipBuffer.from_gguf(dev, synth.q4_0_matrix(rng, r, c), be.Q4_0, r, c) for k, (r, c) in mats.items()}
    xs = {DIM: rng.standard_normal((batch, DIM)).astype(np.float32),
          FFN: rng.standard_normal((batch, FFN)).astype(np.float32)}
    packs, xb = {}, {}
    for k, xv in xs.items():
        xb[k] = be.HipBuffer.from_host(dev, xv.reshape(-1))
        packs[k] = be.HipBuffer.alloc(dev, dev.gemm_pack_bytes(k, batch), np.uint8)
        dev.quantize_q8_0_gemm(xb[k], packs[k], k, batch)
    y = be.HipBuffer.alloc(dev, batch * FFN)
    dev.sync()
    if profile:
        for _ in range(profile):
            dev.quantize_q8_0_gemm(xb[DIM], packs[DIM], DIM, batch)
            for k, (r, c) in mats.items():
                dev.gemm_q4_0_gpack(w[k], packs[c], y, r, c, batch)
        dev.sync()
        return {"profile_gemm": profile, "launches": 4 * profile}
    per, total_ops, total_s = {}, 0, 0.0
    per_graph = 10  # launches per graph, so host-side graph launch cost stays hidden
    for k, (r, c) in mats.items():
        g = dev.capture(lambda: [dev.gemm_q4_0_gpack(w[k], packs[c], y, r, c, batch) for _ in range(per_graph)])
        st = sample_launches(dev, ev, g, per_graph)
        g.close()
        secs = st["median_s"]
        ops = 2 * batch * r * c
        per[k] = {"us": round(secs * 1e6, 2), "us_min": round(st["min_s"] * 1e6, 2), "tops": round(ops / secs / 1e12, 2),
                  "launches_per_sample": st["launches_per_sample"]}
        total_ops += ops
        total_s += secs
    # the tolerance path's one-FMA fold (mrml_hip_gemm_q4_0_relaxed) beside
    # the exact one, both from f32 activations (quantisation included)
    relaxed = {}
    for k in ("gate", "down"):
        r, c = mats[k]
        dev.gemm_q4_0(w[k], xb[c], y, r, c, batch)  # workspace sized before capture
        row = {}
        for name, fn in (("exact", dev.gemm_q4_0), ("relaxed", dev.gemm_q4_0_relaxed)):
            g = dev.capture(lambda: [fn(w[k], xb[c], y, r, c, batch) for _ in range(per_graph)])
            st = sample_launches(dev, ev, g, per_graph)
            g.close()
            row[name + "_us"] = round(st["median_s"] * 1e6, 2)
        row["speedup"] = round(row["exact_us"] / row["relaxed_us"], 3)
        relaxed[k] = row
    # quantising the [M][K] activations into the GEMM pack (once per input)
    gq = dev.capture(lambda: [dev.quantize_q8_0_gemm(xb[DIM], packs[DIM], DIM, batch) for _ in range(20)])
    time_graph(dev, ev, gq, 2)
    tq = time_graph(dev, ev, gq, 10) / 200
    gq.close()
    tops = total_ops / total_s / 1e12
    # achieved int8 TOPS over the dense peak; the matrix cores' busy fraction
    # from SQ_VALU_MFMA_BUSY_CYCLES is in the committed PMC summary
    out = {"tops": round(tops, 2), "unit": "TOPS (int8)", "tops_over_peak": round(tops / PEAK_INT8_TOPS, 4),
           "mfma_busy": "profiles/gemm_q4_0_mfma_pmc.md (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x 1024 SIMDs))",
           "peak_tops": PEAK_INT8_TOPS, "per_matrix": per, "batch": batch,
           "quantize_q8_0_us": round(tq * 1e6, 2), "kernel": "gemm_q4_0_mfma_kernel",
           "relaxed_fold": dict(relaxed, how="f32 activations in (quantisation included); the FAST numerics' prefill "
                                             "uses the relaxed fold (within 1e-5 of the exact product)"),
           "workload": f"BASELINE configs[4]: M={batch} tokens, Q4_0 gate/up 9216x2304 + down 2304x9216, "
                       "activations pre-quantised to Q8_0 (GEMM pack), hipEvent around graph replays"}
    if cpu_tokens > 0:
        sys.path.insert(0, str(ROOT))
        from oracle import orc
        threads = len(os.sched_getaffinity(0))
        hw = synth.q4_0_matrix(synth.rng_for(5), FFN, DIM)
        xq = [orc.quantize_q8_0(xs[DIM][m]) for m in range(cpu_tokens)]
        orc.mat_vec_mul_q4_0_q8_0(hw, xq[0], FFN, DIM, threads=threads)
        t0 = time.perf_counter()
        for m in range(cpu_tokens):
            orc.mat_vec_mul_q4_0_q8_0(hw, xq[m], FFN, DIM, threads=threads)
        t_cpu = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(2 * cpu_tokens * FFN * DIM / t_cpu / 1e12, 4), "unit": "TOPS",
                               "cores": threads, "kind": "port",
                               "sample": f"{cpu_tokens} tokens of the 9216x2304 gate product, token at a time "
                                         f"(the reference CPU prefill), {threads} threads"}
    return out


def cpu_best_of(fn, budget_s: float) -> tuple[float, int]:
    """Best-of-N wall clock of fn() (benches/hot_paths.rs:21-30) over about
    budget_s seconds (at least 3 rounds)."""
    fn()
    best, rounds, t_end = float("inf"), 0, time.perf_counter() + budget_s
    while time.perf_counter() < t_end or rounds < 3:
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
        rounds += 1
    return best, rounds


def q8_0_bench(be, synth, dev, ev, cpu_s: float) -> dict:
    """Q8_0 2048x2048 batch-1 matvec, x quantised once by
    the reference routine, weights rotated over 128 copies (570 MB, more than
    twice the MALL).  Algorithmic bytes per run: W + x (f32) + y (f32)."""
    rows = cols = 2048
    nbytes_w = rows * cols // 32 * 34
    nbytes = nbytes_w + cols * 4 + rows * 4
    rng = synth.rng_for(1)
    w = synth.q8_0_matrix(rng, rows, cols)
    x = synth.normal_vector(rng, cols)
    first = be.HipBuffer.from_gguf(dev, w, be.Q8_0, rows, cols)
    copies = 128
    pool = [first] + [be.HipBuffer(dev, first.nbytes) for _ in range(copies - 1)]
    for b in pool[1:]:
        dev.copy_kernel(b, first, first.nbytes)
    xb = be.HipBuffer.from_host(dev, x)
    pk = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(cols), np.uint8)
    y = be.HipBuffer.alloc(dev, rows)
    dev.quantize_q8_0(xb, None, pk, cols)
    dev.sync()
    g = dev.capture(lambda: [dev.gemv_q8_0_q8(b, pk, y, rows, cols) for b in pool])
    st = sample_launches(dev, ev, g, copies)
    g.close()
    gbs = nbytes / st["median_s"] / 1e9
    out = {"gb_s": round(gbs, 1), "gb_s_best": round(nbytes / st["min_s"] / 1e9, 1),
           "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2), "us_median": round(st["median_s"] * 1e6, 3),
           "us_min": round(st["min_s"] * 1e6, 3), "bytes_per_launch": nbytes, "kernel": "gemv_q8_0_kernel",
           "launches_per_sample": st["launches_per_sample"], "rotating_copies": copies,
           "workload": "BASELINE configs[0]: Q8_0 2048x2048, batch 1, x pre-quantised (Q8_0 pack), "
                       "hipEvent around graph replays over 128 weight copies"}
    for b in pool[1:]:
        b.close()
    if cpu_s > 0:
        sys.path.insert(0, str(ROOT))
        from oracle import orc
        threads = len(os.sched_getaffinity(0))
        xq = orc.quantize_q8_0(x)
        best, rounds = cpu_best_of(lambda: orc.mat_vec_mul_q8_0_q8_0(w, xq, rows, cols, threads=threads), cpu_s)
        isa = {2: "avx-vnni", 1: "avx2", 0: "scalar"}[orc.host_isa()]
        out["cpu_baseline"] = {"value": round(nbytes / best / 1e9, 2), "unit": "GB/s", "cores": threads,
                               "kind": "port", "sample": f"{rounds} matvecs 2048x2048 (vec_dot_q8_0_q8_0 per row, "
                                                         f"{isa} path), best-of wall clock, {threads} threads"}
    return out


def q4_k_bench(be, synth, dev, ev, cpu_s: float) -> dict:
    """Q4_K 256000x2304 batch-1 matvec (331.8 MB, two
    copies alternated so no launch finds its weights in the MALL) and the
    greedy argmax over the 256000 logits."""
    rows, cols = 256000, 2304
    nbytes_w = rows * cols // 256 * 144
    nbytes = nbytes_w + cols * 4 + rows * 4
    rng = synth.rng_for(3)
    w = synth.q4_k_matrix(rng, rows, cols)
    x = synth.normal_vector(rng, cols)
    first = be.HipBuffer.from_gguf(dev, w, be.Q4_K, rows, cols)
    second = be.HipBuffer(dev, first.nbytes)
    dev.copy_kernel(second, first, first.nbytes)
    pool = [first, second]
    xb = be.HipBuffer.from_host(dev, x)
    pk = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(cols), np.uint8)
    y = be.HipBuffer.alloc(dev, rows)
    am = be.HipBuffer.alloc(dev, 1, np.int32)
    dev.quantize_q8_0(xb, None, pk, cols)
    dev.argmax_f32(y, rows, am)
    dev.vocab_select(y, rows, generated_count=9, temperature=0.8, pos=7, k=40, token=am)
    dev.sync()                                        # workspace at its largest before any capture
    # Timing: graph replays of 20 launches (the two copies alternating), 7
    # samples of at least 100 launches -- the method of every other leg.  The
    # same launches issued eagerly from Python are reported beside it; between
    # boxes either method has been the faster by several us a launch, while
    # kernel-trace durations stay within the two.
    per = 20

    def eager(fn):
        te = []
        for _ in range(8):
            a, b = ev.new(), ev.new()
            dev.sync()
            ev.record(a, dev.stream)
            for i in range(per):
                fn(i)
            ev.record(b, dev.stream)
            te.append(ev.elapsed_ms(a, b) / 1e3 / per)
        te = sorted(te[1:])                           # the first sample warms up
        return {"median_s": te[len(te) // 2], "min_s": te[0], "launches_per_sample": per, "samples": len(te)}

    mv = lambda i: dev.gemv_q4_k_q8(pool[i % 2], pk, y, rows, cols)
    st = eager(mv)
    ga = dev.capture(lambda: [dev.argmax_f32(y, rows, am) for _ in range(10)])  # 7.5 us: replayed, not host-bound
    sa = sample_launches(dev, ev, ga, 10)
    ga.close()
    # the reference's pick over these logits (model.rs:2842-2907): masks,
    # softcap, recent-token penalty, then greedy (k = 1) or the top-40 draw
    gp = dev.capture(lambda: [dev.vocab_select(y, rows, generated_count=9, k=1, token=am) for _ in range(10)])
    sp = sample_launches(dev, ev, gp, 10)
    gp.close()
    gd = dev.capture(lambda: [dev.vocab_select(y, rows, generated_count=9, temperature=0.8, pos=7, k=40, token=am)
                              for _ in range(10)])
    sd = sample_launches(dev, ev, gd, 10)
    gd.close()
    sb = eager(lambda i: (mv(i), dev.argmax_f32(y, rows, am)))
    g = dev.capture(lambda: [mv(i) for i in range(per)])
    sg = sample_launches(dev, ev, g, per)
    g.close()
    dev.sync()
    gbs = nbytes / sg["median_s"] / 1e9
    out = {"gb_s": round(gbs, 1), "gb_s_best": round(nbytes / sg["min_s"] / 1e9, 1),
           "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2), "us_median": round(sg["median_s"] * 1e6, 3),
           "us_min": round(sg["min_s"] * 1e6, 3), "bytes_per_launch": nbytes, "kernel": "gemv_q4_k_kernel",
           "argmax_us": round(sa["median_s"] * 1e6, 3),
           "pick_us": {"penalised_greedy": round(sp["median_s"] * 1e6, 3),
                       "top40_draw": round(sd["median_s"] * 1e6, 3),
                       "how": "mrml_hip_vocab_select over the 256000 logits (CPU-path scoring), 10 per graph"},
           "matvec_plus_argmax_us": round(sb["median_s"] * 1e6, 3),
           "matvec_plus_argmax_gb_s": round(nbytes / sb["median_s"] / 1e9, 1),
           "eager": {"us_median": round(st["median_s"] * 1e6, 3), "us_min": round(st["min_s"] * 1e6, 3),
                     "gb_s": round(nbytes / st["median_s"] / 1e9, 1), "launches_per_sample": per,
                     "samples": st["samples"]},
           "argmax": int(am.numpy()[0]), "launches_per_sample": sg["launches_per_sample"], "samples": sg["samples"],
           "workload": "BASELINE configs[2]: Q4_K 256000x2304 (GGUF super-blocks), batch 1, x pre-quantised, "
                       "then the greedy argmax; hipEvent around graph replays of 20 launches alternating 2 weight "
                       "copies (663 MB), median of 7 samples of >= 100 launches"}
    second.close()
    if cpu_s > 0:
        sys.path.insert(0, str(ROOT))
        from oracle import orc
        threads = len(os.sched_getaffinity(0))
        xq = orc.quantize_q8_0(x)
        sub = 32000                                   # a row sample: 1/8 of the matrix
        ws = w[:sub * (cols // 256) * 144]
        best, rounds = cpu_best_of(lambda: orc.mat_vec_mul_q4_k_q8_0(ws, xq, sub, cols, threads=threads), cpu_s)
        sbytes = sub * cols // 256 * 144 + cols * 4 + sub * 4
        out["cpu_baseline"] = {"value": round(sbytes / best / 1e9, 2), "unit": "GB/s", "cores": threads,
                               "kind": "port", "sample": f"{rounds} matvecs over the first {sub} rows (the oracle's "
                                                         f"Q4_K dot; the reference has none), best-of wall clock, "
                                                         f"{threads} threads"}
    return out


def lmhead_profile(be, synth, dev, n: int) -> dict:
    """Profiling aid for BASELINE configs[2]: n launches each of the Q4_K
    256000x2304 matvec and, for comparison, the Q4_0 matvec of the same shape
    (the tied LM head of configs[3]), each alternating two weight copies."""
    rows, cols = 256000, 2304
    rng = synth.rng_for(3)
    x = synth.normal_vector(rng, cols)
    wk = be.HipBuffer.from_gguf(dev, synth.q4_k_matrix(rng, rows, cols), be.Q4_K, rows, cols)
    w0 = be.HipBuffer.from_gguf(dev, synth.q4_0_matrix(rng, rows, cols), be.Q4_0, rows, cols)
    wk2, w02 = be.HipBuffer(dev, wk.nbytes), be.HipBuffer(dev, w0.nbytes)
    dev.copy_kernel(wk2, wk, wk.nbytes)
    dev.copy_kernel(w02, w0, w0.nbytes)
    xb = be.HipBuffer.from_host(dev, x)
    pk = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(cols), np.uint8)
    y = be.HipBuffer.alloc(dev, rows)
    dev.quantize_q8_0(xb, None, pk, cols)
    for i in range(n):
        dev.gemv_q4_k_q8(wk if i % 2 == 0 else wk2, pk, y, rows, cols)
    for i in range(n):
        dev.gemv_q4_0_q8(w0 if i % 2 == 0 else w02, pk, y, rows, cols)
    dev.sync()
    return {"profile_lmhead": n, "launches": 2 * n}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sets", type=int, default=0, help="rotating weight sets (default: > 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-seconds-small", type=float, default=3.0, help="CPU baseline budget of the C1 and C3 legs")
    ap.add_argument("--no-q8", action="store_true", help="skip BASELINE configs[0] (Q8_0 2048x2048)")
    ap.add_argument("--no-q4k", action="store_true", help="skip BASELINE configs[2] (Q4_K 256000x2304 + argmax)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-loop", type=int, default=0,
                    help="only replay the FFN step graph over the weight sets this many times (for rocprofv3)")
    ap.add_argument("--decode-prefill", type=int, default=512)
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--cpu-decode-steps", type=int, default=8)
    ap.add_argument("--gemm-batch", type=int, default=512)
    ap.add_argument("--profile-gemm", type=int, default=0,
                    help="profiling aid: N eager launches of each C5 product, then exit")
    ap.add_argument("--profile-decode", type=int, default=0,
                    help="profiling aid: prefill, then N eager decode steps of the C4 model, then exit")
    ap.add_argument("--profile-prefilled", action="store_true",
                    help="with --profile-decode: the prompt through one batched prefill call")
    ap.add_argument("--fast-numerics", action="store_true",
                    help="with --profile-decode: the FAST numerics (tree-order norm sums, split-K attention)")
    ap.add_argument("--profile-prefill", type=int, default=0,
                    help="profiling aid: one chunked prefill of N tokens of the C4 model, then exit")
    ap.add_argument("--profile-lmhead", type=int, default=0,
                    help="profiling aid: N launches each of the Q4_K and Q4_0 256000x2304 matvecs, then exit")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--cpu-gemm-tokens", type=int, default=64)
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
    if args.profile_gemm:
        print(json.dumps(gemm_bench(be, synth, dev, ev, args.gemm_batch, 0, profile=args.profile_gemm)))
        return 0
    if args.profile_decode:
        print(json.dumps(decode_profile(be, synth, dev, args.decode_prefill, args.profile_decode,
                                        be.NUMERICS_FAST if args.fast_numerics else be.NUMERICS_EXACT,
                                        args.profile_prefilled)))
        return 0
    if args.profile_lmhead:
        print(json.dumps(lmhead_profile(be, synth, dev, args.profile_lmhead)))
        return 0
    if args.profile_prefill:
        print(json.dumps(prefill_profile(be, synth, dev, args.profile_prefill)))
        return 0

    # ---- synthetic config-2 data: `sets` copies of gate, up and down (the
    # default 15 sets: 45 matrices, 537 MB, more than twice the MALL).  FFN
    # step i uses pool entries 3j, 3j+1, 3j+2 with j = i mod sets; the
    # per-matrix rates rotate one kernel over all entries (the three matrices
    # have the same bytes, and the timing does not depend on the values).
    rng = synth.rng_for(2)
    host = {"g": synth.q4_0_matrix(rng, FFN, DIM), "u": synth.q4_0_matrix(rng, FFN, DIM),
            "d": synth.q4_0_matrix(rng, DIM, FFN)}
    x = synth.rms_normalised(synth.normal_vector(rng, DIM))
    sets = args.sets or int(np.ceil(2 * MALL_BYTES / (3 * W_BYTES)))
    first = {"g": be.HipBuffer.from_gguf(dev, host["g"], be.Q4_0, FFN, DIM),
             "u": be.HipBuffer.from_gguf(dev, host["u"], be.Q4_0, FFN, DIM),
             "d": be.HipBuffer.from_gguf(dev, host["d"], be.Q4_0, DIM, FFN)}
    rot = [first]
    for _ in range(sets - 1):
        s = {k: be.HipBuffer(dev, v.nbytes) for k, v in first.items()}
        for k in s:
            dev.copy_kernel(s[k], first[k], first[k].nbytes)
        rot.append(s)
    pool = [s[k] for s in rot for k in ("g", "u", "d")]
    bx = be.HipBuffer.from_host(dev, x)
    act = be.HipBuffer.alloc(dev, FFN)
    y = be.HipBuffer.alloc(dev, DIM)
    dev.reserve_workspace(1 << 20)
    dev.sync()

    # one FFN step = mrml_hip_ffn_geglu_q4_0: two launches (the GeGLU
    # quantising x itself, 256 workgroups of 36 rows, writing the f32 output
    # and the pack blocks it holds whole, its staging waves reading the down
    # projection's rows ahead into the caches; then the down projection,
    # which quantises the 32 tail blocks itself)
    def ffn_step(s):
        dev.ffn_geglu_q4_0(s["g"], s["u"], s["d"], bx, None, y, DIM, FFN)

    for s in rot:
        ffn_step(s)
    dev.sync()
    graphs = {}

    def steps_graph(n):
        """A graph of n consecutive FFN steps (n <= sets), cached."""
        if n not in graphs:
            graphs[n] = dev.capture(lambda: [ffn_step(rot[i]) for i in range(n)])
        return graphs[n]

    def run_steps(n):
        for _ in range(n // sets):
            steps_graph(sets).launch()
        if n % sets:
            steps_graph(n % sets).launch()

    q_pack = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(DIM), np.uint8)
    dev.quantize_q8_0(bx, None, q_pack, DIM)
    a_pack = be.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(FFN), np.uint8)

    if args.profile_loop:
        # the FFN step (GeGLU then down) over every weight set, N times
        for _ in range(args.profile_loop):
            steps_graph(sets).launch()
        dev.sync()
        print(json.dumps({"profile_loop": args.profile_loop, "steps": args.profile_loop * sets,
                          "source_sha256_16": kernel_source_hash()}))
        return 0

    # ---- W warm-up steps, then timed regions of exactly K steps each
    K, W = args.steps, args.warmup
    run_steps(W)
    steps_graph(sets)
    if K % sets:
        steps_graph(K % sets)
    regions = max(5, -(-100 // (2 * K)))
    times = []
    for _ in range(regions):
        a, b = ev.new(), ev.new()
        dev.sync()
        ev.record(a, dev.stream)
        run_steps(K)
        ev.record(b, dev.stream)
        times.append(ev.elapsed_ms(a, b) / 1e3)
    dev.sync()
    times.sort()
    t_med, t_min = times[len(times) // 2], times[0]
    ms_per_step = t_med / K * 1e3
    value = BYTES_STEP * K / t_med / 1e9

    # ---- per-kernel rates, each kernel rotated over the whole pool
    def rate(fn, nbytes, n):
        g = dev.capture(lambda: [fn(i) for i in range(n)])
        st = sample_launches(dev, ev, g, n)
        g.close()
        return st, nbytes / st["median_s"] / 1e9

    out_f = be.HipBuffer.alloc(dev, FFN)
    npool = len(pool)
    # the step's first launch (f32 x in, activation pack out), over gate/up
    # pairs of the pool, as it runs in the step: reading the next matrix of the
    # pool ahead as the step's GeGLU reads its down projection (11.99 MB more
    # from HBM a launch, not counted in its bytes); and without the read-ahead
    st_geglu, gbs_geglu = rate(lambda i: dev.ffn_split_geglu(pool[2 * i], pool[2 * i + 1], bx, act, a_pack, DIM,
                                                             FFN, w_down_next=pool[(2 * i + 2) % npool]),
                               BYTES_GEGLU, npool // 2)
    st_geglu_own, gbs_geglu_own = rate(lambda i: dev.ffn_split_geglu(pool[2 * i], pool[2 * i + 1], bx, act, a_pack,
                                                                     DIM, FFN), BYTES_GEGLU, npool // 2)
    st_geglu_e, gbs_geglu_e = rate(lambda i: dev.gemv_q4_0_geglu_pack(pool[2 * i], pool[2 * i + 1], bx, None, a_pack,
                                                                      FFN, DIM), BYTES_GEGLU, npool // 2)
    st_gate, gbs_gate = rate(lambda i: dev.gemv_q4_0_q8(pool[i], q_pack, out_f, FFN, DIM), BYTES_GATE, npool)
    st_up, gbs_up = rate(lambda i: dev.gemv_q4_0_q8(pool[(i + 1) % npool], q_pack, out_f, FFN, DIM), BYTES_GATE,
                         npool)
    # the step's second launch (the pack's whole blocks and the f32 activations in)
    st_down, gbs_down = rate(lambda i: dev.ffn_split_down(pool[i], a_pack, act, y, DIM, FFN), BYTES_DOWN, npool)
    st_down_e, gbs_down_e = rate(lambda i: dev.gemv_q4_0_q8(pool[i], a_pack, y, DIM, FFN), BYTES_DOWN, npool)
    # the previous two-launch form of the step: the GeGLU emitting the
    # activation pack (32-row workgroups), the down projection reading it
    g_emit = dev.capture(lambda: [(dev.gemv_q4_0_geglu_pack(s_["g"], s_["u"], bx, None, a_pack, FFN, DIM),
                                   dev.gemv_q4_0_q8(s_["d"], a_pack, y, DIM, FFN)) for s_ in rot])
    st_emit = sample_launches(dev, ev, g_emit, sets)
    g_emit.close()
    k_geglu = st_geglu["median_s"]
    # the tolerance path's FFN step (not the headline): the same GeGLU launch,
    # then the down projection with tree-order row sums
    # (mrml_hip_gemv_q4_0_q8_relaxed, within 1e-5 of the exact product)
    st_down_r, gbs_down_r = rate(lambda i: dev.gemv_q4_0_q8_relaxed(pool[i], a_pack, y, DIM, FFN), BYTES_DOWN, npool)
    g_fast = dev.capture(lambda: [(dev.gemv_q4_0_geglu_pack(s_["g"], s_["u"], bx, None, a_pack, FFN, DIM),
                                   dev.gemv_q4_0_q8_relaxed(s_["d"], a_pack, y, DIM, FFN)) for s_ in rot])
    st_fast = sample_launches(dev, ev, g_fast, len(rot))
    g_fast.close()
    # stream-copy ceiling on a buffer well above the MALL
    cbytes = 1 << 30
    src, dst = be.HipBuffer(dev, cbytes), be.HipBuffer(dev, cbytes)
    gc = dev.capture(lambda: dev.copy_kernel(dst, src, cbytes))
    time_graph(dev, ev, gc, 2)
    tc = time_graph(dev, ev, gc, 10) / 10
    copy_gbs = 2 * cbytes / tc / 1e9
    gc.close()
    # launch floor inside a graph, with product kernels: a 256-byte zero fill
    # (no memory traffic to speak of) and a copy of one 11.94 MB matrix
    zb = be.HipBuffer(dev, 256)
    gz = dev.capture(lambda: [dev.zero(zb, 256) for _ in range(100)])
    st_zero = sample_launches(dev, ev, gz, 100)
    gz.close()
    ncp = 24
    gcp = dev.capture(lambda: [dev.copy_kernel(dst.ptr + i * W_BYTES, src.ptr + i * W_BYTES, W_BYTES)
                               for i in range(ncp)])
    st_copy = sample_launches(dev, ev, gcp, ncp)
    gcp.close()
    dev.sync()
    floors = read_floors(be, dev, ev)

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT))
        from oracle import orc
        cpu = cpu_baseline(orc, synth, args.cpu_seconds)
    # release the FFN bench buffers before the other legs
    for g_ in graphs.values():
        g_.close()
    del rot, first, pool, src, dst
    q8 = None if args.no_q8 else q8_0_bench(be, synth, dev, ev, 0 if args.no_cpu else args.cpu_seconds_small)
    q4k = None if args.no_q4k else q4_k_bench(be, synth, dev, ev, 0 if args.no_cpu else args.cpu_seconds_small)
    gemm = None
    if not args.no_gemm:
        gemm = gemm_bench(be, synth, dev, ev, args.gemm_batch, 0 if args.no_cpu else args.cpu_gemm_tokens)
    decode, decode_cpu = (None, None)
    if not args.no_decode:
        decode, decode_cpu = decode_bench(be, synth, dev, ev, args.decode_prefill, args.decode_tokens,
                                          0 if args.no_cpu else args.cpu_decode_steps)
        decode["fast"] = decode_fast_bench(be, synth, dev, ev, args.decode_prefill, args.decode_tokens,
                                           decode.pop("_exact_hist"))
    # each matvec against the read floor of its own bytes (floor µs / kernel µs)
    vs_floor = {"gate": floors["gate_9216x2304"]["us"] / (st_gate["median_s"] * 1e6),
                "down": floors["gate_9216x2304"]["us"] / (st_down["median_s"] * 1e6),
                "fused_gate_up_geglu": floors["geglu_2x9216x2304"]["us"] / (k_geglu * 1e6),
                "ffn_step": (floors["geglu_2x9216x2304"]["us"] + floors["gate_9216x2304"]["us"]) / ms_per_step / 1e3}
    if q8:
        vs_floor["q8_0"] = floors["q8_0_2048x2048"]["us"] / q8["us_median"]
    if q4k:
        vs_floor["q4_k"] = floors["lm_head_256000x2304"]["us"] / q4k["us_median"]

    line = {
        "metric": "Q4_0 matvec GB/s (Gemma-2-2B FFN: fused gate+up GeGLU + down, batch 1)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 -> int32, f32 fold",
        "data": "synthetic (seeded GGUF Q4_0 bytes, N(0,1) RMS-normalised x)",
        "config": {"workload": "BASELINE configs[1]: Q4_0 gate/up 9216x2304 + down 2304x9216, batch 1",
                   "bytes_per_step": BYTES_STEP, "rotating_weight_sets": sets,
                   "rotating_bytes": sets * 3 * W_BYTES,
                   "timing": f"hipEvent around graph replays: {W} warm-up steps, then {regions} timed regions of "
                             f"exactly {K} steps (2 launches each); value from the median region"},
        "timed_regions": regions,
        "ms_per_step_min": round(t_min / K * 1e3, 5),
        "value_best": round(BYTES_STEP * K / t_min / 1e9, 2),
        "pct_of_hbm_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "per_matrix_gbs": {"gate": round(gbs_gate, 1), "up": round(gbs_up, 1), "down": round(gbs_down, 1),
                           "fused_gate_up_geglu": round(gbs_geglu, 1)},
        "ffn_tolerance_path": {"gb_s": round(BYTES_STEP / st_fast["median_s"] / 1e9, 1),
                               "us_per_step": round(st_fast["median_s"] * 1e6, 3),
                               "down_relaxed_us": round(st_down_r["median_s"] * 1e6, 3),
                               "down_relaxed_gb_s": round(gbs_down_r, 1),
                               "how": "GeGLU launch as in the headline, then mrml_hip_gemv_q4_0_q8_relaxed (tree-order "
                                      "row sums, within 1e-5 of the exact product); graph replays over the weight sets; "
                                      "not the headline, which stays bit-exact"},
        "per_kernel_us": {k_: {"median": round(v_["median_s"] * 1e6, 3), "min": round(v_["min_s"] * 1e6, 3),
                               "launches_per_sample": v_["launches_per_sample"]}
                          for k_, v_ in (("geglu", st_geglu), ("geglu_no_read_ahead", st_geglu_own), ("gate", st_gate),
                                         ("up", st_up), ("down", st_down), ("geglu_emit_pack", st_geglu_e),
                                         ("down_from_pack", st_down_e))},
        "down_in_step_us": round(ms_per_step * 1e3 - k_geglu * 1e6, 3),
        "per_kernel_how": "each launch alone over the pool (graph replays); geglu as in the step, reading the next "
                          "down-shaped matrix ahead; down alone reads its weights from HBM, while in the step it finds "
                          "them read ahead (down_in_step_us = step time minus the GeGLU launch, boundary included)",
        "ffn_emit_pack_form": {"gb_s": round(BYTES_STEP / st_emit["median_s"] / 1e9, 1),
                               "us_per_step": round(st_emit["median_s"] * 1e6, 3),
                               "how": "the GeGLU emitting the Q8_0 activation pack (288 workgroups of 32 rows), then "
                                      "the down projection reading it; graph replays over the weight sets"},
        "per_matrix_rotation": f"each kernel over all {sets * 3} pool matrices ({sets * 3 * W_BYTES} B)",
        "stream_copy_gbs": round(copy_gbs, 1),
        "read_floor": {"sizes": floors,
                       "how": "mrml_hip_read_kernel (16-byte non-temporal loads, nothing written) over slices of a "
                              "700 MB buffer, graph replays, median per launch: the one-launch floor for those bytes"},
        "matvec_vs_read_floor": {k_: round(v_, 3) for k_, v_ in vs_floor.items()},
        "launch_floor": {"zero_fill_256B_us": round(st_zero["median_s"] * 1e6, 3),
                         "copy_11.94MB_us": round(st_copy["median_s"] * 1e6, 3),
                         "how": "product kernels (mrml_hip_zero_async, mrml_hip_copy_kernel) replayed in a graph, "
                                "median per launch"},
        "roofline": {"bound": "hbm", "kernel": GEGLU_KERNEL, "achieved": round(gbs_geglu, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs_geglu / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(GEGLU_KERNEL), "bytes_per_launch": BYTES_GEGLU,
                     "read_ahead_bytes_per_launch": W_BYTES,
                     "avg_launch_us": round(k_geglu * 1e6, 3), "source_sha256_16": kernel_source_hash(),
                     "note": "achieved counts the GeGLU's own bytes only; the launch also reads the down "
                             "projection's rows ahead (read_ahead_bytes_per_launch), which traffic includes"},
        "cpu_baseline": cpu,
        "q8_0": q8,
        "q4_k": q4k,
        "decode": decode,
        "decode_cpu_baseline": decode_cpu,
        "gemm": gemm,
        "device": {"name": info["name"], "compute_units": info["compute_units"]},
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
