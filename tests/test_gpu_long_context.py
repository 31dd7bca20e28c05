"""GPU parity of attention and the token step at long KV capacities (C ABI).

Capacities past 6144 positions take the long forms of the attention kernels:
the exact softmax sums the window's exps in chunks of 8191 staged in LDS,
each chunk's exact sequential sum started from the running sum, and forms
the weights again from the global scores; the split-K combine walks more
tiles than its LDS arrays hold.  Bar: bit-identical to the CPU oracle
(model.rs:1457-1590, ops.rs:133-158) for the exact path at every window up
to 131072 positions (test_gpu_attention_any.py takes a 262144-position
window; the ops take capacities up to 2^20); within 1e-5 relative to
the output's largest magnitude for the split path.  The reference serves
such windows with its streaming online-softmax kernel (kernels.rs:1463-1561,
dispatch cuda.rs:1097-1126).
"""

from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import THREADS, TINY, assert_bits, check_pack, max_rel

pytestmark = pytest.mark.gpu

MAX_CAP = 131072            # the longest window these tests run (2^17, Gemma-2's longest context)
CAP_LIMIT = 1 << 20         # the largest capacity the attention entries take
SPLIT_TOL = 1e-5


def window_rows(n_past: int, cap: int) -> np.ndarray:
    """Cache rows of the window: the last min(n_past + 1, cap) positions, oldest first."""
    count = n_past + 1
    return np.arange(max(0, count - cap), count) % cap


def long_case(backend, dev, n_past, cap, seed, split, nh=8, nkv=4, qscale=0.5):
    hd = 256
    rng = np.random.default_rng(3700 + seed)
    kvd = nkv * hd
    q = rng.standard_normal(nh * hd, dtype=np.float32) * np.float32(qscale)
    kc = rng.standard_normal(cap * kvd, dtype=np.float32).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(cap * kvd, dtype=np.float32).astype(np.float16).view(np.uint16)
    qb, kb, vb = (backend.HipBuffer.from_host(dev, a) for a in (q, kc, vc))
    out = backend.HipBuffer.alloc(dev, nh * hd)
    pk = backend.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(nh * hd), np.uint8)
    fn = dev.attention_causal_split if split else dev.attention_causal
    fn(qb, kb, vb, out, n_past, nh, nkv, hd, 1.0 / 16.0, cap, pack=pk)
    dev.sync()
    got, pack = out.numpy(), pk.numpy()
    for b in (qb, kb, vb, out, pk):
        b.close()
    rows = window_rows(n_past, cap)
    kr = kc.reshape(cap, kvd)[rows].reshape(-1)
    vr = vc.reshape(cap, kvd)[rows].reshape(-1)
    return got, pack, q, kr, vr


def attention_f64(q, kr, vr, nh, nkv, hd, scale):
    """softmax(scale q.K) V per head in float64: the value both paths round."""
    K = kr.view(np.float16).reshape(-1, nkv, hd)
    V = vr.view(np.float16).reshape(-1, nkv, hd)
    out = np.empty(nh * hd, np.float64)
    for g in range(nkv):
        Kg, Vg = K[:, g, :].astype(np.float64), V[:, g, :].astype(np.float64)
        for h in range(g * (nh // nkv), (g + 1) * (nh // nkv)):
            s = Kg @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
            w = np.exp(s - s.max())
            out[h * hd:(h + 1) * hd] = (w / w.sum()) @ Vg
    return out


# (n_past, capacity): the LDS form's last capacity, the long form at windows
# in registers (<= 2048), in one chunk, across the chunk boundary (8191
# terms a chunk) and over whole chunks, ring windows of a non-power-of-two
# capacity, and the largest capacity with a full window
LONG_CASES = [(6143, 6144), (0, 6145), (1500, 8192), (4000, 8192), (8190, 8192), (8191, 8192), (16381, 16384),
              (16383, 16384), (12000, 7000), (40000, 24577)]


@pytest.mark.parametrize("n_past,cap", LONG_CASES)
def test_attention_long_bit_exact(backend, orc, dev, n_past, cap):
    got, pack, q, kr, vr = long_case(backend, dev, n_past, cap, n_past % 97, split=False)
    ref = orc.attention_f16(q, kr, vr, len(kr) // 1024 - 1, 8, 4, 256, 1.0 / 16.0)
    assert_bits(got, ref, f"attention n_past {n_past} capacity {cap}")
    check_pack(orc, pack, got, "long attention")


def test_attention_long_max_capacity_bit_exact(backend, orc, dev):
    """A full window of 131072 positions: bit-exact."""
    n_past = MAX_CAP - 1
    print(f"\n[long attn] exact, n_past {n_past} capacity {MAX_CAP}", flush=True)
    got, pack, q, kr, vr = long_case(backend, dev, n_past, MAX_CAP, 5, split=False)
    ref = orc.attention_f16(q, kr, vr, n_past, 8, 4, 256, 1.0 / 16.0)
    assert_bits(got, ref, "attention at the largest capacity")
    check_pack(orc, pack, got, "attention at the largest capacity")


def test_attention_long_capacity_limit(backend, dev):
    """A capacity past the entries' limit is refused before any launch (the
    caches here are far too small for any real call: nothing may run)."""
    qb = backend.HipBuffer.alloc(dev, 8 * 256)
    kb = backend.HipBuffer.alloc(dev, 64, np.uint16)
    out = backend.HipBuffer.alloc(dev, 8 * 256)
    for fn in (dev.attention_causal, dev.attention_causal_split):
        with pytest.raises(backend.HipError):
            fn(qb, kb, kb, out, 0, 8, 4, 256, 1.0 / 16.0, CAP_LIMIT + 1)


# split-K: the combine's LDS arrays hold 192 tiles (6144 positions); longer
# windows walk the tiles where they lie
SPLIT_LONG_CASES = [(6143, 6144), (6144, 8192), (8191, 8192), (12000, 7000), (30000, 32768)]


@pytest.mark.parametrize("n_past,cap", SPLIT_LONG_CASES)
def test_attention_split_long_within_tolerance(backend, orc, dev, n_past, cap):
    got, pack, q, kr, vr = long_case(backend, dev, n_past, cap, 11 + n_past % 89, split=True)
    ref = orc.attention_f16(q, kr, vr, len(kr) // 1024 - 1, 8, 4, 256, 1.0 / 16.0)
    err = max_rel(got, ref)
    print(f"\n[split long] n_past {n_past} capacity {cap}: max-rel {err:.2e}", flush=True)
    assert err <= SPLIT_TOL
    check_pack(orc, pack, got, "long split attention")


def test_attention_split_max_capacity(backend, orc, dev):
    """Full window at the largest capacity.  Over 131072 terms the sequential
    f32 sums of the CPU path themselves drift from the exact value by about
    1e-5 of the output, so the split path is held to 1e-5 of the float64
    attention, and to twice the CPU path's own distance from it."""
    n_past = MAX_CAP - 1
    got, _, q, kr, vr = long_case(backend, dev, n_past, MAX_CAP, 6, split=True)
    ref = orc.attention_f16(q, kr, vr, n_past, 8, 4, 256, 1.0 / 16.0)
    exact = attention_f64(q, kr, vr, 8, 4, 256, 1.0 / 16.0)
    e_gpu, e_cpu = max_rel(got, exact), max_rel(ref, exact)
    print(f"\n[split long] capacity {MAX_CAP}: split vs f64 {e_gpu:.2e}, CPU path vs f64 {e_cpu:.2e}, "
          f"split vs CPU path {max_rel(got, ref):.2e}", flush=True)
    assert e_gpu <= SPLIT_TOL
    assert e_gpu <= max(2.0 * e_cpu, 1e-6)


@pytest.mark.parametrize("numerics", [0, 1])
def test_gemma2_tiny_long_context(backend, dev, orc, synth, numerics):
    """The whole model at the largest capacity: caches holding 9000 seeded
    rows (the same rows in the oracle's), then a 200-token prefill from
    position 9000 (one chunk, attention rows in launches of 64 so the
    scores stay within their bound) and 4 token steps replayed from a graph.
    EXACT: the cache rows written, the prefill's last logits and every
    step's logits are bit-identical to the oracle's token steps.  FAST: the
    logits within the bound of the FAST tiny-model test (each op within 1e-5;
    a quantised activation may move by one quantum)."""
    cfg = dict(TINY, ctx_len=MAX_CAP)
    model = synth.gemma2_model(cfg, seed=21)
    P0, n_pf, n_st = 9000, 200, 4
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    rng = np.random.default_rng(23)
    fill = np.zeros((cfg["n_layers"], MAX_CAP, kvd), np.uint16)
    fill[:, :P0] = rng.standard_normal((cfg["n_layers"], P0, kvd), dtype=np.float32).astype(np.float16).view(np.uint16)
    kfill = fill.reshape(-1)
    vfill = np.ascontiguousarray(fill[:, :, ::-1]).reshape(-1)
    del fill
    toks = synth.prompt_tokens(P0 + n_pf + n_st, cfg["vocab"], seed=3)
    o = orc.OracleGemma2(model)
    o.k_cache[:] = kfill
    o.v_cache[:] = vfill
    lg = np.zeros(cfg["vocab"], np.float32)
    ref = []
    for i in range(n_pf + n_st):
        o.step(int(toks[P0 + i]), P0 + i, threads=THREADS, logits=lg)
        ref.append(lg.copy())

    m = backend.Gemma2Model.from_host(dev, model, numerics=numerics)
    kc = backend.HipBuffer.from_host(dev, kfill)
    vc = backend.HipBuffer.from_host(dev, vfill)
    tb = backend.HipBuffer.from_host(dev, np.asarray(toks, np.int32))
    logits = backend.HipBuffer.alloc(dev, cfg["vocab"])
    print(f"\n[long model] numerics {numerics}: prefill {n_pf} at {P0}, capacity {MAX_CAP}", flush=True)
    m.prefill(tb.ptr + 4 * P0, n_pf, P0, kc, vc, logits=logits)
    dev.sync()
    lg_pf = logits.numpy()
    P1 = P0 + n_pf
    state = backend.HipBuffer.from_host(dev, np.array([toks[P1], P1], np.int32))
    hist = backend.HipBuffer.from_host(dev, np.full(P1 + n_st, -1, np.int32))
    g = dev.capture(lambda: m.step(state, kc, vc, logits=logits, hist=hist, hist_cap=P1 + n_st, prompt=tb,
                                   prompt_len=P1 + n_st))
    got = []
    for _ in range(n_st):
        g.launch()
        dev.sync()
        got.append(logits.numpy())
    g.close()
    rows = slice(P0, P1 + n_st)
    kg = kc.numpy().reshape(cfg["n_layers"], MAX_CAP, kvd)[:, rows]
    vg = vc.numpy().reshape(cfg["n_layers"], MAX_CAP, kvd)[:, rows]
    ko = o.k_cache.reshape(cfg["n_layers"], MAX_CAP, kvd)[:, rows]
    vo = o.v_cache.reshape(cfg["n_layers"], MAX_CAP, kvd)[:, rows]
    m.close()
    if numerics == 0:
        assert np.array_equal(kg, ko) and np.array_equal(vg, vo)
        assert_bits(lg_pf, ref[n_pf - 1], "prefill logits at the chunk's last position")
        for i in range(n_st):
            assert_bits(got[i], ref[n_pf + i], f"logits at position {P1 + i}")
    else:
        errs = [max_rel(lg_pf, ref[n_pf - 1])] + [max_rel(got[i], ref[n_pf + i]) for i in range(n_st)]
        print(f"[long model] FAST worst logit max-rel {max(errs):.2e}", flush=True)
        assert max(errs) <= 2e-2
