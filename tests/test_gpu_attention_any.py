"""Attention and the K/V append at every head size the reference's models use
and over its three cache formats (KvCacheFormat::cuda_code 0 f16, 1 Q8_0,
2 Q4_0; kv_cache.rs:16-31): bit-exact against the oracle's restatement of the
CPU loop (model.rs:1526-1547 over KvCacheRow::dot_head / add_head_scaled,
kv_cache.rs:73-125), through the C ABI (mrml_hip_attention_causal,
_attention_prefill, _rope_kv_append_f16_batch)."""

from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import assert_bits

pytestmark = pytest.mark.gpu

FMT_NAMES = {0: "f16", 1: "q8_0", 2: "q4_0"}


def window_rows(n_past, sw, cap):
    window = min(n_past + 1, cap if sw is None or sw <= 0 else min(sw, cap))
    return [t % cap for t in range(n_past + 1 - window, n_past + 1)]


def cache_bytes(orc, rows_f32: np.ndarray, fmt: int) -> np.ndarray:
    """[cap, kvd] f32 rows -> the cache's bytes in format fmt, row after row."""
    return np.concatenate([orc.kv_store(r, fmt) for r in rows_f32])


def oracle_rows(orc, q, kc, vc, n_past, sw, cap, nh, nkv, hd, scale, kf, vf):
    """Oracle attention of one query over the window's rows of ring caches."""
    rows = window_rows(n_past, sw, cap)
    kb, vb = orc.kv_row_bytes(nkv * hd, kf), orc.kv_row_bytes(nkv * hd, vf)
    kw = kc.reshape(cap, kb)[rows].reshape(-1)
    vw = vc.reshape(cap, vb)[rows].reshape(-1)
    return orc.attention_kv(q, kw, vw, len(rows) - 1, nh, nkv, hd, scale, kf, vf)


def upload_cache(backend, dev, b: np.ndarray):
    """Cache bytes on the device (padded to an even length: the ABI takes u16 caches)."""
    if b.size % 2:
        b = np.concatenate([b, np.zeros(1, np.uint8)])
    return backend.HipBuffer.from_host(dev, b)


# (n_heads, n_kv_heads, head_dim, k_format, v_format, capacity, sliding_window, n_pasts)
CASES = [
    # the reference model's global layers: 16 query and 2 kv heads of 512 (model.rs:590-595)
    (16, 2, 512, 0, 0, 4096, None, [0, 1, 63, 64, 65, 777, 4095]),
    (16, 2, 512, 1, 1, 1024, None, [0, 300, 1023]),
    (16, 2, 512, 2, 2, 1024, 512, [5, 700, 1500]),
    # head_dim 64 (the reference's own attention test) and 128
    (4, 2, 64, 0, 0, 4096, None, [0, 7, 129, 4095]),
    (8, 1, 128, 0, 0, 2048, None, [0, 100, 2047]),
    (8, 8, 128, 1, 2, 512, None, [0, 33, 511]),
    (12, 4, 128, 2, 1, 600, 200, [199, 200, 901]),
    # head_dim 256 outside the tuned kernels: quantised caches, groups past 8
    (8, 4, 256, 1, 1, 4096, None, [0, 511, 767, 4095]),
    (8, 4, 256, 2, 2, 4096, None, [0, 64, 767]),
    (8, 4, 256, 1, 0, 768, None, [767]),
    (8, 4, 256, 0, 2, 768, None, [767]),
    (32, 2, 256, 0, 0, 256, None, [0, 255]),
    # odd head sizes that are multiples of 32, the long softmax form (capacity past 6144)
    (6, 3, 96, 1, 1, 128, None, [0, 127]),
    (2, 1, 32, 2, 0, 64, None, [0, 63]),
    (4, 2, 160, 0, 1, 8192, None, [6000, 8191]),
]


@pytest.mark.parametrize("nh,nkv,hd,kf,vf,cap,sw,n_pasts", CASES)
def test_attention_any_bit_exact(backend, dev, orc, nh, nkv, hd, kf, vf, cap, sw, n_pasts):
    rng = np.random.default_rng(8000 + nh * 7 + hd + 13 * kf + vf)
    kvd = nkv * hd
    kx = rng.standard_normal((cap, kvd), dtype=np.float32)
    vx = rng.standard_normal((cap, kvd), dtype=np.float32)
    kc, vc = cache_bytes(orc, kx, kf), cache_bytes(orc, vx, vf)
    kb, vb = upload_cache(backend, dev, kc), upload_cache(backend, dev, vc)
    out = backend.HipBuffer.alloc(dev, nh * hd)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    for n_past in n_pasts:
        q = (rng.standard_normal(nh * hd) * 0.7).astype(np.float32)
        qb = backend.HipBuffer.from_host(dev, q)
        print(f"\n[attention any] heads {nh}/{nkv} hd {hd} formats {FMT_NAMES[kf]}/{FMT_NAMES[vf]} capacity {cap} "
              f"window {sw} n_past {n_past}", flush=True)
        dev.attention_causal_ref(qb, kb, vb, out, n_past, nh, nkv, hd, scale, sw, cap, kf, vf)
        dev.sync()
        ref = oracle_rows(orc, q, kc, vc, n_past, sw, cap, nh, nkv, hd, scale, kf, vf)
        assert_bits(out.numpy(), ref, f"n_past {n_past}")
        # the split (tolerance) entry serves these shapes with the exact form
        dev.attention_causal_ref(qb, kb, vb, out, n_past, nh, nkv, hd, scale, sw, cap, kf, vf, split=True)
        dev.sync()
        assert_bits(out.numpy(), ref, f"split entry, n_past {n_past}")
        qb.close()


def test_attention_reference_head_dim_64_case(backend, dev, orc):
    """ops_test.rs:375-449 (test_cuda_causal_attention_matches_cpu): 4 query
    and 2 kv heads of 64, 8 tokens, sliding window 4, capacity 8, caches of
    the truncating f32_to_f16, scale 1/8: within the test's 2e-4 of its own
    expected values, and bit-exact against the oracle."""
    nh, nkv, hd, tokens = 4, 2, 64, 8
    q = np.sin(np.arange(nh * hd, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
    keys = np.cos(np.arange(tokens * nkv * hd, dtype=np.float32) * np.float32(0.007)).astype(np.float32)
    values = np.sin(np.arange(tokens * nkv * hd, dtype=np.float32) * np.float32(0.011)).astype(np.float32)
    trunc = lambda a: np.array([orc.f32_to_f16(float(v)) for v in a], np.uint16)
    kc, vc = trunc(keys), trunc(values)
    scale = float(np.float32(1.0) / np.float32(np.sqrt(np.float32(hd))))
    qb, kb, vb = (backend.HipBuffer.from_host(dev, a) for a in (q, kc, vc))
    out = backend.HipBuffer.alloc(dev, nh * hd)
    dev.attention_causal_ref(qb, kb, vb, out, tokens - 1, nh, nkv, hd, scale, 4, tokens)
    dev.sync()
    got = out.numpy()
    k64 = kc.view(np.float16).astype(np.float64).reshape(tokens, nkv, hd)
    v64 = vc.view(np.float16).astype(np.float64).reshape(tokens, nkv, hd)
    for h in range(nh):
        kvh = h // (nh // nkv)
        sc = k64[4:, kvh] @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        w = np.exp(sc - sc.max())
        exp = (w / w.sum()) @ v64[4:, kvh]
        assert np.max(np.abs(got[h * hd:(h + 1) * hd] - exp)) < 2e-4
    ref = oracle_rows(orc, q, kc.view(np.uint8), vc.view(np.uint8), tokens - 1, 4, tokens, nh, nkv, hd, scale, 0, 0)
    assert_bits(got, ref, "reference head_dim 64 case")


@pytest.mark.parametrize("hd,kf,vf", [(64, 1, 2), (128, 2, 1), (256, 1, 1), (512, 2, 2), (512, 0, 1), (96, 2, 0)])
def test_rope_kv_append_quantised(backend, dev, orc, hd, kf, vf):
    """qkv_postprocess_batch without head norms (cuda.rs:2478-2519) into
    quantised caches: every row's q and k rotated as rope_1d_batched does and
    its k and v stored as KvCacheRow::from_f32 (kv_cache.rs:54-71) stores them
    -- the reference quantisers' bytes, bit for bit; other rows untouched."""
    nh, nkv, cap, batch, start_pos, cache_start = 8, 2, 24, 20, 37, 15  # the batch wraps the ring
    width = (nh + 2 * nkv) * hd
    rng = np.random.default_rng(8100 + hd + kf * 3 + vf)
    qkv = (rng.standard_normal(batch * width) * 2).astype(np.float32)
    qkv[5 * width + nh * hd + 3] = 0.0
    qkv[6 * width + (nh + nkv) * hd: 6 * width + (nh + nkv) * hd + 32] = 0.0  # an all-zero V block
    kvd = nkv * hd
    kb, vb = orc.kv_row_bytes(kvd, kf), orc.kv_row_bytes(kvd, vf)
    k0 = np.full(cap * kb + (cap * kb) % 2, 0xA5, np.uint8)
    v0 = np.full(cap * vb + (cap * vb) % 2, 0x5A, np.uint8)
    qb = backend.HipBuffer.from_host(dev, qkv)
    kcb, vcb = backend.HipBuffer.from_host(dev, k0), backend.HipBuffer.from_host(dev, v0)
    print(f"\n[rope kv quant] hd {hd} formats {kf}/{vf}", flush=True)
    dev.qkv_postprocess_batch(qb, kcb, vcb, start_pos, cache_start, nh, nkv, hd, 10000.0, batch, cap,
                              k_format=kf, v_format=vf)
    dev.sync()
    got = qb.numpy().reshape(batch, width)
    kc, vc = kcb.numpy()[:cap * kb].reshape(cap, kb), vcb.numpy()[:cap * vb].reshape(cap, vb)
    written = np.zeros(cap, bool)
    for i in range(batch):
        row = qkv.reshape(batch, width)[i]
        q_ref = orc.rope_1d_batched(row[:nh * hd], start_pos + i, nh, hd, 10000.0)
        k_ref = orc.rope_1d_batched(row[nh * hd:nh * hd + kvd], start_pos + i, nkv, hd, 10000.0)
        assert_bits(got[i, :nh * hd], q_ref, f"row {i} q")
        assert_bits(got[i, nh * hd:nh * hd + kvd], k_ref, f"row {i} k")
        r = (cache_start + i) % cap
        assert np.array_equal(kc[r], orc.kv_store(k_ref, kf)), f"row {i}: k cache bytes"
        assert np.array_equal(vc[r], orc.kv_store(row[nh * hd + kvd:], vf)), f"row {i}: v cache bytes"
        written[r] = True
    assert np.all(kc[~written] == 0xA5) and np.all(vc[~written] == 0x5A)


@pytest.mark.parametrize("nh,nkv,hd,kf,vf", [(16, 2, 512, 1, 1), (8, 4, 128, 2, 2), (8, 4, 256, 1, 2),
                                             (4, 4, 64, 0, 0)])
def test_attention_prefill_any(backend, dev, orc, nh, nkv, hd, kf, vf):
    """attention_prefill (cuda.rs:2727-2770) over quantised caches and other
    head sizes: row i bit-exact to the oracle at n_past = cache_start + i."""
    cap, start, batch, sw = 512, 300, 37, 128
    kvd, qd = nkv * hd, nh * hd
    rng = np.random.default_rng(8200 + hd + kf + vf)
    kc = cache_bytes(orc, rng.standard_normal((cap, kvd), dtype=np.float32), kf)
    vc = cache_bytes(orc, rng.standard_normal((cap, kvd), dtype=np.float32), vf)
    stride = qd + 2 * kvd
    q = (rng.standard_normal(batch * stride) * 0.5).astype(np.float32)
    qb, kb, vb = backend.HipBuffer.from_host(dev, q), upload_cache(backend, dev, kc), upload_cache(backend, dev, vc)
    out = backend.HipBuffer.alloc(dev, batch * qd)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    print(f"\n[prefill any] heads {nh}/{nkv} hd {hd} formats {kf}/{vf}", flush=True)
    dev.attention_prefill(qb, kb, vb, out, start, batch, nh, nkv, hd, scale, sw, cap, kf, vf, q_stride=stride)
    dev.sync()
    got = out.numpy().reshape(batch, qd)
    for i in range(batch):
        ref = oracle_rows(orc, q[i * stride:i * stride + qd], kc, vc, start + i, sw, cap, nh, nkv, hd, scale, kf, vf)
        assert_bits(got[i], ref, f"row {i}")


@pytest.mark.parametrize("hd,kf,vf", [(256, 0, 0), (128, 1, 1)])
def test_attention_past_131072(backend, dev, orc, hd, kf, vf):
    """Capacities past 2^17 (the reference's default max_context is 256000,
    model.rs:64-73): a full 262144-position window (the long softmax form,
    chunked exact sums), bit-exact."""
    nh, nkv, cap = 8, 4, 262144
    n_past = cap - 1
    kvd = nkv * hd
    rng = np.random.default_rng(8300 + hd)
    kx = rng.standard_normal((cap, kvd), dtype=np.float32)
    vx = (rng.standard_normal((cap, kvd), dtype=np.float32) * 0.5).astype(np.float32)
    if kf == 0:
        kc, vc = kx.astype(np.float16).view(np.uint8).reshape(-1), vx.astype(np.float16).view(np.uint8).reshape(-1)
    else:
        kc, vc = cache_bytes(orc, kx, kf), cache_bytes(orc, vx, vf)
    del kx, vx
    q = (rng.standard_normal(nh * hd) * 0.3).astype(np.float32)
    qb, kb, vb = backend.HipBuffer.from_host(dev, q), upload_cache(backend, dev, kc), upload_cache(backend, dev, vc)
    out = backend.HipBuffer.alloc(dev, nh * hd)
    print(f"\n[attention 262144] hd {hd} formats {kf}/{vf}", flush=True)
    dev.attention_causal_ref(qb, kb, vb, out, n_past, nh, nkv, hd, 0.0625, None, cap, kf, vf)
    dev.sync()
    ref = orc.attention_kv(q, kc, vc, n_past, nh, nkv, hd, 0.0625, kf, vf)
    assert_bits(out.numpy(), ref, "full 262144-position window")
    for b in (qb, kb, vb, out):
        b.close()


def test_attention_any_rejects(backend, dev):
    nh, nkv = 8, 4
    qb = backend.HipBuffer.alloc(dev, 4 * nh * 512)
    kb = backend.HipBuffer.alloc(dev, 64 * nkv * 512, np.uint16)
    out = backend.HipBuffer.alloc(dev, nh * 512)
    with pytest.raises(backend.HipError) as e:
        dev.attention_causal_ref(qb, kb, kb, out, 3, nh, nkv, 256, 0.0625, None, 64, 3, 0)
    assert e.value.status == -4  # MRML_HIP_E_UNSUPPORTED: no such cache format
    for hd, h, kvh in ((80, nh, nkv), (1024, nh, nkv), (256, 34, 2)):
        with pytest.raises(backend.HipError):
            dev.attention_causal_ref(qb, kb, kb, out, 3, h, kvh, hd, 0.0625, None, 64)
    with pytest.raises(backend.HipError):
        dev.attention_causal_ref(qb, kb, kb, out, 3, nh, nkv, 256, 0.0625, None, (1 << 20) + 1)
