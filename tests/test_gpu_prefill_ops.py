"""GPU parity of the batched prefill boundary and the elementwise ops (C ABI).

The entries prefill_cuda calls between its products (model.rs:2485-2522):
qkv_postprocess_batch without the Gemma-4 head norms
(mrml_hip_rope_kv_append_f16_batch, cuda.rs:2478-2519) and attention_prefill
(mrml_hip_attention_prefill, cuda.rs:2727-2770); and CudaDevice's
elementwise ops geglu / swiglu (cuda.rs:2182-2246) and rope_256k
(cuda.rs:2248-2285).  Bar: bit-identical to the CPU oracle (ops.rs:99-130,
185-208; model.rs:1457-1590), RoPE angles from the host table or evaluated
on the device with the host libm's cosf/sinf algorithm.
"""

from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import assert_bits

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------ geglu / swiglu
def glu_inputs(n, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 4.0).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    # exp overflow and underflow, signed zeros, the tails of tanh
    edge = np.array([0.0, -0.0, 88.0, 88.8, 89.0, -88.0, -103.0, -104.0, 1e-30, -1e-30, 20.0, -20.0, 9.0, -9.0,
                     1e30, -1e30], np.float32)
    k = min(n, edge.size)
    g[:k] = edge[:k]
    return g, u


@pytest.mark.parametrize("n", [1, 255, 256, 100003])
def test_swiglu_bit_exact(backend, dev, orc, n):
    g, u = glu_inputs(n, 4100 + n)
    gb, ub = backend.HipBuffer.from_host(dev, g), backend.HipBuffer.from_host(dev, u)
    out = backend.HipBuffer.alloc(dev, n)
    dev.swiglu(gb, ub, out, n)
    dev.sync()
    assert_bits(out.numpy(), orc.swiglu(g, u), f"swiglu n={n}")


def test_swiglu_reference_known_values(backend, dev):
    """ops_test.rs:14-24: swiglu([0, 2, -2], [1, 3, 4]) = [0, 5.28478, .]."""
    gb = backend.HipBuffer.from_host(dev, np.array([0.0, 2.0, -2.0], np.float32))
    ub = backend.HipBuffer.from_host(dev, np.array([1.0, 3.0, 4.0], np.float32))
    out = backend.HipBuffer.alloc(dev, 3)
    dev.swiglu(gb, ub, out, 3)
    dev.sync()
    got = out.numpy()
    assert got[0] == 0.0
    assert abs(got[1] - 5.28478) < 1e-3
    assert abs(got[2] - (-2.0 / (1.0 + np.exp(2.0)) * 4.0)) < 1e-5


@pytest.mark.parametrize("n", [1, 257, 100003])
def test_geglu_bit_exact(backend, dev, orc, n):
    g, u = glu_inputs(n, 4200 + n)
    gb, ub = backend.HipBuffer.from_host(dev, g), backend.HipBuffer.from_host(dev, u)
    out = backend.HipBuffer.alloc(dev, n)
    dev.geglu(gb, ub, out, n)
    dev.sync()
    assert_bits(out.numpy(), orc.geglu(g, u), f"geglu n={n}")


@pytest.mark.parametrize("n", [1, 1000, 100003])
def test_add_bit_exact(backend, dev, n):
    """CudaDevice::add (cuda.rs:2579-2593): one IEEE f32 add per element, the
    same bits as numpy's float32 add (NaN where it gives NaN), with
    infinities, NaN, signed zeros and values whose sum rounds; in place too."""
    rng = np.random.default_rng(4700 + n)
    a = (rng.standard_normal(n) * 1e3).astype(np.float32)
    b = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    special = np.array([np.inf, -np.inf, np.nan, -0.0, 0.0, 3.4e38, 1e-45, 1.0], np.float32)
    k = min(n, special.size)
    a[:k] = special[:k]
    b[:k] = special[::-1][:k]
    ab, bb = backend.HipBuffer.from_host(dev, a), backend.HipBuffer.from_host(dev, b)
    out = backend.HipBuffer.alloc(dev, n)
    dev.add(ab, bb, out, n)
    dev.add(ab, bb, ab, n)  # out aliasing an input
    dev.sync()
    with np.errstate(over="ignore", invalid="ignore"):
        ref = a + b
    nan = np.isnan(ref)  # a NaN's payload is the hardware's choice
    for got, what in ((out.numpy(), "add"), (ab.numpy(), "add in place")):
        assert np.array_equal(np.isnan(got), nan), what
        assert_bits(got[~nan], ref[~nan], f"{what} n={n}")


def test_glu_empty_and_invalid(backend, dev):
    out = backend.HipBuffer.alloc(dev, 4)
    dev.swiglu(out, out, out, 0)
    dev.geglu(out, out, out, 0)
    for fn in (dev.swiglu, dev.geglu):
        with pytest.raises(backend.HipError):
            fn(out, out, out, -1)
        with pytest.raises(backend.HipError):
            fn(None, None, None, 4)


# ------------------------------------------------------------ rope_256k
@pytest.mark.parametrize("pos", [0, 37, 4095])
@pytest.mark.parametrize("hd,nh", [(256, 8), (64, 4), (128, 3)])
@pytest.mark.parametrize("freq_scale", [1.0, 0.25])
def test_rope_256k(backend, dev, orc, pos, hd, nh, freq_scale):
    rng = np.random.default_rng(4300 + pos + hd)
    v = rng.standard_normal(nh * hd).astype(np.float32)
    ref = orc.rope_1d_batched(v, pos, nh, hd, 10000.0, freq_scale)
    cap = 4096
    table = backend.HipBuffer.alloc(dev, cap * hd)
    dev.rope_table(table, cap, hd, 10000.0, freq_scale)
    vb = backend.HipBuffer.from_host(dev, v)
    dev.rope_256k(vb, pos, hd, nh, 10000.0, freq_scale, table=table, n_table=cap)
    dev.sync()
    assert_bits(vb.numpy(), ref, f"rope_256k pos {pos} head_dim {hd} (table)")
    # no table: powf in double rounded once (equal to the host's powf at base
    # 10000 for these head sizes), cosf/sinf in the host libm's algorithm
    vb.copy_from_host(v)
    dev.rope_256k(vb, pos, hd, nh, 10000.0, freq_scale)
    dev.sync()
    got = vb.numpy()
    assert_bits(got, ref, f"rope_256k pos {pos} head_dim {hd} (device angles)")
    if pos == 0:
        assert_bits(got, v, "rope at position 0 is the identity")


@pytest.mark.parametrize("pos", [131071, 262143, 1 << 24, 100000007])
def test_rope_256k_far_positions(backend, dev, orc, pos):
    """Positions far past any table (rope_256k's name: 256k positions and
    more): the angles' large-argument reduction (Payne-Hanek) against the
    host libm, bit-exact."""
    hd, nh = 256, 8
    v = np.random.default_rng(4350 + pos % 1000).standard_normal(nh * hd).astype(np.float32)
    vb = backend.HipBuffer.from_host(dev, v)
    dev.rope_256k(vb, pos, hd, nh, 10000.0)
    dev.sync()
    assert_bits(vb.numpy(), orc.rope_1d_batched(v, pos, nh, hd, 10000.0), f"rope_256k at position {pos}")


@pytest.mark.parametrize("base", [10000.0, 500000.0, 1000000.0])
def test_rope_256k_random_positions(backend, dev, orc, base):
    """256 random positions below 2^24 (both reductions of the angle: the
    fast one below 120 and Payne-Hanek above), 512 pairs each (head_dim
    1024, so 131072 angles per base), device angles against the oracle's
    host cosf/sinf: bit-exact.  The host's powf equals powf in double
    rounded once at every pair of these bases and head size."""
    hd, nh = 1024, 1
    rng = np.random.default_rng(4360 + int(base) % 997)
    positions = np.concatenate([rng.integers(0, 200, 64), rng.integers(0, 1 << 24, 192)])
    v = rng.standard_normal(nh * hd).astype(np.float32)
    vb = backend.HipBuffer.from_host(dev, v)
    outs = []
    for pos in positions:
        vb.copy_from_host(v)
        dev.rope_256k(vb, int(pos), hd, nh, base)
        outs.append(vb.numpy())
    for pos, got in zip(positions, outs):
        assert_bits(got, orc.rope_1d_batched(v, int(pos), nh, hd, base), f"rope_256k base {base} position {pos}")


def test_rope_256k_invalid(backend, dev):
    vb = backend.HipBuffer.alloc(dev, 256)
    for pos, hd, nh in ((-1, 256, 1), (0, 255, 1), (0, 2048, 1), (0, 256, 0)):
        with pytest.raises(backend.HipError):
            dev.rope_256k(vb, pos, hd, nh, 10000.0)


# ------------------------------------------------------------ qkv_postprocess_batch
# (start_pos, cache_start, batch, capacity): prefill_cuda's start_pos ==
# cache_start, a chunk past position 0, a ring wrap inside the batch, and
# rotation positions apart from the cache rows
QKV_CASES = [(0, 0, 16, 16), (128, 128, 37, 512), (60, 60, 9, 64), (100, 3, 5, 16), (4090, 10, 6, 4096)]


@pytest.mark.parametrize("start_pos,cache_start,batch,cap", QKV_CASES)
@pytest.mark.parametrize("use_table", [True, False])
def test_qkv_postprocess_batch(backend, dev, orc, start_pos, cache_start, batch, cap, use_table):
    nh, nkv, hd = 8, 4, 256
    kvd, width = nkv * hd, (nh + 2 * nkv) * hd
    rng = np.random.default_rng(4400 + start_pos + batch)
    qkv = rng.standard_normal(batch * width).astype(np.float32)
    qb = backend.HipBuffer.from_host(dev, qkv)
    kc = backend.HipBuffer.from_host(dev, np.zeros(cap * kvd, np.uint16))
    vc = backend.HipBuffer.from_host(dev, np.zeros(cap * kvd, np.uint16))
    table, n_table = None, 0
    if use_table:
        n_table = start_pos + batch
        table = backend.HipBuffer.alloc(dev, n_table * hd)
        dev.rope_table(table, n_table, hd, 10000.0)
    dev.qkv_postprocess_batch(qb, kc, vc, start_pos, cache_start, nh, nkv, hd, 10000.0, batch, cap, table=table,
                              n_table=n_table)
    dev.sync()
    got = qb.numpy().reshape(batch, width)
    kh, vh = kc.numpy().reshape(cap, kvd), vc.numpy().reshape(cap, kvd)
    written = np.zeros(cap, bool)
    for i in range(batch):
        row = qkv.reshape(batch, width)[i]
        q_ref = orc.rope_1d_batched(row[:nh * hd], start_pos + i, nh, hd, 10000.0)
        k_ref = orc.rope_1d_batched(row[nh * hd:nh * hd + kvd], start_pos + i, nkv, hd, 10000.0)
        q_got, k_got = got[i, :nh * hd], got[i, nh * hd:nh * hd + kvd]
        assert_bits(q_got, q_ref, f"batch row {i} q")
        assert_bits(k_got, k_ref, f"batch row {i} k")
        assert_bits(got[i, nh * hd + kvd:], row[nh * hd + kvd:], f"batch row {i} v unchanged")
        r = (cache_start + i) % cap
        assert np.array_equal(kh[r], k_got.astype(np.float16).view(np.uint16))
        assert np.array_equal(vh[r], row[nh * hd + kvd:].astype(np.float16).view(np.uint16))
        written[r] = True
    assert not kh[~written].any() and not vh[~written].any()

    # the same rows one at a time through the single-token entry, when the
    # cache rows follow the positions: the same bits, table or not
    if start_pos == cache_start:
        qb1 = backend.HipBuffer.from_host(dev, qkv)
        kc1 = backend.HipBuffer.from_host(dev, np.zeros(cap * kvd, np.uint16))
        vc1 = backend.HipBuffer.from_host(dev, np.zeros(cap * kvd, np.uint16))
        for i in range(batch):
            dev._check(dev.lib.mrml_hip_rope_kv_append_f16(dev.ctx, qb1.ptr + 4 * i * width, kc1.ptr, vc1.ptr,
                                                           start_pos + i, None, nh, nkv, hd, 10000.0, 1.0, cap,
                                                           table.ptr if table else None, n_table))
        dev.sync()
        assert_bits(got.reshape(-1), qb1.numpy(), "batched rows equal the single-token entry")
        assert np.array_equal(kc1.numpy(), kc.numpy()) and np.array_equal(vc1.numpy(), vc.numpy())


def test_qkv_postprocess_batch_invalid(backend, dev):
    nh, nkv, hd = 8, 4, 256
    qb = backend.HipBuffer.alloc(dev, 20 * (nh + 2 * nkv) * hd)
    kc = backend.HipBuffer.alloc(dev, 16 * nkv * hd, np.uint16)
    bad = [dict(batch=17, cap=16), dict(batch=4, cap=16, k_format=3), dict(batch=4, cap=16, v_format=-1),
           dict(batch=0, cap=16), dict(batch=4, cap=16, start_pos=-1)]
    for b in bad:
        with pytest.raises(backend.HipError):
            dev.qkv_postprocess_batch(qb, kc, kc, b.get("start_pos", 0), 0, nh, nkv, hd, 10000.0, b["batch"],
                                      b["cap"], k_format=b.get("k_format", 0), v_format=b.get("v_format", 0))


# ------------------------------------------------------------ attention_prefill
def window_rows(n_past, sw, cap):
    window = min(n_past + 1, cap if sw is None or sw <= 0 else min(sw, cap))
    return [t % cap for t in range(n_past + 1 - window, n_past + 1)]


# (cache_start, batch, sliding_window, capacity, n_heads, n_kv_heads, stacked q):
# prefill_cuda's first chunk over the stacked projection, a later chunk, a
# sliding window shorter than the chunk, a ring whose window covers the
# whole capacity, a group of 8 query heads per kv head, the long softmax form
# (capacity past 6144), a batch split over two launches (40 rows of 2 MiB of
# scores against a 64 MiB bound), and windows past 2048 in the prefill
# softmax form (groups of 2 and 4)
PREFILL_CASES = [(0, 16, None, 16, 8, 4, True), (128, 37, None, 512, 8, 4, True), (200, 40, 24, 256, 8, 4, True),
                 (300, 9, 64, 64, 8, 4, False), (700, 64, None, 2048, 8, 8, False), (20, 7, 5, 32, 16, 2, True),
                 (6000, 3, None, 8192, 8, 4, False), (100, 40, None, 65536, 8, 4, True),
                 (3000, 20, None, 4096, 8, 4, True), (3900, 9, None, 4096, 16, 4, False),
                 # the rows form at groups of 4 and 3 (spans ~2000-4000)
                 (1990, 10, None, 4096, 16, 4, False), (3290, 10, None, 4096, 16, 4, True),
                 (2490, 12, None, 4096, 12, 4, False), (3990, 6, None, 4096, 12, 4, True),
                 # windows up to 1024 (each thread's exps in registers) at groups
                 # of 4 and 3, and both sides of that bound (spans 1024, 1025)
                 (500, 24, None, 4096, 16, 4, False), (900, 30, None, 1024, 12, 4, True),
                 (1000, 24, None, 4096, 8, 4, True), (1001, 24, None, 4096, 8, 4, False)]


def prefill_span(cache_start, batch, sw, cap):
    """The widest row window of a launch (launch_attn_rows_f16's span)."""
    wlimit = sw if sw is not None and 0 < sw < cap else cap
    return min(wlimit, cache_start + batch)


def rows_form(nh, nkv, span):
    """Whether attention_prefill runs attn_softmax_v_rows_kernel (the form
    whose workgroup serves a kv head's whole group) rather than the
    per-head attn_softmax_v_kernel: windows up to 4096, groups up to 4, and
    the group's weights (a row of span floats per head, at a stride rounded
    up to 4 floats) plus span flag bytes within 60 KiB of dynamic LDS
    (launch_attn_rows_f16 in decode.hip)."""
    g = nh // nkv
    return span <= 4096 and g <= 4 and g * ((span + 3) & ~3) * 4 + ((span + 15) & ~15) <= 60 << 10


def test_prefill_cases_cover_both_forms():
    """The case list reaches the rows form at every group size it serves
    (1, 2, 3, 4) and the per-head form too, so no group size is covered
    only by a silent fallback."""
    forms = {}
    for start, batch, sw, cap, nh, nkv, _ in PREFILL_CASES:
        forms.setdefault((nh // nkv, rows_form(nh, nkv, prefill_span(start, batch, sw, cap))), []).append(start)
    for g in (1, 2, 3, 4):
        assert (g, True) in forms, f"no attention_prefill case takes the rows form at group {g}"
    assert any(not rows for _, rows in forms), "no case takes the per-head form"
    # the two group-of-4 and group-of-3 cases above are rows-form cases
    for start, batch, sw, cap, nh, nkv, _ in PREFILL_CASES[-4:]:
        assert rows_form(nh, nkv, prefill_span(start, batch, sw, cap))


@pytest.mark.parametrize("cache_start,batch,sw,cap,nh,nkv,stacked", PREFILL_CASES)
def test_attention_prefill_bit_exact(backend, dev, orc, cache_start, batch, sw, cap, nh, nkv, stacked):
    hd = 256
    kvd, qd = nkv * hd, nh * hd
    stride = (nh + 2 * nkv) * hd if stacked else qd
    rng = np.random.default_rng(4500 + cache_start + batch)
    q = (rng.standard_normal(batch * stride) * 0.5).astype(np.float32)
    kc = rng.standard_normal(cap * kvd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(cap * kvd).astype(np.float16).view(np.uint16)
    qb, kb, vb = (backend.HipBuffer.from_host(dev, a) for a in (q, kc, vc))
    out = backend.HipBuffer.alloc(dev, batch * qd)
    form = "rows" if rows_form(nh, nkv, prefill_span(cache_start, batch, sw, cap)) else "per-head"
    print(f"\n[attention_prefill] start {cache_start} batch {batch} window {sw} capacity {cap} heads {nh}/{nkv} "
          f"({form} form)", flush=True)
    dev.attention_prefill(qb, kb, vb, out, cache_start, batch, nh, nkv, hd, 1.0 / 16.0, sw, cap)
    dev.sync()
    got = out.numpy().reshape(batch, qd)
    for i in range(batch):
        rows = window_rows(cache_start + i, sw, cap)
        ref = orc.attention_f16(q[i * stride:i * stride + qd], kc.reshape(cap, kvd)[rows].reshape(-1),
                                vc.reshape(cap, kvd)[rows].reshape(-1), len(rows) - 1, nh, nkv, hd, 1.0 / 16.0)
        assert_bits(got[i], ref, f"prefill attention row {i} (position {cache_start + i})")


def test_attention_prefill_matches_causal_rows(backend, dev):
    """Row i of one prefill launch is the single-token attention_causal at
    n_past = cache_start + i on the same caches (the reference's two kernels
    are one kernel at batch 1, cuda.rs:2658-2770)."""
    nh, nkv, hd, cap, start, batch, sw = 8, 4, 256, 1024, 900, 50, 300
    rng = np.random.default_rng(4600)
    qd, kvd = nh * hd, nkv * hd
    q = rng.standard_normal(batch * qd).astype(np.float32)
    kc = rng.standard_normal(cap * kvd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(cap * kvd).astype(np.float16).view(np.uint16)
    qb, kb, vb = (backend.HipBuffer.from_host(dev, a) for a in (q, kc, vc))
    out = backend.HipBuffer.alloc(dev, batch * qd)
    one = backend.HipBuffer.alloc(dev, qd)
    dev.attention_prefill(qb, kb, vb, out, start, batch, nh, nkv, hd, 0.0625, sw, cap)
    dev.sync()
    got = out.numpy().reshape(batch, qd)
    for i in range(0, batch, 7):
        qi = backend.HipBuffer.from_host(dev, q[i * qd:(i + 1) * qd])
        dev.attention_causal_ref(qi, kb, vb, one, start + i, nh, nkv, hd, 0.0625, sw, cap)
        dev.sync()
        assert_bits(got[i], one.numpy(), f"row {i}")
        qi.close()


@pytest.mark.parametrize("pad", [1, 4])
def test_attention_prefill_q_stride(backend, dev, orc, pad):
    """Query rows pad floats apart beyond n_heads*head_dim: a stride that
    16-byte reads cannot follow (pad 1: the rows' scores take the one-row
    workgroup form) and one they can (pad 4: the multi-row form), each row
    bit-exact against the CPU attention."""
    nh, nkv, hd, cap, start, batch = 8, 4, 256, 512, 100, 40
    rng = np.random.default_rng(4700 + pad)
    qd, kvd, stride = nh * hd, nkv * hd, nh * hd + pad
    q = (rng.standard_normal(batch * stride) * 0.5).astype(np.float32)
    kc = rng.standard_normal(cap * kvd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(cap * kvd).astype(np.float16).view(np.uint16)
    qb, kb, vb = (backend.HipBuffer.from_host(dev, a) for a in (q, kc, vc))
    out = backend.HipBuffer.alloc(dev, batch * qd)
    dev.attention_prefill(qb, kb, vb, out, start, batch, nh, nkv, hd, 1.0 / 16.0, None, cap, q_stride=stride)
    dev.sync()
    got = out.numpy().reshape(batch, qd)
    for i in range(batch):
        rows = window_rows(start + i, None, cap)
        ref = orc.attention_f16(q[i * stride:i * stride + qd], kc.reshape(cap, kvd)[rows].reshape(-1),
                                vc.reshape(cap, kvd)[rows].reshape(-1), len(rows) - 1, nh, nkv, hd, 1.0 / 16.0)
        assert_bits(got[i], ref, f"q stride {stride}: row {i}")


def test_attention_prefill_invalid(backend, dev):
    nh, nkv, hd = 8, 4, 256
    qb = backend.HipBuffer.alloc(dev, 4 * nh * hd)
    kb = backend.HipBuffer.alloc(dev, 64 * nkv * hd, np.uint16)
    out = backend.HipBuffer.alloc(dev, 4 * nh * hd)
    with pytest.raises(backend.HipError) as e:
        dev.attention_prefill(qb, kb, kb, out, 0, 4, nh, nkv, hd, 0.0625, None, 64, 3, 0)
    assert e.value.status == -4  # MRML_HIP_E_UNSUPPORTED
    for kw in (dict(q_stride=nh * hd - 1), dict(batch=0), dict(head_dim=100)):
        with pytest.raises(backend.HipError):
            dev.attention_prefill(qb, kb, kb, out, 0, kw.get("batch", 4), nh, nkv, kw.get("head_dim", hd), 0.0625,
                                  None, 64, q_stride=kw.get("q_stride", nh * hd))
