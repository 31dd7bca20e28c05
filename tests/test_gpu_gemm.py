"""GPU parity of the batched (prefill) Q4_0 x Q8_0 product on int8 MFMA.

The reference has no CPU batched path (CPU prefill runs token at a time,
model.rs:2694-2696), so the oracle is the CPU matvec applied per token:
every output y[m][r] must be bit-identical to ops::mat_vec_mul_q4_0 on token
m (ops.rs:162-180 via quant.rs:339-366).  The integer accumulators are pinned
separately: with one block per row and unit scales each output IS the block's
int32 dot, checked against a numpy integer product.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

THREADS = 16


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bit_exact(got, ref, what):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    bad = np.flatnonzero(bits(got) != bits(ref))
    assert bad.size == 0, f"{what}: {bad.size} of {ref.size} differ, first {bad[:5]}: {got.flat[bad[:5]]} vs " \
                          f"{ref.flat[bad[:5]]}"


def run_gemm(backend, dev, w, x, rows, cols, batch, prequantised=False):
    wb = backend.HipBuffer.from_gguf(dev, w, backend.Q4_0, rows, cols)
    xb = backend.HipBuffer.from_host(dev, np.ascontiguousarray(x, np.float32).reshape(-1))
    yb = backend.HipBuffer.alloc(dev, rows * batch)
    if prequantised:
        pk = backend.HipBuffer.alloc(dev, dev.q8_0_pack_bytes(batch * cols), np.uint8)
        dev.quantize_q8_0(xb, None, pk, batch * cols)
        dev.gemm_q4_0_q8(wb, pk, yb, rows, cols, batch)
    else:
        dev.gemm_q4_0(wb, xb, yb, rows, cols, batch)
    dev.sync()
    return yb.numpy().reshape(batch, rows)


def oracle_gemm(orc, w, x, rows, cols, tokens):
    return np.stack([orc.mat_vec_mul_q4_0(w, x[m], rows, cols, threads=THREADS) for m in tokens])


# C5: the Gemma-2-2B gate/up and down shapes at M = 512 prefill tokens.
@pytest.mark.parametrize("rows,cols", [(9216, 2304), (2304, 9216)])
def test_gemm_q4_0_prefill_512_bit_exact(backend, dev, orc, synth, rows, cols):
    batch = 512
    rng = synth.rng_for(5000 + rows)
    w = synth.q4_0_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    got = run_gemm(backend, dev, w, x, rows, cols, batch)
    ref = oracle_gemm(orc, w, x, rows, cols, range(batch))
    assert_bit_exact(got, ref, f"gemm {rows}x{cols} M={batch}")


@pytest.mark.parametrize("rows,cols,batch", [
    (32, 32, 1), (64, 64, 17), (96, 256, 33), (128, 2304, 100), (32, 96, 129), (256, 512, 255),
    (1024, 2304, 16), (64, 16384, 40),
    # K tails of 5, 6 and 7 blocks past the last 8-block chunk (more tail
    # blocks than B prefetch slots), with and without full chunks before them
    (32, 160, 33), (64, 192, 40), (96, 224, 65), (32, 416, 7), (64, 480, 100), (32, 2272, 50),
])
def test_gemm_q4_0_ragged_bit_exact(backend, dev, orc, synth, rows, cols, batch):
    rng = synth.rng_for(5100 + rows + cols + batch)
    w = synth.q4_0_matrix(rng, rows, cols)
    x = (rng.standard_normal((batch, cols)) * 10.0 ** rng.uniform(-3, 3, (batch, 1))).astype(np.float32)
    x[0, :32] = 0.0                                   # a zero block: scale 0, quants 0
    got = run_gemm(backend, dev, w, x, rows, cols, batch)
    ref = oracle_gemm(orc, w, x, rows, cols, range(batch))
    assert_bit_exact(got, ref, f"gemm {rows}x{cols} M={batch}")


def test_gemm_q4_0_integer_accumulators(backend, dev):
    """One block per row, unit scales, activations exactly representable as
    Q8_0 (amax 127 in every token): y[m][r] == sum_i (n_i(r)-8) * x_i(m), the
    int32 block dot, for every nibble and quant pattern incl. -128 and 0/15."""
    rows, cols, batch = 256, 32, 200
    rng = np.random.default_rng(77)
    nib = rng.integers(0, 16, (rows, 32))
    nib[0], nib[1] = 0, 15                             # extreme rows
    q = rng.integers(-127, 128, (batch, 32))
    q[:, 0] = 127                                      # amax 127 -> scale 1.0, q == x exactly
    q[1, 1:] = -127
    w = np.zeros((rows, 18), np.uint8)
    w[:, 1] = 0x3C                                     # f16 1.0
    w[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    got = run_gemm(backend, dev, w.reshape(-1), q.astype(np.float32), rows, cols, batch)
    isum = q.astype(np.int64) @ (nib - 8).T.astype(np.int64)
    assert np.array_equal(got, isum.astype(np.float32)), "integer block dots differ"


def test_gemm_q4_0_matches_gemv_and_pack_entry(backend, dev, orc, synth):
    """The f32 entry, the pre-quantised entry and the batch-1 matvec agree bit
    for bit on every token."""
    rows, cols, batch = 2048, 2304, 48
    rng = synth.rng_for(5200)
    w = synth.q4_0_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    a = run_gemm(backend, dev, w, x, rows, cols, batch)
    b = run_gemm(backend, dev, w, x, rows, cols, batch, prequantised=True)
    assert_bit_exact(a, b, "f32 entry vs pack entry")
    # the GEMM pack, quantised once and used for two products
    wb2 = backend.HipBuffer.from_gguf(dev, w, backend.Q4_0, rows, cols)
    xb = backend.HipBuffer.from_host(dev, x.reshape(-1))
    gp = backend.HipBuffer.alloc(dev, dev.gemm_pack_bytes(cols, batch), np.uint8)
    y1 = backend.HipBuffer.alloc(dev, rows * batch)
    y2 = backend.HipBuffer.alloc(dev, rows * batch)
    dev.quantize_q8_0_gemm(xb, gp, cols, batch)
    dev.gemm_q4_0_gpack(wb2, gp, y1, rows, cols, batch)
    dev.gemm_q4_0_gpack(wb2, gp, y2, rows, cols, batch)
    dev.sync()
    assert_bit_exact(y1.numpy().reshape(batch, rows), a, "gpack entry vs f32 entry")
    assert_bit_exact(y2.numpy().reshape(batch, rows), a, "gpack entry, second use")
    wb = backend.HipBuffer.from_gguf(dev, w, backend.Q4_0, rows, cols)
    yb = backend.HipBuffer.alloc(dev, rows)
    for m in (0, 1, 31, 32, 47):
        xb = backend.HipBuffer.from_host(dev, x[m])
        dev.gemv_q4_0(wb, xb, yb, rows, cols)
        dev.sync()
        assert_bit_exact(a[m], yb.numpy(), f"gemm token {m} vs gemv")


def test_gemm_q4_0_rejects_bad_shapes(backend, dev):
    w = backend.HipBuffer.alloc(dev, 64 * 18, np.uint8)
    x = backend.HipBuffer.alloc(dev, 64 * 4)
    y = backend.HipBuffer.alloc(dev, 64 * 4)
    # the last case: the activations would pass 2 GiB (32-bit buffer offsets)
    for rows, cols, batch in [(0, 32, 2), (32, 48, 2), (32, 32, 0), (32, 2304, 1 << 22)]:
        with pytest.raises(backend.HipError):
            dev.gemm_q4_0(w, x, y, rows, cols, batch)


# Row counts that are not multiples of 32 (the reference's grid is ceil(rows / 8),
# cuda.rs:627-673): the last 32-row tile is partial, and outputs whose row
# stride is not a multiple of 4 are stored one float at a time.
@pytest.mark.parametrize("rows,cols,batch", [(1, 32, 1), (5, 64, 3), (33, 256, 40), (100, 2304, 37), (31, 96, 64),
                                             (2305, 2304, 17), (7, 9216, 33)])
def test_gemm_q4_0_any_rows_bit_exact(backend, dev, orc, synth, rows, cols, batch):
    rng = synth.rng_for(5150 + rows + cols + batch)
    w = synth.q4_0_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    got = run_gemm(backend, dev, w, x, rows, cols, batch)
    ref = oracle_gemm(orc, w, x, rows, cols, range(batch))
    assert_bit_exact(got, ref, f"gemm {rows}x{cols} M={batch}")
    # the pre-quantised entry and the relaxed fold take the same shapes
    assert_bit_exact(run_gemm(backend, dev, w, x, rows, cols, batch, prequantised=True), ref, "pack entry")


@pytest.mark.parametrize("rows,cols,batch", [(2300, 2304, 500), (1100, 512, 1000), (1056, 256, 1024)])
def test_gemm_q4_0_split_tiles_bit_exact(backend, dev, orc, synth, rows, cols, batch):
    """Products whose 32x32 tiles (one per row tile and 32-token group) number
    just over one per SIMD (1024 on MI355X) run their last row tiles as
    32-row x 16-token tiles on the 16x16x32 int8 MFMA: here with a partial
    last row tile and a partial last token group among them (1152 and 1120
    tiles), and at 1056 rows x 32 groups (1056 tiles, every tile whole)."""
    rng = synth.rng_for(5170 + rows + cols + batch)
    w = synth.q4_0_matrix(rng, rows, cols)
    x = (rng.standard_normal((batch, cols)) * 10.0 ** rng.uniform(-3, 3, (batch, 1))).astype(np.float32)
    x[batch - 1, :32] = 0.0  # a zero block in the last (HALF-tiled) token group
    got = run_gemm(backend, dev, w, x, rows, cols, batch)
    ref = oracle_gemm(orc, w, x, rows, cols, range(batch))
    assert_bit_exact(got, ref, f"gemm {rows}x{cols} M={batch}")
    assert_bit_exact(run_gemm(backend, dev, w, x, rows, cols, batch, prequantised=True), ref, "pack entry")


def test_gemm_q4_0_qkv_geglu_any_rows(backend, dev, orc, synth):
    """The fused batched entries at row counts that are not multiples of 32
    or of 4: the k and v products then start off a 16-byte boundary of the
    stacked rows, stored one float at a time."""
    q_rows, kv_rows, cols, batch = 42, 19, 256, 45
    rng = synth.rng_for(5160)
    ws = {k: synth.q4_0_matrix(rng, r, cols) for k, r in (("q", q_rows), ("k", kv_rows), ("v", kv_rows))}
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bufs = [backend.HipBuffer.from_gguf(dev, ws[k], backend.Q4_0, r, cols)
            for k, r in (("q", q_rows), ("k", kv_rows), ("v", kv_rows))]
    xb = backend.HipBuffer.from_host(dev, x.reshape(-1))
    total = q_rows + 2 * kv_rows
    yb = backend.HipBuffer.alloc(dev, batch * total)
    dev.gemm_q4_0_qkv(*bufs, xb, yb, q_rows, kv_rows, cols, batch)
    dev.sync()
    got = yb.numpy().reshape(batch, total)
    for name, lo, r in (("q", 0, q_rows), ("k", q_rows, kv_rows), ("v", q_rows + kv_rows, kv_rows)):
        assert_bit_exact(got[:, lo:lo + r], oracle_gemm(orc, ws[name], x, r, cols, range(batch)), f"qkv {name}")
    rows = 77
    wg, wu = synth.q4_0_matrix(rng, rows, cols), synth.q4_0_matrix(rng, rows, cols)
    bg = backend.HipBuffer.from_gguf(dev, wg, backend.Q4_0, rows, cols)
    bu = backend.HipBuffer.from_gguf(dev, wu, backend.Q4_0, rows, cols)
    ab = backend.HipBuffer.alloc(dev, batch * rows)
    dev.gemm_q4_0_geglu(bg, bu, xb, ab, rows, cols, batch)
    dev.sync()
    g = oracle_gemm(orc, wg, x, rows, cols, range(batch))
    u = oracle_gemm(orc, wu, x, rows, cols, range(batch))
    assert_bit_exact(ab.numpy().reshape(batch, rows), np.stack([orc.geglu(g[m], u[m]) for m in range(batch)]),
                     "geglu")


# ------------------------------------------------------------ fused batched entry points
@pytest.mark.parametrize("batch", [128, 512])
def test_gemm_q4_0_qkv_stacked_rows(backend, dev, orc, synth, batch):
    """CudaDevice::gemm_q4_0_qkv (cuda.rs:2406-2436): y[m] = [Wq x_m | Wk x_m |
    Wv x_m], every output bit-identical to the CPU matvec of its token."""
    q_rows, kv_rows, cols = 2048, 1024, 2304
    rng = synth.rng_for(5300 + batch)
    ws = {k: synth.q4_0_matrix(rng, r, cols) for k, r in (("q", q_rows), ("k", kv_rows), ("v", kv_rows))}
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bufs = [backend.HipBuffer.from_gguf(dev, ws[k], backend.Q4_0, r, cols)
            for k, r in (("q", q_rows), ("k", kv_rows), ("v", kv_rows))]
    xb = backend.HipBuffer.from_host(dev, x.reshape(-1))
    total = q_rows + 2 * kv_rows
    yb = backend.HipBuffer.alloc(dev, batch * total)
    dev.gemm_q4_0_qkv(*bufs, xb, yb, q_rows, kv_rows, cols, batch)
    dev.sync()
    got = yb.numpy().reshape(batch, total)
    for name, lo, r in (("q", 0, q_rows), ("k", q_rows, kv_rows), ("v", q_rows + kv_rows, kv_rows)):
        ref = oracle_gemm(orc, ws[name], x, r, cols, range(batch))
        assert_bit_exact(got[:, lo:lo + r], ref, f"gemm qkv {name} M={batch}")


@pytest.mark.parametrize("batch", [128, 512])
def test_gemm_q4_0_geglu_per_token(backend, dev, orc, synth, batch):
    """CudaDevice::gemm_q4_0_geglu (cuda.rs:2699-2725): act[m] = gelu(Wg x_m) *
    (Wu x_m) with the CPU semantics (model.rs:2093-2105), bit-identical to
    the oracle per token."""
    rows, cols = 9216, 2304
    rng = synth.rng_for(5400 + batch)
    wg, wu = synth.q4_0_matrix(rng, rows, cols), synth.q4_0_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bg = backend.HipBuffer.from_gguf(dev, wg, backend.Q4_0, rows, cols)
    bu = backend.HipBuffer.from_gguf(dev, wu, backend.Q4_0, rows, cols)
    xb = backend.HipBuffer.from_host(dev, x.reshape(-1))
    ab = backend.HipBuffer.alloc(dev, batch * rows)
    dev.gemm_q4_0_geglu(bg, bu, xb, ab, rows, cols, batch)
    dev.sync()
    got = ab.numpy().reshape(batch, rows)
    g = oracle_gemm(orc, wg, x, rows, cols, range(batch))
    u = oracle_gemm(orc, wu, x, rows, cols, range(batch))
    ref = np.stack([orc.geglu(g[m], u[m]) for m in range(batch)])
    assert_bit_exact(got, ref, f"gemm geglu M={batch}")


# The tolerance path's fold (mrml_hip_gemm_q4_0_relaxed): integer block sums
# exact, one FMA per block term; bound 1e-5 of the largest output.
RELAXED_TOL = 1e-5


@pytest.mark.parametrize("rows,cols,batch", [(9216, 2304, 128), (2304, 9216, 512), (2048, 2304, 37)])
def test_gemm_q4_0_relaxed_within_tolerance(backend, dev, synth, rows, cols, batch):
    rng = synth.rng_for(7000 + rows + batch)
    w = synth.q4_0_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    wb = backend.HipBuffer.from_gguf(dev, w, backend.Q4_0, rows, cols)
    xb = backend.HipBuffer.from_host(dev, x.reshape(-1))
    ye = backend.HipBuffer.alloc(dev, rows * batch)
    yr = backend.HipBuffer.alloc(dev, rows * batch)
    dev.gemm_q4_0(wb, xb, ye, rows, cols, batch)
    dev.gemm_q4_0_relaxed(wb, xb, yr, rows, cols, batch)
    dev.sync()
    e, r = ye.numpy(), yr.numpy()
    err = float(np.max(np.abs(r.astype(np.float64) - e))) / float(np.max(np.abs(e)))
    print(f"\n[relaxed gemm] {rows}x{cols} M={batch}: max-rel {err:.2e}", flush=True)
    assert err <= RELAXED_TOL
    assert not np.array_equal(r.view(np.uint32), e.view(np.uint32))  # the fold did change (a live check)
