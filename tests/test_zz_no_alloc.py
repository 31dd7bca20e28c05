"""The allocation-free batched product, mrml_hip_gemm_q4_0_noalloc, through
the C ABI: the same outputs as mrml_hip_gemm_q4_0 (which quantises the batch
into the context's workspace), with the activations' GEMM pack in the
library's fixed per-GPU device scratch instead.

Two calls in a row, the second on a smaller batch (the scratch keeps the
first call's contents), a graph capture of it replayed over new activations
(the callers it is for cannot allocate: code under capture), and a pack
larger than the scratch rejected with MRML_HIP_E_INVALID.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_noalloc_gemm_equals_gemm_two_calls(backend, dev, orc, synth):
    for rows, cols, batch in [(2304, 9216, 300), (1024, 2304, 37)]:
        rng = synth.rng_for(7000 + batch)
        w = synth.q4_0_matrix(rng, rows, cols)
        x = rng.standard_normal((batch, cols)).astype(np.float32)
        wb = backend.HipBuffer.from_gguf(dev, w, backend.Q4_0, rows, cols)
        xb = backend.HipBuffer.from_host(dev, x.reshape(-1))
        y_ref = backend.HipBuffer.alloc(dev, rows * batch)
        y = backend.HipBuffer.alloc(dev, rows * batch)
        dev.gemm_q4_0(wb, xb, y_ref, rows, cols, batch)
        dev.gemm_q4_0_noalloc(wb, xb, y, rows, cols, batch)
        dev.sync()
        got, ref = y.numpy(), y_ref.numpy()
        assert np.array_equal(bits(got), bits(ref)), f"noalloc {rows}x{cols} M={batch} differs from gemm_q4_0"
        # and the CPU oracle on the first and last tokens
        for m in (0, batch - 1):
            want = orc.mat_vec_mul_q4_0(w, x[m], rows, cols, threads=16)
            assert np.array_equal(bits(got.reshape(batch, rows)[m]), bits(want)), f"token {m} vs the oracle"


def test_noalloc_gemm_under_graph_capture(backend, dev, synth):
    rows, cols, batch = 2048, 2304, 64
    rng = synth.rng_for(7100)
    w = synth.q4_0_matrix(rng, rows, cols)
    wb = backend.HipBuffer.from_gguf(dev, w, backend.Q4_0, rows, cols)
    xb = backend.HipBuffer.alloc(dev, batch * cols)
    y = backend.HipBuffer.alloc(dev, rows * batch)
    y_ref = backend.HipBuffer.alloc(dev, rows * batch)
    graph = dev.capture(lambda: dev.gemm_q4_0_noalloc(wb, xb, y, rows, cols, batch))
    try:
        for rep in range(3):
            x = (rng.standard_normal((batch, cols)) * (rep + 1)).astype(np.float32)
            xb.copy_from_host(x.reshape(-1))
            graph.launch()
            dev.sync()
            dev.gemm_q4_0(wb, xb, y_ref, rows, cols, batch)   # eager work between the replays
            dev.sync()
            assert np.array_equal(bits(y.numpy()), bits(y_ref.numpy())), f"replay {rep}"
    finally:
        graph.close()


def test_noalloc_gemm_rejects_packs_above_the_scratch(backend, dev):
    cap = dev.gemm_q4_0_noalloc_max_pack_bytes()
    assert cap == 8 << 20
    cols = 9216
    groups = cap // (cols // 32 * 1152)              # 25 token groups of 32 fit
    assert dev.gemm_pack_bytes(cols, 32 * groups) <= cap < dev.gemm_pack_bytes(cols, 32 * groups + 1)
    w = backend.HipBuffer.alloc(dev, 32 * cols // 32 * 18, np.uint8)
    x = backend.HipBuffer.alloc(dev, (32 * groups + 1) * cols)
    y = backend.HipBuffer.alloc(dev, 32 * (32 * groups + 1))
    with pytest.raises(backend.HipError) as e:
        dev.gemm_q4_0_noalloc(w, x, y, 32, cols, 32 * groups + 1)
    assert e.value.status == -1 and "scratch" in str(e.value)
    dev.sync()
