"""Pins of the CPU oracle (oracle/mrml_oracle.c) -- CPU only.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
a swapped nibble, rounding instead of truncating, an FMA, a wrong fold order)
fails it.  Sources:
  * the reference's own tests: crates/mrml-tensor/tests/quant_test.rs,
    ops_test.rs, src/quant.rs:406-439 (SIMD == scalar);
  * closed forms of examples/cuda_prefill_primitives.rs:23-49;
  * IEEE facts checked against numpy's float16 (round-to-nearest-even);
  * brute force: an independent numpy evaluation of the integer block sums
    (int64 matmul over unpacked nibbles) and of the block-ordered float32 fold.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- helpers
def unpack_q4_0(blocks: np.ndarray, nb: int):
    """GGUF Q4_0 bytes -> (int8 values q-8 [.., nb, 32], f16 scales as f32 [.., nb])."""
    b = blocks.reshape(-1, nb, 18)
    d = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    qs = b[..., 2:]
    vals = np.concatenate([(qs & 15).astype(np.int64) - 8, (qs >> 4).astype(np.int64) - 8], axis=-1)
    return vals, d


def unpack_q8_0(blocks: np.ndarray, nb: int):
    b = blocks.reshape(-1, nb, 34)
    d = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    q = b[..., 2:].view(np.int8).astype(np.int64)
    return q, d


def fold_f32(isums: np.ndarray, dw: np.ndarray, da: np.ndarray) -> np.ndarray:
    """Block-ordered float32 fold: s = s + f32(isum_b) * (dw_b * da_b), every op rounded to f32."""
    s = np.zeros(isums.shape[0], dtype=np.float32)
    for b in range(isums.shape[1]):
        scale = (dw[:, b] * da[b]).astype(np.float32)          # exact: 11-bit x 11-bit significands
        t = (isums[:, b].astype(np.float32) * scale).astype(np.float32)
        s = (s + t).astype(np.float32)
    return s


def roundf(v: np.ndarray) -> np.ndarray:
    """C roundf (half away from zero), evaluated exactly in float64."""
    v = v.astype(np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


# ---------------------------------------------------------------- f16
def test_f16_known_answers(orc):
    # truncation, not rounding (quant.rs:81-104): 100/127 is 0x3A4D under RNE
    assert orc.f32_to_f16(np.float32(1) / np.float32(127)) == 0x2008
    assert orc.f32_to_f16(np.float32(100) / np.float32(127)) == 0x3A4C
    assert orc.f32_to_f16(np.float32(2.5) / np.float32(127)) == 0x250A
    assert int(np.float16(np.float32(100) / np.float32(127)).view(np.uint16)) == 0x3A4D
    assert orc.f32_to_f16(1.0) == 0x3C00
    assert orc.f32_to_f16(1e-6) == 0x0000           # f16-subnormal range -> +0
    assert orc.f32_to_f16(-1e-6) == 0x0000          # sign dropped too
    assert orc.f32_to_f16(float("inf")) == 0x7C00
    assert orc.f32_to_f16(float("-inf")) == 0xFC00
    assert orc.f32_to_f16(1e6) == 0x7C00            # overflow -> Inf
    assert orc.f32_to_f16(float("nan")) == 0x7E00
    assert orc.f32_to_f16(-float("nan")) == 0xFE00


def test_f16_to_f32_exhaustive(orc):
    """All 65536 halves: exact conversion equals numpy's (IEEE) widening."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(x)) for x in h], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    # NaN payload rule of quant.rs:70: mant << 13
    assert np.float32(orc.f16_to_f32(0x7E01)).view(np.uint32) == (0xFF << 23) | (0x201 << 13)


def test_f32_to_f16_truncation_vs_numpy(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4000) * 10.0 ** rng.uniform(-4, 4, 4000)).astype(np.float32)
    bits = x.view(np.uint32)
    for xi, bi in zip(x, bits):
        got = orc.f32_to_f16(float(xi))
        rne = int(np.float16(xi).view(np.uint16))
        h_abs = np.float16(xi)
        if abs(xi) < 6.103515625e-05 or not np.isfinite(h_abs):
            continue
        if bi & 0x1FFF == 0:                      # exactly representable: both agree
            assert got == rne
        else:                                     # truncation never rounds up in magnitude
            assert abs(np.uint16(got).view(np.float16)) <= abs(xi) <= abs(np.uint16(got + 1).view(np.float16))


def test_f32_to_f16_rne_vs_numpy(orc):
    rng = np.random.default_rng(2)
    x = np.concatenate([
        (rng.standard_normal(3000) * 10.0 ** rng.uniform(-9, 5, 3000)).astype(np.float32),
        np.array([65504, 65519.99, 65520, 7e4, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26,
                  -0.0, 0.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32)])
    got = np.array([orc.f32_to_f16_rne(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- Q8_0 quantiser
def test_q8_0_roundtrip_quant_test(orc):
    # quant_test.rs:3-22
    x = ((np.arange(64, dtype=np.float32) - 32.0) * np.float32(0.1)).astype(np.float32)
    back = orc.dequantize_q8_0(orc.quantize_q8_0(x), 64)
    assert np.max(np.abs(back - x)) < 0.05


def test_q8_0_all_ones_closed_form(orc):
    q = orc.quantize_q8_0(np.ones(32, dtype=np.float32))
    assert (int(q[0]) | (int(q[1]) << 8)) == 0x2008            # f16 trunc of 1/127
    assert np.all(q[2:].view(np.int8) == 127)


def test_q8_0_rounding_ties_away_from_zero(orc):
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0                                   # amax 127 -> scale 1, id 1
    x[1:7] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5]
    q = orc.quantize_q8_0(x)[2:].view(np.int8)
    assert list(q[:7]) == [127, 3, -3, 1, -1, 2, -2]


def test_q8_0_zero_and_nan_blocks(orc):
    q = orc.quantize_q8_0(np.zeros(32, dtype=np.float32))
    assert q[0] == 0 and q[1] == 0 and np.all(q[2:] == 0)
    x = np.ones(32, dtype=np.float32)
    x[3] = np.nan                                  # NaN never becomes amax; its quant is 0
    q = orc.quantize_q8_0(x)
    assert (int(q[0]) | (int(q[1]) << 8)) == 0x2008
    assert q[2 + 3] == 0 and np.all(np.delete(q[2:].view(np.int8), 3) == 127)


def test_q8_0_quantiser_brute_force(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 200) * 10.0 ** rng.uniform(-3, 3, 32 * 200)).astype(np.float32)
    got = orc.quantize_q8_0(x).reshape(-1, 34)
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    d_trunc = (scale.view(np.uint32) >> 13) - ((127 - 15) << 10)          # valid in this range
    inv = np.where(scale != 0, (np.float32(1.0) / scale).astype(np.float32), np.float32(0))
    prod = (xb * inv[:, None]).astype(np.float32)
    q = np.clip(roundf(prod), -128, 127).astype(np.int8)
    assert np.array_equal(got[:, 2:].view(np.int8), q)
    assert np.array_equal(got[:, 0].astype(np.uint32) | (got[:, 1].astype(np.uint32) << 8),
                          d_trunc.astype(np.uint32))


# ---------------------------------------------------------------- Q4_0 quantiser
# quant.rs:372-389: amax folds from 0.0 with f32::max (a NaN never wins),
# scale = amax / 8, d = the truncating f16 of scale, inverse = 1 / scale
# (0 when scale is 0), q = clamp(round(x * inverse) as i32, -8, 7) + 8 with
# round half away from zero and a saturating cast (NaN -> 0), value j in the
# low nibble of byte j and value j + 16 in its high nibble.
def q4_bytes(q: np.ndarray, d_bits: int) -> np.ndarray:
    """18-byte block from 32 unsigned nibbles (0..15) and the d bits."""
    out = np.zeros(18, np.uint8)
    out[0], out[1] = d_bits & 0xFF, d_bits >> 8
    out[2:] = (q[:16] | (q[16:] << 4)).astype(np.uint8)
    return out


def test_q4_0_quantiser_closed_forms(orc):
    # amax 8: scale 1, d 0x3C00, inverse 1 -- q = round(x) clamped, ties away from zero
    x = np.zeros(32, np.float32)
    x[:10] = [8, -8, 4, -4, 0.5, -0.5, 2.5, -2.5, 1.4999999, 7.5]
    x[16:22] = [-7.5, 3.5, -3.5, 6.49, -1.5, 1.5]
    want = np.full(32, 8, np.int64)
    want[:10] = np.array([7, -8, 4, -4, 1, -1, 3, -3, 1, 7]) + 8      # 8 -> 7 (clamp), 7.5 -> 8 -> 7
    want[16:22] = np.array([-8, 4, -4, 6, -2, 2]) + 8
    assert np.array_equal(orc.quantize_q4_0(x), q4_bytes(want, 0x3C00))
    # a zero block: scale 0, d 0, every nibble 8
    assert np.array_equal(orc.quantize_q4_0(np.zeros(32, np.float32)), q4_bytes(np.full(32, 8), 0))
    # NaN is never the amax (f32::max); its own quant is `NaN as i32` = 0 -> 8
    x = np.zeros(32, np.float32)
    x[:3] = [np.nan, 4.0, -2.0]
    x[20] = np.nan
    want = np.full(32, 8, np.int64)
    want[1], want[2] = 8 + 8 - 1, 8 - 4                                # 4 / 0.5 = 8 -> 7; -2 / 0.5 = -4
    assert np.array_equal(orc.quantize_q4_0(x), q4_bytes(want, 0x3800))  # d = f16(0.5)
    # the scale's f16 truncates: amax 0.3 -> scale 0.0375 -> 0x28CC (RNE gives 0x28CD)
    x = np.zeros(32, np.float32)
    x[0] = np.float32(0.3)
    got = orc.quantize_q4_0(x)
    assert (int(got[0]) | (int(got[1]) << 8)) == 0x28CC
    assert int(np.float16(np.float32(0.3) / np.float32(8.0)).view(np.uint16)) == 0x28CD
    assert got[2] & 15 == 15                                            # 0.3 * (1/0.0375) = 8 -> 7 -> 15


def test_q4_0_quantiser_saturating_cast(orc):
    """A subnormal amax: amax / 8 is the smallest subnormal, 1 / scale
    overflows to +inf, x * inf = +-inf saturates to i32::MAX / MIN (-> 7 /
    -8) and 0 * inf = NaN casts to 0; the scale's f16 is +0."""
    tiny = np.float32(2.0 ** -146)
    x = np.zeros(32, np.float32)
    x[0], x[1], x[17] = tiny, -tiny, tiny
    want = np.full(32, 8, np.int64)
    want[0], want[1], want[17] = 15, 0, 15
    assert np.array_equal(orc.quantize_q4_0(x), q4_bytes(want, 0x0000))
    # an amax too small for amax / 8 (scale rounds to 0): inverse 0, all 8
    x = np.zeros(32, np.float32)
    x[5] = np.float32(2.0 ** -149)
    assert np.array_equal(orc.quantize_q4_0(x), q4_bytes(np.full(32, 8), 0))


def test_q4_0_quantiser_brute_force(orc):
    """Random blocks over a wide range, NaN included, against a vectorised
    numpy restatement; a swapped nibble pair, /7 instead of /8, RNE f16 or
    banker's rounding each fail it."""
    rng = np.random.default_rng(33)
    n = 32 * 400
    x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 3, n)).astype(np.float32)
    x[rng.integers(0, n, 40)] = np.nan
    got = orc.quantize_q4_0(x).reshape(-1, 18)
    xb = x.reshape(-1, 32)
    amax = np.fmax.reduce(np.abs(xb), axis=1, initial=0.0).astype(np.float32)
    scale = np.where(amax > 0, (amax / np.float32(8.0)).astype(np.float32), np.float32(0))
    with np.errstate(divide="ignore"):
        inv = np.where(scale > 0, (np.float32(1.0) / scale).astype(np.float32), np.float32(0))
    with np.errstate(invalid="ignore"):
        r = roundf((xb * inv[:, None]).astype(np.float32))
    q = np.where(np.isnan(r), 0, np.clip(np.nan_to_num(r, nan=0.0), -8, 7)).astype(np.int64) + 8
    want_qs = (q[:, :16] | (q[:, 16:] << 4)).astype(np.uint8)
    assert np.array_equal(got[:, 2:], want_qs)
    d_trunc = np.where(scale > 0, (scale.view(np.uint32) >> 13) - ((127 - 15) << 10), 0)  # normal f16 range here
    assert np.array_equal(got[:, 0].astype(np.uint32) | (got[:, 1].astype(np.uint32) << 8), d_trunc.astype(np.uint32))
    # dequantised round trip: within about one scale step (the top value
    # clamps from 8 to 7 steps; the truncated d is within 2^-10 of scale)
    ok = ~np.isnan(xb).any(axis=1)
    back = orc.dequantize_q4_0(orc.quantize_q4_0(xb[ok].reshape(-1)), int(ok.sum()) * 32).reshape(-1, 32)
    assert np.all(np.abs(back - xb[ok]) <= 1.01 * scale[ok][:, None])


# ---------------------------------------------------------------- Q4_0 x Q8_0
def q4_block(d_bits: int, byte: int) -> np.ndarray:
    b = np.full(18, byte, dtype=np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    return b


def test_q4_0_dequantize_0x88_is_zero(orc):
    # quant_test.rs:24-40
    assert np.all(orc.dequantize_q4_0(q4_block(0x3C00, 0x88), 32) == 0.0)


def test_q4_0_dot_0x99_closed_form(orc):
    # quant_test.rs:42-57 asserts ~32; the exact value is 4064 * (1 * f16(0x2008)) = 4064*129/16384
    a = orc.quantize_q8_0(np.ones(32, dtype=np.float32))
    for isa in (0, 1, 2, -1):
        got = orc.vec_dot_q4_0_q8_0(q4_block(0x3C00, 0x99), a, 32, isa)
        if math.isnan(got):
            continue                                # ISA absent on this host
        assert got == 31.998046875


def test_q4_0_nibble_pairing_closed_forms(orc):
    """examples/cuda_prefill_primitives.rs:23-49: 0x98 -> +x[16..32], 0x87 -> -x[0..16]."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal(32).astype(np.float32)
    a = orc.quantize_q8_0(x)
    qa = a[2:].view(np.int8).astype(np.int64)
    da = np.uint16(int(a[0]) | (int(a[1]) << 8)).view(np.float16).astype(np.float32)
    upper = orc.vec_dot_q4_0_q8_0(q4_block(0x3C00, 0x98), a, 32)
    lower = orc.vec_dot_q4_0_q8_0(q4_block(0x3C00, 0x87), a, 32)
    assert upper == np.float32(np.float32(qa[16:].sum()) * da)
    assert lower == np.float32(np.float32(-qa[:16].sum()) * da)


def test_q4_0_isa_variants_bit_equal(orc):
    # quant.rs:406-432 (formula inputs of the reference test) and random rows
    values = ((np.arange(256) * 37 % 101).astype(np.float32) - 50.0) / np.float32(13.0)
    other = ((np.arange(256) * 19 % 89).astype(np.float32) - 44.0) / np.float32(11.0)
    q4 = orc.quantize_q4_0(values)
    q8 = orc.quantize_q8_0(other)
    ref = orc.vec_dot_q4_0_q8_0(q4, q8, 256, 0)
    for isa in (1, 2):
        got = orc.vec_dot_q4_0_q8_0(q4, q8, 256, isa)
        assert math.isnan(got) or got == ref


def test_q4_0_matvec_brute_force_fold(orc, synth):
    """Independent numpy: int64 block sums + float32 fold in block order == oracle, bit for bit."""
    rng = synth.rng_for(99)
    rows, cols = 97, 2304
    nb = cols // 32
    w = synth.q4_0_matrix(rng, rows, cols)
    x = synth.normal_vector(rng, cols)
    a = orc.quantize_q8_0(x)
    y = orc.mat_vec_mul_q4_0_q8_0(w, a, rows, cols)
    vals, dw = unpack_q4_0(w, nb)
    qa, da = unpack_q8_0(a, nb)
    isums = np.einsum("rbi,bi->rb", vals, qa[0])
    for r in (0, 5, 96):
        assert np.array_equal(orc.block_isums_q4_0_q8_0(w[r * nb * 18:(r + 1) * nb * 18], a, cols), isums[r])
    ref = fold_f32(isums, dw[:, :] if dw.ndim == 2 else dw, da[0])
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    # and the float64 dequantised dot agrees to rounding error
    deq = (vals * dw[..., None]).reshape(rows, cols).astype(np.float64)
    xq = (qa[0] * da[0][:, None]).reshape(cols).astype(np.float64)
    exact = deq @ xq
    assert np.max(np.abs(y - exact)) <= 1e-5 * np.max(np.abs(exact))


def test_q4_0_fold_has_no_fma(orc):
    """A fused multiply-add would change the low bits of some rows; the float32
    two-rounding fold is what the oracle computes (checked above); here a case
    where fma and mul+add differ is built explicitly."""
    # t = isum * scale with isum*scale not representable; s + t rounding differs with fma
    w = np.concatenate([q4_block(0x3C00, 0x99), q4_block(0x2E66, 0x9A)])  # d=1.0, d~0.1
    x = np.concatenate([np.ones(32, np.float32), np.linspace(-1, 1, 32, dtype=np.float32)])
    a = orc.quantize_q8_0(x)
    got = orc.vec_dot_q4_0_q8_0(w, a, 64)
    vals, dw = unpack_q4_0(w, 2)
    qa, da = unpack_q8_0(a, 2)
    isums = np.einsum("rbi,bi->rb", vals, qa[0])
    assert np.float32(got) == fold_f32(isums, dw, da[0])[0]


def test_matvec_entry_points_bit_equal(orc):
    # ops_test.rs:116-140: mat_vec_mul_q4_0 == mat_vec_mul_q4_0_q8_0 bit for bit
    rows, cols = 73, 64
    w = np.zeros(rows * (cols // 32) * 18, dtype=np.uint8).reshape(-1, 18)
    d = orc.f32_to_f16(0.125)
    for bi in range(w.shape[0]):
        w[bi, 0], w[bi, 1] = d & 0xFF, d >> 8
        w[bi, 2:] = [(bi * 17 + i * 29) & 0xFF for i in range(16)]
    w = w.reshape(-1)
    x = np.sin(np.arange(cols, dtype=np.float32) * np.float32(0.31)).astype(np.float32)
    expected = orc.mat_vec_mul_q4_0(w, x, rows, cols)
    actual = orc.mat_vec_mul_q4_0_q8_0(w, orc.quantize_q8_0(x), rows, cols)
    assert np.array_equal(expected.view(np.uint32), actual.view(np.uint32))
    # row-parallel split (parallel.rs:73-116) does not change any bit
    assert np.array_equal(orc.mat_vec_mul_q4_0_q8_0(w, orc.quantize_q8_0(x), rows, cols, threads=8), actual)


# ---------------------------------------------------------------- Q8_0 x Q8_0
def test_q8_0_dot_matches_dequantized_quant_test(orc):
    # quant_test.rs:59-76
    i = np.arange(96, dtype=np.float32)
    x = (np.sin(i * np.float32(0.13)) * 3).astype(np.float32)
    y = (np.cos(i * np.float32(0.07)) * 2).astype(np.float32)
    qx, qy = orc.quantize_q8_0(x), orc.quantize_q8_0(y)
    expected = float(np.sum(orc.dequantize_q8_0(qx, 96) * orc.dequantize_q8_0(qy, 96), dtype=np.float32))
    for isa in (0, 1, 2):
        got = orc.vec_dot_q8_0_q8_0(qx, qy, 96, isa)
        assert math.isnan(got) or abs(got - expected) < 1e-3


def test_q8_0_scalar_vnni_bit_equal_and_brute_force(orc, synth):
    rng = synth.rng_for(98)
    rows, cols = 33, 2048
    nb = cols // 32
    w = synth.q8_0_matrix(rng, rows, cols)
    a = orc.quantize_q8_0(synth.normal_vector(rng, cols))
    y0 = orc.mat_vec_mul_q8_0_q8_0(w, a, rows, cols, isa=0)
    y2 = orc.mat_vec_mul_q8_0_q8_0(w, a, rows, cols, isa=2)
    if not np.isnan(y2).any():
        assert np.array_equal(y0.view(np.uint32), y2.view(np.uint32))
    qw, dw = unpack_q8_0(w, nb)
    qa, da = unpack_q8_0(a, nb)
    isums = np.einsum("rbi,bi->rb", qw, qa[0])
    assert np.array_equal(y0.view(np.uint32), fold_f32(isums, dw, da[0]).view(np.uint32))
    # the AVX2-only order (quant.rs:534-561) differs only in rounding
    y1 = orc.mat_vec_mul_q8_0_q8_0(w, a, rows, cols, isa=1)
    if not np.isnan(y1).any():
        assert np.max(np.abs(y1 - y0)) <= 1e-5 * np.max(np.abs(y0))


def test_q8_0_softcap(orc):
    # model.rs:2853: 30*tanh(y/30) after the dot (shape of ops_test.rs:188-237)
    rows, cols = 73, 64
    w = np.zeros((rows * 2, 34), dtype=np.uint8)
    d = orc.f32_to_f16(0.02)
    for bi in range(rows * 2):
        w[bi, 0], w[bi, 1] = d & 0xFF, d >> 8
        w[bi, 2:] = [(bi * 17 + i * 11) & 0xFF for i in range(32)]
    w = w.reshape(-1)
    x = np.sin(np.arange(cols, dtype=np.float32) * np.float32(0.031)).astype(np.float32)
    a = orc.quantize_q8_0(x)
    raw = orc.mat_vec_mul_q8_0_q8_0(w, a, rows, cols)
    capped = orc.mat_vec_mul_q8_0_q8_0(w, a, rows, cols, softcap=True)
    ref = (np.float32(30.0) * np.tanh(raw / np.float32(30.0))).astype(np.float32)
    assert np.max(np.abs(capped - ref)) <= 2e-6 * 30
    # the float64 f32-activation reference of the CUDA test is within the Q8_0 quantisation error
    wf = orc.dequantize_q8_0(w, rows * cols).reshape(rows, cols).astype(np.float64)
    f32ref = 30 * np.tanh((wf @ x.astype(np.float64)) / 30)
    assert np.max(np.abs(capped - f32ref)) < 0.1


# ---------------------------------------------------------------- ops
def test_rms_norm_constant(orc):
    # ops_test.rs:79-88
    out = orc.rms_norm(np.full(4, 2.0, dtype=np.float32), None, 1e-6)
    assert np.all(np.abs(out - 1.0) < 1e-4)


def test_swiglu_known_value(orc):
    # ops_test.rs:90-100: silu(2)*3
    assert abs(orc.silu(2.0) * 3.0 - 5.28478) < 1e-3
    assert orc.silu(0.0) == 0.0


def test_swiglu_reference_case(orc):
    """ops_test.rs:14-24: swiglu([0, 2, -2], [1, 3, 4]); out[0] exactly 0."""
    out = orc.swiglu(np.array([0.0, 2.0, -2.0], np.float32), np.array([1.0, 3.0, 4.0], np.float32))
    assert out[0] == 0.0
    assert abs(out[1] - 5.28478) < 1e-3


def test_swiglu_argument_roles(orc):
    """ops.rs:123-130: out = silu(gate) * up, not silu(up) * gate: against
    float64 silu on gate times up.  Bound: a few f32 roundings (expf within
    1 ulp, the add, the divide and the product), 4e-7 relative."""
    rng = np.random.default_rng(71)
    g = (rng.standard_normal(4096) * 4.0).astype(np.float32)
    u = (rng.standard_normal(4096) * 0.1 + 0.3).astype(np.float32)
    got = orc.swiglu(g, u).astype(np.float64)
    g64 = g.astype(np.float64)
    ref = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    assert np.all(np.abs(got - ref) <= 4e-7 * np.abs(ref) + 1e-30)
    # the elementwise form is silu() of each element
    assert all(np.float32(got[i]) == np.float32(np.float32(orc.silu(float(g[i]))) * u[i]) for i in range(0, 4096, 97))
    swapped = orc.swiglu(u, g).astype(np.float64)
    assert np.max(np.abs(swapped - ref)) > 1e-2


def test_rope_batched_equals_per_head(orc):
    # ops_test.rs:142-158, bit equality
    n_heads, hd = 8, 64
    v = np.cos(np.arange(n_heads * hd, dtype=np.float32) * np.float32(0.071)).astype(np.float32)
    per = np.concatenate([orc.rope_1d(v[h * hd:(h + 1) * hd], 137, hd) for h in range(n_heads)])
    bat = orc.rope_1d_batched(v, 137, n_heads, hd)
    assert np.array_equal(per.view(np.uint32), bat.view(np.uint32))


def test_rope_closed_forms(orc):
    v = np.random.default_rng(5).standard_normal(256).astype(np.float32)
    assert np.array_equal(orc.rope_1d(v, 0, 256), v)          # pos 0: identity
    r = orc.rope_1d(v, 17, 256)                                  # rotations preserve pair norms
    pn = lambda a: np.hypot(a[:128].astype(np.float64), a[128:].astype(np.float64))
    assert np.allclose(pn(r), pn(v), rtol=1e-6)
    theta0 = 17.0                                                # i = 0: theta = pos
    assert abs(r[0] - (v[0] * math.cos(theta0) - v[128] * math.sin(theta0))) < 1e-5


@pytest.mark.parametrize("pos", [1, 17, 511, 767])
def test_rope_frequency_schedule(orc, pos):
    """ops.rs:185-208: pair i of a head rotates by theta_i = pos * base^(-2i/d)
    (NeoX halves: element i pairs with i + d/2).  Checked at every i against
    float64 angles; the f32 angle is off by a few ulps of theta, so the bound
    grows with theta.  A wrong exponent (i/d, 2i/(d-2)), a swapped sine, or
    interleaved pairs fail it."""
    hd, nh, base = 256, 3, 10000.0
    rng = np.random.default_rng(40 + pos)
    v = rng.standard_normal(nh * hd).astype(np.float32)
    got = orc.rope_1d_batched(v, pos, nh, hd, base).reshape(nh, hd).astype(np.float64)
    half = hd // 2
    i = np.arange(half, dtype=np.float64)
    theta = pos * base ** (-2.0 * i / hd)
    c, s_ = np.cos(theta), np.sin(theta)
    x = v.reshape(nh, hd).astype(np.float64)
    ref0 = x[:, :half] * c - x[:, half:] * s_
    ref1 = x[:, :half] * s_ + x[:, half:] * c
    tol = (np.abs(x[:, :half]) + np.abs(x[:, half:])) * (4e-7 * (1.0 + theta)) + 1e-7
    assert np.all(np.abs(got[:, :half] - ref0) <= tol)
    assert np.all(np.abs(got[:, half:] - ref1) <= tol)
    # the single-head form follows the same schedule
    one = orc.rope_1d(v[:hd], pos, hd, base).astype(np.float64)
    assert np.all(np.abs(one[:half] - ref0[0]) <= tol[0]) and np.all(np.abs(one[half:] - ref1[0]) <= tol[0])


@pytest.mark.parametrize("dim", [4, 256, 2304])
def test_rms_norm_weighted(orc, dim):
    """ops.rs:24-49 with a weight: sum of squares accumulated in f32 in
    order, scale = 1/sqrtf(sum/dim + eps), out = (x * scale) * w.  Bit-exact
    against a numpy float32 loop (each op an IEEE single op), and within 2e-6
    of the float64 x / rms(x) * w, so a dropped or misplaced w, eps outside
    the root or a sum in another order fail it."""
    rng = np.random.default_rng(50 + dim)
    x = (rng.standard_normal(dim) * 3.0).astype(np.float32)
    w = (1.0 + 0.5 * rng.standard_normal(dim)).astype(np.float32)
    eps = np.float32(1e-6)
    got = orc.rms_norm(x, w, 1e-6)
    s = np.float32(0.0)
    for xi in x:
        s = np.float32(s + np.float32(xi * xi))
    scale = np.float32(np.float32(1.0) / np.sqrt(np.float32(np.float32(s / np.float32(dim)) + eps)))
    ref = ((x * scale).astype(np.float32) * w).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    x64 = x.astype(np.float64)
    ref64 = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w.astype(np.float64)
    assert np.max(np.abs(got - ref64)) <= 2e-6 * np.max(np.abs(ref64))
    # the unweighted form is the weighted one with w = 1
    assert np.array_equal(orc.rms_norm(x, None, 1e-6), orc.rms_norm(x, np.ones(dim, np.float32), 1e-6))


def test_q4_0_dequantize_nibble_order(orc):
    """quant.rs:135-163 on random blocks: the low nibble of byte j is weight
    j, the high nibble weight j + 16, each (q - 8) * d with d the block's f16
    scale (numpy's float16 widening).  An interleaved order (the reference's
    own Q4_K dequantiser interleaves) or a missing offset fails it."""
    rng = np.random.default_rng(60)
    nb = 64
    blocks = rng.integers(0, 256, (nb, 18), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(nb)) * 0.05).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    got = orc.dequantize_q4_0(blocks.reshape(-1), nb * 32).reshape(nb, 32)
    qs = blocks[:, 2:].astype(np.int64)
    q = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1).astype(np.float32)
    ref = (q * d.astype(np.float32)[:, None]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_geglu_argument_roles(orc):
    """ops.rs:107-114: out = gelu_tanh(gate) * up, not gelu(up) * gate:
    against float64 gelu on gate times up, on gate and up drawn from
    different ranges.  Bound: 1e-6 relative (f32 rounding, glibc tanhf's
    ulp) plus the cancellation of 1 + tanh(.) in f32 for large negative gate,
    a few ulps of 1 times 0.5 |gate up|."""
    rng = np.random.default_rng(70)
    g = (rng.standard_normal(4096) * 2.0).astype(np.float32)
    u = (rng.standard_normal(4096) * 0.1 + 0.3).astype(np.float32)
    got = orc.geglu(g, u).astype(np.float64)
    g64 = g.astype(np.float64)
    gelu = 0.5 * g64 * (1.0 + np.tanh(0.7978845608 * (g64 + 0.044715 * g64 ** 3)))
    ref = gelu * u.astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-6 * np.abs(ref) + 2e-7 * np.abs(g64 * u))
    swapped = orc.geglu(u, g).astype(np.float64)
    assert np.max(np.abs(swapped - ref)) > 1e-2


def test_softmax_closed_forms(orc):
    assert np.allclose(orc.softmax(np.full(7, 3.0, dtype=np.float32)), 1 / 7, rtol=1e-6)
    s = orc.softmax(np.array([0.0, np.log(3.0)], dtype=np.float32))
    assert np.allclose(s, [0.25, 0.75], rtol=1e-6)
    assert orc.softmax(np.array([], dtype=np.float32)).size == 0


def test_gelu_closed_forms(orc):
    assert orc.gelu_approx(0.0) == 0.0
    for x in (-3.0, -1.0, 0.5, 2.0):
        k = 0.7978845608
        ref = 0.5 * x * (1 + math.tanh(k * (x + 0.044715 * x ** 3)))
        assert abs(orc.gelu_approx(x) - ref) <= 1e-6 * max(1.0, abs(ref))


def test_argmax_ties_and_nan(orc):
    assert orc.argmax_f32(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert orc.argmax_f32(np.array([np.nan, 1.0, np.nan, 5.0, 5.0], np.float32)) == 3
    assert orc.argmax_f32(np.array([np.nan, np.nan], np.float32)) == 0
    assert orc.argmax_f32(np.array([-0.0, 0.0], np.float32)) == 0


def test_attention_f16_against_float64(orc):
    rng = np.random.default_rng(6)
    n_heads, n_kv, hd, n_past = 8, 4, 64, 9
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    kf = rng.standard_normal((n_past + 1, n_kv, hd)).astype(np.float32)
    vf = rng.standard_normal((n_past + 1, n_kv, hd)).astype(np.float32)
    kc = kf.astype(np.float16).view(np.uint16)
    vc = vf.astype(np.float16).view(np.uint16)
    out = orc.attention_f16(q, kc, vc, n_past, n_heads, n_kv, hd, 0.125)
    k64 = kc.view(np.float16).astype(np.float64)
    v64 = vc.view(np.float16).astype(np.float64)
    for h in range(n_heads):
        g = h // (n_heads // n_kv)
        sc = k64[:, g, :] @ q[h * hd:(h + 1) * hd].astype(np.float64) * 0.125
        p = np.exp(sc - sc.max())
        p /= p.sum()
        ref = p @ v64[:, g, :]
        assert np.allclose(out[h * hd:(h + 1) * hd], ref, rtol=1e-5, atol=1e-6)
    # identical keys -> uniform weights -> mean of values
    kc2 = np.repeat(kc[:1], n_past + 1, axis=0)
    out2 = orc.attention_f16(q, kc2, vc, n_past, n_heads, n_kv, hd, 0.125)
    assert np.allclose(out2[:hd], v64[:, 0, :].mean(axis=0), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- Q4_K (build-defined)
# ---------------------------------------------------------------- quantised KV caches
def test_kv_row_bytes_reference_sizes(orc):
    # kv_cache.rs:164-169 (cuda_layout_sizes_match_block_formats): f16 rows, Q8_0 and Q4_0 blocks
    assert orc.kv_row_bytes(2048, 0) == 4096
    assert orc.kv_row_bytes(2048, 1) == 2176
    assert orc.kv_row_bytes(2048, 2) == 1152


def test_kv_quantised_rows_reference_case(orc):
    """kv_cache.rs:133-161 (quantized_rows_preserve_attention_operations):
    the second head (offset 64) of a 128-value row, dot within 0.03 (Q8) and
    1.0 (Q4) of the exact f32 dot, and add_head_scaled(0.37) within the same."""
    values = ((np.arange(128) * 29 % 97).astype(np.float32) - 48.0) / np.float32(23.0)
    query = ((np.arange(64) * 11 % 53).astype(np.float32) - 26.0) / np.float32(17.0)
    exact = np.float32(np.dot(values[64:].astype(np.float64), query.astype(np.float64)))
    for fmt, tol in ((1, 0.03), (2, 1.0)):
        row = orc.kv_store(values, fmt)
        head = row[orc.kv_row_bytes(64, fmt):]
        assert abs(orc.kv_dot_head(head, query, fmt) - exact) < tol
        out = orc.kv_add_head_scaled(head, np.zeros(64, np.float32), 0.37, fmt)
        assert np.max(np.abs(out - values[64:] * np.float32(0.37))) < tol


def test_kv_store_formats(orc):
    rng = np.random.default_rng(70)
    x = (rng.standard_normal(256) * 3).astype(np.float32)
    assert np.array_equal(orc.kv_store(x, 0).view(np.uint16), x.astype(np.float16).view(np.uint16))  # RNE
    assert np.array_equal(orc.kv_store(x, 1), orc.quantize_q8_0(x))
    assert np.array_equal(orc.kv_store(x, 2), orc.quantize_q4_0(x))


def numpy_kv_head(row: np.ndarray, fmt: int, hd: int):
    """(int64 quants [hd], f32 block scales [hd/32]) of one cached head."""
    if fmt == 1:
        q, d = unpack_q8_0(row, hd // 32)
    else:
        q, d = unpack_q4_0(row, hd // 32)
    return q.reshape(-1), d.reshape(-1)


@pytest.mark.parametrize("fmt", [1, 2])
def test_kv_dot_and_add_brute_force(orc, fmt):
    """dot_head and add_head_scaled of Q8_0 / Q4_0 heads against numpy: int64
    block sums of the quants with quantize_q8_0(q), the float32 block fold
    s = s + isum * (d_k * d_q); out += (d * p) * q per value.  A swapped
    nibble half, a missing -8, p * (d * q) instead of (d * p) * q, or an FMA
    each fail it (p carries full mantissa bits)."""
    rng = np.random.default_rng(71 + fmt)
    for hd in (32, 64, 256, 512):
        nb = hd // 32
        for trial in range(20):
            x = (rng.standard_normal(hd) * 10.0 ** rng.uniform(-2, 2)).astype(np.float32)
            q = rng.standard_normal(hd).astype(np.float32)
            row = orc.kv_store(x, fmt)
            kq, kd = numpy_kv_head(row, fmt, hd)
            q8 = orc.quantize_q8_0(q)
            aq, ad = unpack_q8_0(q8, nb)
            isum = (kq.reshape(nb, 32) * aq.reshape(nb, 32)).sum(axis=1)
            s = np.float32(0.0)
            for b in range(nb):
                s = np.float32(s + np.float32(np.float32(isum[b]) * np.float32(kd[b] * ad.reshape(-1)[b])))
            assert np.float32(orc.kv_dot_head(row, q, fmt)) == s
            p = np.float32(rng.uniform(0.01, 1.0))
            base = rng.standard_normal(hd).astype(np.float32)
            got = orc.kv_add_head_scaled(row, base.copy(), float(p), fmt)
            dd = np.repeat((kd * p).astype(np.float32), 32)
            want = (base + (dd * kq.astype(np.float32)).astype(np.float32)).astype(np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (hd, trial)


def test_attention_kv_f16_is_attention_f16(orc):
    rng = np.random.default_rng(72)
    nh, nkv, hd, n_past = 8, 2, 128, 17
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((n_past + 1) * nkv * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((n_past + 1) * nkv * hd).astype(np.float16).view(np.uint16)
    a = orc.attention_f16(q, kc, vc, n_past, nh, nkv, hd, 0.0884)
    b = orc.attention_kv(q, kc, vc, n_past, nh, nkv, hd, 0.0884, 0, 0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("kf,vf", [(1, 1), (2, 2), (1, 0), (0, 2)])
def test_attention_kv_against_float64(orc, kf, vf):
    """Quantised caches: within float32 rounding of float64 attention over the
    dequantised caches with the query's Q8_0 quantisation (K formats 1, 2)
    -- a wrong kv head, nibble order, scale or format mix-up fails it; the
    group mapping h -> h / (n_heads / n_kv_heads) is checked through head 5."""
    rng = np.random.default_rng(73 + 3 * kf + vf)
    nh, nkv, hd, n_past = 8, 2, 64, 12
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kx = rng.standard_normal((n_past + 1, nkv, hd)).astype(np.float32)
    vx = rng.standard_normal((n_past + 1, nkv, hd)).astype(np.float32)
    kc = np.concatenate([orc.kv_store(r, kf) for r in kx.reshape(n_past + 1, -1)])
    vc = np.concatenate([orc.kv_store(r, vf) for r in vx.reshape(n_past + 1, -1)])
    out = orc.attention_kv(q, kc, vc, n_past, nh, nkv, hd, 1.0, kf, vf).reshape(nh, hd)

    def deq(buf, fmt):
        rows = buf.reshape(n_past + 1, -1)
        if fmt == 0:
            return rows.view(np.float16).astype(np.float64).reshape(n_past + 1, nkv, hd)
        f = orc.dequantize_q8_0 if fmt == 1 else orc.dequantize_q4_0
        return np.stack([f(r, nkv * hd) for r in rows]).astype(np.float64).reshape(n_past + 1, nkv, hd)

    k64, v64 = deq(kc, kf), deq(vc, vf)
    for h in range(nh):
        qh = q[h * hd:(h + 1) * hd]
        q64 = orc.dequantize_q8_0(orc.quantize_q8_0(qh), hd).astype(np.float64) if kf else qh.astype(np.float64)
        sc = k64[:, h // (nh // nkv)] @ q64
        w = np.exp(sc - sc.max())
        w /= w.sum()
        ref = w @ v64[:, h // (nh // nkv)]
        assert np.max(np.abs(out[h] - ref)) <= 2e-5 * max(1.0, np.max(np.abs(ref))), h


def numpy_q4_k_dequant(blocks: np.ndarray, nsb: int) -> np.ndarray:
    """Independent GGUF Q4_K dequantiser (from the published format)."""
    b = blocks.reshape(nsb, 144)
    d = b[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32)
    dmin = b[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float32)
    s = b[:, 4:16].astype(np.int64)
    sc = np.zeros((nsb, 8), np.int64)
    mn = np.zeros((nsb, 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = b[:, 16:].astype(np.int64).reshape(nsb, 4, 32)
    out = np.zeros((nsb, 8, 32), np.float32)
    for c in range(4):
        for half, sub in ((0, 2 * c), (1, 2 * c + 1)):
            q = (qs[:, c, :] >> (4 * half)) & 15
            d1 = (d * sc[:, sub].astype(np.float32)).astype(np.float32)
            m1 = (dmin * mn[:, sub].astype(np.float32)).astype(np.float32)
            out[:, sub, :] = ((d1[:, None] * q.astype(np.float32)).astype(np.float32) - m1[:, None]).astype(np.float32)
    return out.reshape(-1), sc, mn


def test_q4_k_scale_packing_roundtrip(orc, synth):
    rng = np.random.default_rng(7)
    sc = rng.integers(0, 64, (50, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (50, 8), dtype=np.uint8)
    packed = synth.pack_q4_k_scales(sc, mn)
    for i in range(50):
        for j in range(8):
            assert orc.q4_k_scale_min(packed[i], j) == (sc[i, j], mn[i, j])


def test_q4_k_dequant_brute_force(orc, synth):
    rng = synth.rng_for(97)
    w = synth.q4_k_matrix(rng, 3, 512)
    got = orc.dequantize_q4_k(w, 3 * 512)
    ref, _, _ = numpy_q4_k_dequant(w, 6)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_q4_k_dot_brute_force(orc, synth):
    rng = synth.rng_for(96)
    rows, cols = 19, 2304
    nsb = cols // 256
    w = synth.q4_k_matrix(rng, rows, cols)
    a = orc.quantize_q8_0(synth.normal_vector(rng, cols))
    y = orc.mat_vec_mul_q4_k_q8_0(w, a, rows, cols)
    _, sc, mn = numpy_q4_k_dequant(w, rows * nsb)
    b = w.reshape(rows, nsb, 144)
    d = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    dmin = b[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    qs = b[:, :, 16:].astype(np.int64).reshape(rows, nsb, 4, 32)
    qa, da = unpack_q8_0(a, cols // 32)
    qa, da = qa[0].reshape(nsb, 8, 32), da[0].reshape(nsb, 8)
    sc = sc.reshape(rows, nsb, 8)
    mn = mn.reshape(rows, nsb, 8)
    s = np.zeros(rows, np.float32)
    for k in range(nsb):
        for j in range(8):
            q = (qs[:, k, j // 2, :] >> (4 * (j % 2))) & 15
            isum = (q * qa[k, j][None, :]).sum(axis=1)
            bsum = qa[k, j].sum()
            ds = ((d[:, k] * sc[:, k, j].astype(np.float32)).astype(np.float32) * da[k, j]).astype(np.float32)
            dm = ((dmin[:, k] * mn[:, k, j].astype(np.float32)).astype(np.float32) * da[k, j]).astype(np.float32)
            t = ((isum.astype(np.float32) * ds).astype(np.float32)
                 - (np.float32(bsum) * dm).astype(np.float32)).astype(np.float32)
            s = (s + t).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), s.view(np.uint32))
    # float64 dequantised dot agrees to rounding error
    deq, _, _ = numpy_q4_k_dequant(w, rows * nsb)
    xq = (qa * da[..., None]).reshape(-1).astype(np.float64)
    exact = deq.reshape(rows, cols).astype(np.float64) @ xq
    assert np.max(np.abs(y - exact)) <= 1e-4 * np.max(np.abs(exact))


# ---------------------------------------------------------------- committed fixtures
def test_golden_fixture_kats(orc):
    """tests/golden/kats.json: the reference tests' known answers, as data."""
    kats = json.loads((GOLDEN / "kats.json").read_text())
    for case in kats["f32_to_f16_trunc"]:
        assert orc.f32_to_f16(np.float32(case["x"])) == case["h"], case
    for case in kats["q4_0_dot"]:
        w = np.array(case["w"], dtype=np.uint8)
        a = orc.quantize_q8_0(np.array(case["x"], dtype=np.float32))
        assert orc.vec_dot_q4_0_q8_0(w, a, len(case["x"])) == np.float32(case["y"]), case["name"]
    for case in kats["q8_0_quantize"]:
        q = orc.quantize_q8_0(np.array(case["x"], dtype=np.float32))
        assert list(q) == case["bytes"], case["name"]


# ---------------------------------------------------------------- decode step composition
TINY_GEMMA2 = dict(n_layers=2, dim=64, n_heads=4, n_kv_heads=2, head_dim=32, ffn_dim=128, vocab=96,
                   ctx_len=16, rope_base=10000.0, eps=1e-6, attn_scale=1.0 / math.sqrt(32.0))


def numpy_gemma2_step(orc, model, token, pos, kc, vc):
    """The Gemma-2 token step composed independently from the pinned oracle ops
    (model.rs:1164-1201 embedding, per-layer order of model.rs:1185-2260 with
    sandwich norms and a dense GeGLU FFN, tied Q4_0 head, lowest-index argmax)."""
    c = model["cfg"]
    d, hd, nh, nkv = c["dim"], c["head_dim"], c["n_heads"], c["n_kv_heads"]
    qd, kvd, f, V = nh * hd, nkv * hd, c["ffn_dim"], c["vocab"]
    row = model["tok_embd"].reshape(V, -1)[token]
    h = (orc.dequantize_q4_0(row, d) * np.float32(math.sqrt(d))).astype(np.float32)
    for l, L in enumerate(model["layers"]):
        xq = orc.quantize_q8_0(orc.rms_norm(h, L["attn_norm"], c["eps"]))
        q = orc.mat_vec_mul_q4_0_q8_0(L["wq"], xq, qd, d)
        k = orc.mat_vec_mul_q4_0_q8_0(L["wk"], xq, kvd, d)
        v = orc.mat_vec_mul_q4_0_q8_0(L["wv"], xq, kvd, d)
        q = orc.rope_1d_batched(q, pos, nh, hd, c["rope_base"])
        k = orc.rope_1d_batched(k, pos, nkv, hd, c["rope_base"])
        base = l * c["ctx_len"] * kvd
        kc[base + pos * kvd: base + (pos + 1) * kvd] = k.astype(np.float16).view(np.uint16)
        vc[base + pos * kvd: base + (pos + 1) * kvd] = v.astype(np.float16).view(np.uint16)
        att = orc.attention_f16(q, kc[base: base + (pos + 1) * kvd], vc[base: base + (pos + 1) * kvd], pos, nh,
                                nkv, hd, c["attn_scale"])
        o = orc.mat_vec_mul_q4_0_q8_0(L["wo"], orc.quantize_q8_0(att), d, qd)
        h = (h + orc.rms_norm(o, L["post_attn_norm"], c["eps"])).astype(np.float32)
        xq = orc.quantize_q8_0(orc.rms_norm(h, L["ffn_norm"], c["eps"]))
        act = orc.geglu(orc.mat_vec_mul_q4_0_q8_0(L["w_gate"], xq, f, d),
                        orc.mat_vec_mul_q4_0_q8_0(L["w_up"], xq, f, d))
        dn = orc.mat_vec_mul_q4_0_q8_0(L["w_down"], orc.quantize_q8_0(act), d, f)
        h = (h + orc.rms_norm(dn, L["post_ffw_norm"], c["eps"])).astype(np.float32)
    xq = orc.quantize_q8_0(orc.rms_norm(h, model["output_norm"], c["eps"]))
    logits = orc.mat_vec_mul_q4_0_q8_0(model["tok_embd"], xq, V, d)
    return orc.argmax_f32(logits), logits


def test_gemma2_step_matches_independent_composition(orc, synth):
    # numpy's float16 cast is IEEE round-to-nearest-even, the cache rule of the step
    model = synth.gemma2_model(TINY_GEMMA2, seed=9)
    o = orc.OracleGemma2(model)
    kvd = TINY_GEMMA2["n_kv_heads"] * TINY_GEMMA2["head_dim"]
    kc = np.zeros(TINY_GEMMA2["n_layers"] * TINY_GEMMA2["ctx_len"] * kvd, np.uint16)
    vc = np.zeros_like(kc)
    tok = 7
    logits = np.zeros(TINY_GEMMA2["vocab"], np.float32)
    for pos in range(6):
        got = o.step(tok, pos, threads=1, logits=logits)
        want, want_logits = numpy_gemma2_step(orc, model, tok, pos, kc, vc)
        assert got == want
        assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
        assert np.array_equal(o.k_cache, kc) and np.array_equal(o.v_cache, vc)
        tok = got
    # threads split the matvec rows only: the step's bits do not depend on them
    o2 = orc.OracleGemma2(model)
    tok2 = 7
    for pos in range(6):
        tok2 = o2.step(tok2, pos, threads=4)
    assert tok2 == tok and np.array_equal(o2.k_cache, o.k_cache)


# ---------------------------------------------------------------- vocabulary pick

_LIBM = None


def libm_f32(name: str, x: float) -> float:
    """The host C library's f32 routine (the reference's float_tanh / float_exp bind it)."""
    global _LIBM
    if _LIBM is None:
        import ctypes
        import ctypes.util
        _LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
        for fn in ("tanhf", "expf"):
            getattr(_LIBM, fn).argtypes = [ctypes.c_float]
            getattr(_LIBM, fn).restype = ctypes.c_float
    return float(getattr(_LIBM, name)(np.float32(x)))


def numpy_vocab_rank(logits, valid, recent, generated_count, scoring, k):
    """Candidates and ranking restated with numpy: masks as model.rs:2845-2850,
    scores as model.rs:2851-2856 (scoring 0) or kernels.rs:1114-1121 (1),
    then a lexsort on (-score, id)."""
    ids = np.arange(logits.size)
    keep = np.ones(logits.size, bool) if valid is None else valid.astype(bool)
    if generated_count < 4:
        keep[[i for i in (1, 2, 105, 106) if i < logits.size]] = False
    rec = np.asarray(recent, np.int64)
    if scoring == 0:
        sc = np.array([np.float32(30.0) * np.float32(libm_f32("tanhf", np.float32(v) / np.float32(30.0)))
                       for v in logits], np.float32)
        hit = np.isin(ids, rec)
        sc = np.where(hit, sc - np.float32(3.5), sc).astype(np.float32)
    else:
        sc = logits.astype(np.float32).copy()
        for r in rec:  # one subtraction per occurrence, in list order
            if 0 <= r < sc.size:
                sc[r] = np.float32(sc[r] - np.float32(1.8))
    keep &= ~np.isnan(sc)
    ids, sc = ids[keep], sc[keep]
    order = np.lexsort((ids, -sc.astype(np.float64)))[:k]
    return sc[order], ids[order].astype(np.int32)


@pytest.mark.parametrize("scoring", [0, 1])
def test_vocab_select_ranking_brute_force(orc, scoring):
    rng = np.random.default_rng(40 + scoring)
    V = 3000
    # coarse values so equal scores occur and the id tie rule matters
    logits = (rng.integers(-400, 400, V) * 0.125).astype(np.float32)
    logits[[17, 911]] = np.nan
    valid = (rng.random(V) > 0.1).astype(np.uint8)
    recent = [5, 1234, 5, 77, 2999, 0, 1234, 1234]  # duplicates: once (CPU) vs per occurrence (device)
    for gen in (0, 3, 4, 9):
        for k in (1, 7, 40, 64):
            tok, sc, ids = orc.vocab_select(logits, valid, recent, gen, scoring, 0.0, 0, k)
            want_sc, want_ids = numpy_vocab_rank(logits, valid, recent, gen, scoring, k)
            assert np.array_equal(ids, want_ids), (gen, k)
            assert np.array_equal(sc.view(np.uint32), want_sc.view(np.uint32)), (gen, k)
            assert tok == want_ids[0]


def test_vocab_select_early_token_mask(orc):
    logits = np.zeros(200, np.float32)
    logits[[1, 2, 105, 106]] = 5.0
    logits[50] = 4.0
    for gen, want in ((0, 50), (3, 50), (4, 1), (100, 1)):
        assert orc.vocab_select(logits, generated_count=gen)[0] == want
    # the mask drops ids, it does not penalise them: 105 wins once 1 and 2 are invalid
    valid = np.ones(200, np.uint8)
    valid[[1, 2]] = 0
    assert orc.vocab_select(logits, valid, generated_count=4)[0] == 105


def test_vocab_select_penalty_sizes(orc):
    # CPU path: 30*tanh(x/30) then -3.5 once; device path: -1.8 per occurrence
    logits = np.array([10.0, 8.0, 0.0], np.float32)
    _, sc, ids = orc.vocab_select(logits, recent=[0, 0], generated_count=9, scoring=0, k=3)
    t10 = np.float32(30.0) * np.float32(libm_f32("tanhf", np.float32(10.0) / np.float32(30.0)))
    t8 = np.float32(30.0) * np.float32(libm_f32("tanhf", np.float32(8.0) / np.float32(30.0)))
    assert ids.tolist() == [1, 0, 2]  # 9.64 - 3.5 falls below 7.86
    assert sc[0] == t8 and sc[1] == np.float32(t10 - np.float32(3.5)) and sc[2] == 0.0
    _, sc, ids = orc.vocab_select(logits, recent=[0, 0], generated_count=9, scoring=1, k=3)
    assert ids.tolist() == [1, 0, 2] and sc[1] == np.float32(np.float32(10.0 - np.float32(1.8)) - np.float32(1.8))
    _, sc, ids = orc.vocab_select(logits, recent=[0], generated_count=9, scoring=1, k=3)
    assert ids.tolist() == [0, 1, 2] and sc[0] == np.float32(10.0) - np.float32(1.8)


def test_vocab_select_no_candidate_and_nan(orc):
    logits = np.full(16, np.nan, np.float32)
    tok, sc, ids = orc.vocab_select(logits, temperature=1.0, pos=3)
    assert tok == 506 and sc.size == 0 and ids.size == 0
    assert orc.vocab_select(np.zeros(8, np.float32), valid=np.zeros(8, np.uint8))[0] == 506
    logits = np.array([np.nan, -np.inf, -1.0], np.float32)
    tok, sc, ids = orc.vocab_select(logits, generated_count=9, k=5, scoring=1)
    assert tok == 2 and ids.tolist() == [2, 1]


def lcg_rng(pos: int) -> np.float32:
    return np.float32(np.float32(((pos * 6364136223846793005 + 1) % (1 << 64)) >> 33) / np.float32(2**32 - 1))


def test_vocab_select_lcg_uniform_pick(orc):
    # n equal scores: p_i = 1 and acc_i = (i+1)/n (float32 sums), so the pick is
    # the first i with rng <= acc_i: the inverse CDF of a uniform draw
    n = 10
    logits = np.full(n, 2.0, np.float32)
    counts = np.zeros(n, int)
    for pos in range(2000):
        tok = orc.vocab_select(logits, generated_count=9, temperature=0.7, pos=pos, k=n)[0]
        r, acc, want = lcg_rng(pos), np.float32(0.0), n - 1
        for i in range(n):
            acc = np.float32(acc + np.float32(np.float32(1.0) / np.float32(n)))
            if r <= acc:
                want = i
                break
        assert tok == want, pos
        counts[tok] += 1
    # a 64-bit state shifted right by 33 leaves 31 bits, so the draw covers
    # [0, 0.5) only: the reference never samples the upper half of the CDF
    assert counts[: n // 2].min() > 300 and counts[n // 2:].sum() == 0
    assert max(lcg_rng(p) for p in range(2000)) < 0.5
    assert lcg_rng(0) == 0.0 and orc.vocab_select(logits, temperature=1.0, pos=0, k=n)[0] == 0


@pytest.mark.parametrize("temperature", [0.01, 0.5, 2.0])
def test_vocab_select_draw_frequency(orc, temperature):
    # one best score a and nine at b: P(best) = 1 / (1 + 9 exp((b - a) / max(t, 0.1))),
    # drawn with rng uniform on [0, 0.5), so the best is picked with frequency
    # min(1, 2 P(best)); a wrong sign, a missing clamp or a swapped division
    # moves it far from that
    a, b = 1.0, 0.8
    logits = np.array([b] * 5 + [a] + [b] * 4, np.float32)
    t = max(temperature, 0.1)
    p_best = 1.0 / (1.0 + 9 * math.exp((b - a) / t))
    f = min(1.0, 2 * p_best)
    n = 4000
    best = sum(orc.vocab_select(logits, generated_count=9, temperature=temperature, pos=p, k=10)[0] == 5
               for p in range(n))
    assert abs(best / n - f) < 4 * math.sqrt(f * (1 - f) / n) + 0.01
    # two candidates: the best holds at least half the mass, so it is always drawn
    two = np.array([0.8, 1.0], np.float32)
    assert all(orc.vocab_select(two, generated_count=9, temperature=2.0, pos=p, k=2)[0] == 1 for p in range(500))
    assert orc.vocab_select(logits, generated_count=9, temperature=0.0, pos=12345)[0] == 5


def test_vocab_topk_reference_known_answer(orc):
    # ops_test.rs:165-212: the device path's candidates, whatever the
    # partitioning, hold the exact global top-40 of the penalised logits
    N, K = 4096, 40
    i = np.arange(N)
    logits = (((i * 7919) % 65521).astype(np.float32) * np.float32(0.001) +
              i.astype(np.float32) * np.float32(1e-7)).astype(np.float32)
    valid = (i % 17 != 0).astype(np.uint8)
    recent = [31, 777, 2049, 4001]
    _, sc, ids = orc.vocab_select(logits, valid, recent, 10, 1, 0.0, 0, K)
    want = [(s - np.float32(1.8) if t in recent else s, t) for t, s in enumerate(logits) if valid[t]]
    want.sort(key=lambda e: (-float(e[0]), e[1]))
    assert [t for _, t in want[:K]] == ids.tolist()
    assert np.array_equal(np.array([s for s, _ in want[:K]], np.float32).view(np.uint32), sc.view(np.uint32))


# ---------------------------------------------------------------- per-layer windows
_WIN_CFG = dict(n_layers=1, dim=256, n_heads=2, n_kv_heads=1, head_dim=256, ffn_dim=512, vocab=300, ctx_len=64,
                rope_base=10000.0, eps=1e-6, attn_scale=1.0 / 16.0)


def _oracle_logits(orc, model, tokens):
    o = orc.OracleGemma2(model)
    lg = np.zeros(model["cfg"]["vocab"], np.float32)
    out = []
    for pos, t in enumerate(tokens):
        o.step(int(t), pos, logits=lg)
        out.append(lg.copy())
    return out


def test_windowed_layer_equals_a_ring_of_the_window(orc, synth):
    """model.rs:590, 1465-1467: a windowed layer attends the last
    sliding_window positions.  A one-layer model whose layer is windowed
    (period 2: layer 0 is local) with window 5 must give, at every position,
    the bits of the same model without windows over a 5-row cache (a ring
    attends the last min(pos+1, capacity) positions, oldest first); and a
    period of 1 makes every layer global (the bits of no window at all)."""
    tokens = synth.prompt_tokens(20, _WIN_CFG["vocab"], seed=31)
    base = synth.gemma2_model(dict(_WIN_CFG), seed=30)
    win = dict(base, cfg=dict(base["cfg"], sliding_window=5, swa_period=2))
    ring = dict(base, cfg=dict(base["cfg"], ctx_len=5))
    glob = dict(base, cfg=dict(base["cfg"], sliding_window=5, swa_period=1))
    a, b = _oracle_logits(orc, win, tokens), _oracle_logits(orc, ring, tokens)
    c, d = _oracle_logits(orc, glob, tokens), _oracle_logits(orc, base, tokens)
    for pos in range(len(tokens)):
        assert np.array_equal(a[pos].view(np.uint32), b[pos].view(np.uint32)), pos
        assert np.array_equal(c[pos].view(np.uint32), d[pos].view(np.uint32)), pos
    # the window changes the result once positions fall out of it
    assert not np.array_equal(a[-1], d[-1])
