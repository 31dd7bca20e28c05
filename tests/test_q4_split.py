"""The split-nibble form of a Q8_0 activation block used by the Q4_0 kernels.

The kernels replace the nibble-unpacking Q4_0 x Q8_0 block dot (the integer
sum of ggml's vec_dot_q4_0_q8_0, quant.rs block dot: sum_k (q_k - 8) * a_k)
with 8 dot8 instructions on the raw weight words against a re-encoded
activation block (device.h, split_lo / split_hi / q4_0_isum_split).  This
emulates those instructions bit for bit on the CPU (v_dot8_i32_i4: signed
nibble products, v_dot8_u32_u4: unsigned, both accumulating modulo 2^32) and
checks the identity against the plain block dot on random blocks and on the
extreme ones (every weight nibble 0 or 15, quants -128 / 127 / 0).
"""

from __future__ import annotations

import numpy as np

M32 = 0xFFFFFFFF
LO_NIB = 0x0F0F0F0F


def nibbles(word: int) -> list[int]:
    return [(word >> (4 * i)) & 15 for i in range(8)]


def sdot8(a: int, b: int, c: int) -> int:
    s4 = lambda n: n - 16 if n >= 8 else n
    return (c + sum(s4(x) * s4(y) for x, y in zip(nibbles(a), nibbles(b)))) & M32


def udot8(a: int, b: int, c: int) -> int:
    return (c + sum(x * y for x, y in zip(nibbles(a), nibbles(b)))) & M32


def split_lo(x: int, y: int) -> int:
    return (x & LO_NIB) | (((y & LO_NIB) << 4) & M32)


def split_hi(x: int, y: int) -> int:
    return ((x >> 4) & LO_NIB) | (y & ~LO_NIB & M32)


def words(b: np.ndarray) -> list[int]:
    """Little-endian 32-bit words of a byte array."""
    return [int(v) for v in b.astype(np.uint8).view("<u4")]


def isum_split(wq: np.ndarray, a: np.ndarray) -> int:
    """The kernel's block dot: wq = 16 packed weight bytes, a = 32 int8 quants."""
    w = words(wq)
    aw = words(a.astype(np.int8).view(np.uint8))
    lo = [split_lo(aw[i], aw[4 + i]) for i in range(4)]
    hi = [split_hi(aw[i], aw[4 + i]) for i in range(4)]
    c = (-8 * int(np.sum(a.astype(np.int64) & 15))) & M32
    sh = 0
    for i in range(4):
        sh = sdot8(w[i] ^ 0x88888888, hi[i], sh)
    sl = c
    for i in range(4):
        sl = udot8(w[i], lo[i], sl)
    r = ((sh << 4) + sl) & M32
    return r - (1 << 32) if r >= 1 << 31 else r


def isum_plain(wq: np.ndarray, a: np.ndarray) -> int:
    """GGUF Q4_0 block: byte k holds q[k] (low nibble) and q[k+16] (high)."""
    q = np.concatenate([wq & 15, wq >> 4]).astype(np.int64)
    return int(np.sum((q - 8) * a.astype(np.int64)))


def test_split_identity_random():
    rng = np.random.default_rng(7)
    for _ in range(400):
        wq = rng.integers(0, 256, 16, dtype=np.int64).astype(np.uint8)
        a = rng.integers(-128, 128, 32)
        assert isum_split(wq, a) == isum_plain(wq, a)


def test_split_identity_extremes():
    rng = np.random.default_rng(11)
    for wfill in (0x00, 0xFF, 0x0F, 0xF0, 0x88, 0x77):
        wq = np.full(16, wfill, np.uint8)
        for a in (np.full(32, 127), np.full(32, -128), np.zeros(32, np.int64), np.full(32, -1),
                  np.where(np.arange(32) % 2 == 0, 127, -128), rng.integers(-128, 128, 32)):
            assert isum_split(wq, a) == isum_plain(wq, a)


def test_split_value_decomposition():
    """Every int8 value is 16*hi + lo with hi the signed and lo the unsigned nibble."""
    for v in range(-128, 128):
        b = v & 0xFF
        hi, lo = b >> 4, b & 15
        hi = hi - 16 if hi >= 8 else hi
        assert 16 * hi + lo == v
