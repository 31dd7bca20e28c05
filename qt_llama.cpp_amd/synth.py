"""Seeded synthetic inputs in GGUF byte layout for the benchmark configurations.

Weights are emitted directly as GGUF block bytes (the reference uploads GGUF
bytes unchanged, crates/mrml-tensor/src/model.rs:651-705), with the value
distributions of the benchmark configurations:

* Q8_0: quants uniform in [-127, 127], scale f16(|N(0, sigma)| / 127)
* Q4_0: nibbles uniform in 0..15 (value q - 8), scale f16(|N(0, sigma)| / 8)
* Q4_K: d, dmin = f16(|N(0, 0.01)|), 6-bit scales and mins uniform in 0..63,
  nibbles uniform (GGUF super-block: f16 d, f16 dmin, u8 scales[12], u8 qs[128])

Scales are rounded to f16 with numpy (round-to-nearest-even); this is data
generation only and both the GPU and the CPU oracle read the same bytes.
"""

from __future__ import annotations

import numpy as np


def rng_for(config: int, seed: int = 0x4D524D4C) -> np.random.Generator:
    """One PCG64 stream per (config, seed)."""
    return np.random.Generator(np.random.PCG64([seed, config]))


def _f16_bits(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint16)


def q4_0_matrix(rng: np.random.Generator, rows: int, cols: int, sigma: float = 0.02,
                symmetric: bool = False) -> np.ndarray:
    """Q4_0 blocks; nibbles uniform in 0..15, or in 1..15 (values -7..7, mean 0)
    with `symmetric`."""
    nb = cols // 32
    blocks = np.empty((rows * nb, 18), dtype=np.uint8)
    d = _f16_bits(np.abs(rng.standard_normal(rows * nb, dtype=np.float32)) * np.float32(sigma) / np.float32(8.0))
    blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    if symmetric:
        lo = rng.integers(1, 16, size=(rows * nb, 16), dtype=np.uint8)
        hi = rng.integers(1, 16, size=(rows * nb, 16), dtype=np.uint8)
        blocks[:, 2:] = lo | (hi << 4)
    else:
        blocks[:, 2:] = rng.integers(0, 256, size=(rows * nb, 16), dtype=np.uint8)
    return blocks.reshape(-1)


def q8_0_matrix(rng: np.random.Generator, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    nb = cols // 32
    blocks = np.empty((rows * nb, 34), dtype=np.uint8)
    d = _f16_bits(np.abs(rng.standard_normal(rows * nb, dtype=np.float32)) * np.float32(sigma) / np.float32(127.0))
    blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = rng.integers(-127, 128, size=(rows * nb, 32), dtype=np.int8).view(np.uint8)
    return blocks.reshape(-1)


def pack_q4_k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Encode 8 six-bit (scale, min) pairs per super-block into GGUF's 12 bytes
    (the inverse of get_scale_min_k4).  sc, m: uint8 arrays [..., 8]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.empty(sc.shape[:-1] + (12,), dtype=np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (m[..., j] & 63) | ((m[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 0x0F) | ((m[..., j + 4] & 0x0F) << 4)
    return out


def q4_k_matrix(rng: np.random.Generator, rows: int, cols: int, sigma: float = 0.01) -> np.ndarray:
    nsb = rows * (cols // 256)
    blocks = np.empty((nsb, 144), dtype=np.uint8)
    dd = _f16_bits(np.abs(rng.standard_normal((nsb, 2), dtype=np.float32)) * np.float32(sigma))
    blocks[:, 0:4] = dd.view(np.uint8).reshape(nsb, 4)
    sc = rng.integers(0, 64, size=(nsb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(nsb, 8), dtype=np.uint8)
    blocks[:, 4:16] = pack_q4_k_scales(sc, mn)
    blocks[:, 16:] = rng.integers(0, 256, size=(nsb, 128), dtype=np.uint8)
    return blocks.reshape(-1)


def normal_vector(rng: np.random.Generator, n: int) -> np.ndarray:
    return rng.standard_normal(n, dtype=np.float32)


def rms_normalised(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps), float32 (shape of the FFN input; not a parity path)."""
    x = np.asarray(x, dtype=np.float32)
    s = np.float32(np.mean(x.astype(np.float64) ** 2))
    return (x / np.sqrt(s + np.float32(eps))).astype(np.float32)


# Gemma-2-2B architecture (the decode configuration: 26 layers, hidden 2304,
# 8 query / 4 KV heads of 256, GeGLU FFN 9216, RoPE base 10000, tied
# 256000-entry table, f16 KV cache of 4096 positions).
GEMMA2_2B = dict(n_layers=26, dim=2304, n_heads=8, n_kv_heads=4, head_dim=256, ffn_dim=9216, vocab=256000,
                 ctx_len=4096, rope_base=10000.0, eps=1e-6, attn_scale=1.0 / 16.0)

GEMMA2_MATRICES = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
GEMMA2_NORMS = ("attn_norm", "post_attn_norm", "ffn_norm", "post_ffw_norm")


def gemma2_shapes(cfg: dict) -> dict:
    """(rows, cols) of each layer matrix."""
    d, qd = cfg["dim"], cfg["n_heads"] * cfg["head_dim"]
    kvd, f = cfg["n_kv_heads"] * cfg["head_dim"], cfg["ffn_dim"]
    return {"wq": (qd, d), "wk": (kvd, d), "wv": (kvd, d), "wo": (d, qd),
            "w_gate": (f, d), "w_up": (f, d), "w_down": (d, f)}


def gemma2_model(cfg: dict, seed: int = 4, tie_q8: bool = False) -> dict:
    """Random-init Gemma-2-architecture weights as GGUF block bytes.

    Matrices are Q4_0 with d = f16(|N(0, 0.02)| / 8) and nibbles uniform in
    1..15: weights -7..7 with mean 0.  (Nibbles uniform in 0..15 have mean
    -0.5, which gives every projection a shared component along the sum of its
    input; through 26 layers that common mode decides the argmax for any
    token.)  The tied table is Q4_0 (or Q8_0); norm weights are f32
    1 + 0.1 N(0, 1).
    """
    rng = rng_for(100 + seed)
    shapes = gemma2_shapes(cfg)
    layers = []
    for _ in range(cfg["n_layers"]):
        L = {name: q4_0_matrix(rng, *shapes[name], symmetric=True) for name in GEMMA2_MATRICES}
        for name in GEMMA2_NORMS:
            L[name] = (1.0 + 0.1 * rng.standard_normal(cfg["dim"], dtype=np.float32)).astype(np.float32)
        layers.append(L)
    if tie_q8:
        table = q8_0_matrix(rng, cfg["vocab"], cfg["dim"])
    else:
        table = q4_0_matrix(rng, cfg["vocab"], cfg["dim"], symmetric=True)
    out_norm = (1.0 + 0.1 * rng.standard_normal(cfg["dim"], dtype=np.float32)).astype(np.float32)
    return {"cfg": dict(cfg), "tie_q8": tie_q8, "tok_embd": table, "output_norm": out_norm, "layers": layers}


def prompt_tokens(n: int, vocab: int, seed: int = 5) -> np.ndarray:
    """A seeded random token prompt."""
    return rng_for(200 + seed).integers(0, vocab, size=n, dtype=np.int32)
