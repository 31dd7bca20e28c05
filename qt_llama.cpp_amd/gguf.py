"""GGUF files for the token step: the C-ABI reader and a version-3 writer.

:class:`GgufFile` mirrors the reference's ``GgufFile``
(``crates/mrml-tensor/src/gguf.rs:71-184``) over the ``mrml_gguf_*`` entry
points of ``libmrml_hip.so`` (``include/mrml_hip.h``): ``GgufFile.open(path)``,
``.version``, ``.data_offset``, ``.tensors`` (name -> info, in key order),
``.get_meta(key)``, ``.read_tensor_bytes(name)``.  Reading needs no GPU.

:func:`write_gguf` writes a version-3 file (header, key/value table, tensor
directory, data aligned to ``general.alignment``), and :func:`write_gemma2` /
:func:`read_gemma2` store and load the random-init Gemma-2 weights of
``synth.gemma2_model`` under the tensor names and metadata keys the reference
loader reads (``token_embd.weight``, ``output_norm.weight``,
``blk.N.attn_q.weight`` ..., ``gemma2.embedding_length``,
``gemma2.block_count``: ``model.rs:413-425,524-525,597-618``).
"""

from __future__ import annotations

import ctypes
import struct
from pathlib import Path

import numpy as np

from . import HipError, load_library

GGUF_MAGIC = 0x46554747

# value type ids (gguf.rs:203-228)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)

# tensor type ids and their (elements, bytes) per block (types.rs:32-70)
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, BF16 = 0, 1, 2, 3, 8, 12, 13, 14, 16, 30
TYPE_LAYOUT = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34), Q4_K: (256, 144),
               Q5_K: (256, 176), Q6_K: (256, 210), IQ4_XS: (256, 136), BF16: (1, 2)}

_SCALAR_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
               BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("size_bytes", ctypes.c_uint64)]


_P, _I64, _U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64
_SIGNATURES = {
    "mrml_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(_P)], ctypes.c_int),
    "mrml_gguf_close": ([_P], ctypes.c_int),
    "mrml_gguf_last_error": ([], ctypes.c_char_p),
    "mrml_gguf_header": ([_P, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_U64), ctypes.POINTER(_I64),
                          ctypes.POINTER(_I64)], ctypes.c_int),
    "mrml_gguf_tensor": ([_P, _I64, ctypes.POINTER(TensorInfo)], ctypes.c_int),
    "mrml_gguf_find_tensor": ([_P, ctypes.c_char_p, ctypes.POINTER(_I64)], ctypes.c_int),
    "mrml_gguf_read_tensor": ([_P, _I64, _P, _U64], ctypes.c_int),
    "mrml_gguf_meta_key": ([_P, _I64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int32)],
                           ctypes.c_int),
    "mrml_gguf_meta_u32": ([_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
    "mrml_gguf_meta_f32": ([_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)], ctypes.c_int),
    "mrml_gguf_meta_str": ([_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U64)],
                           ctypes.c_int),
    "mrml_gguf_meta_array": ([_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_U64)],
                             ctypes.c_int),
}


def _lib():
    lib = load_library()
    if not getattr(lib, "_gguf_bound", False):
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        lib._gguf_bound = True
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


class GgufError(HipError):
    pass


def _check(rc: int) -> None:
    if rc != 0:
        raise GgufError(rc, _lib().mrml_gguf_last_error().decode("utf-8", "replace"))


class GgufFile:
    """An open GGUF file (gguf.rs:71-77): version, metadata, tensor directory
    and data offset; tensor bytes are read on demand."""

    def __init__(self, path: str | Path):
        lib = _lib()
        self.path = str(path)
        h = _P()
        _check(lib.mrml_gguf_open(self.path.encode(), ctypes.byref(h)))
        self._h = h
        ver, off, nt, nm = ctypes.c_uint32(), _U64(), _I64(), _I64()
        _check(lib.mrml_gguf_header(h, ctypes.byref(ver), ctypes.byref(off), ctypes.byref(nt), ctypes.byref(nm)))
        self.version, self.data_offset = int(ver.value), int(off.value)
        self.tensors: dict[str, dict] = {}
        for i in range(nt.value):
            ti = TensorInfo()
            _check(lib.mrml_gguf_tensor(h, i, ctypes.byref(ti)))
            name = ti.name.decode("utf-8")
            self.tensors[name] = {"index": i, "name": name, "type": int(ti.type), "n_dims": int(ti.n_dims),
                                  "dims": [int(d) for d in ti.dims], "offset": int(ti.offset),
                                  "size_bytes": int(ti.size_bytes)}
        self.meta_keys: list[tuple[str, int]] = []
        for i in range(nm.value):
            k, t = ctypes.c_char_p(), ctypes.c_int32()
            _check(lib.mrml_gguf_meta_key(h, i, ctypes.byref(k), ctypes.byref(t)))
            self.meta_keys.append((k.value.decode("utf-8"), int(t.value)))

    @classmethod
    def open(cls, path: str | Path) -> "GgufFile":
        return cls(path)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib().mrml_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _key_type(self, key: str) -> int | None:
        for k, t in self.meta_keys:
            if k == key:
                return t
        return None

    def meta_u32(self, key: str) -> int | None:
        """GgufValue::as_u32 of `key`, or None (gguf.rs:25-36)."""
        v = ctypes.c_uint32()
        rc = _lib().mrml_gguf_meta_u32(self._h, key.encode(), ctypes.byref(v))
        return int(v.value) if rc == 0 else None

    def meta_f32(self, key: str) -> float | None:
        """GgufValue::as_f32 of `key`, or None (gguf.rs:38-45)."""
        v = ctypes.c_float()
        rc = _lib().mrml_gguf_meta_f32(self._h, key.encode(), ctypes.byref(v))
        return float(v.value) if rc == 0 else None

    def meta_str(self, key: str) -> str | None:
        """GgufValue::as_str of `key`, or None (gguf.rs:47-52)."""
        p, n = ctypes.c_char_p(), _U64()
        rc = _lib().mrml_gguf_meta_str(self._h, key.encode(), ctypes.byref(p), ctypes.byref(n))
        return ctypes.string_at(p, n.value).decode("utf-8") if rc == 0 else None

    def meta_array(self, key: str) -> tuple[int, int] | None:
        """(item type, length) of an array value, or None (gguf.rs:54-59)."""
        t, n = ctypes.c_int32(), _U64()
        rc = _lib().mrml_gguf_meta_array(self._h, key.encode(), ctypes.byref(t), ctypes.byref(n))
        return (int(t.value), int(n.value)) if rc == 0 else None

    def read_tensor_bytes(self, name: str) -> np.ndarray:
        """GgufFile::read_tensor_bytes (gguf.rs:173-183) as a uint8 array."""
        info = self.tensors.get(name)
        if info is None:
            raise GgufError(-8, f"GGUF: no tensor named {name}")
        out = np.empty(info["size_bytes"], np.uint8)
        _check(_lib().mrml_gguf_read_tensor(self._h, info["index"], out.ctypes.data, out.nbytes))
        return out


# ---- writer -------------------------------------------------------------------

def _enc_str(s: str | bytes) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _enc_value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _enc_str(value)
    if vtype == ARRAY:
        item_type, items = value
        return struct.pack("<IQ", item_type, len(items)) + b"".join(_enc_value(item_type, v) for v in items)
    if vtype == BOOL:
        return struct.pack("<B", 1 if value else 0)
    return struct.pack(_SCALAR_FMT[vtype], value)


def write_gguf(path: str | Path, metadata: list[tuple[str, int, object]],
               tensors: list[tuple[str, list[int], int, np.ndarray]], alignment: int = 32,
               version: int = 3) -> None:
    """Write a GGUF file: `metadata` as (key, value type, value) -- an ARRAY
    value is (item type, [items]) -- and `tensors` as (name, dims in ggml order,
    type id, bytes).  Each tensor's bytes must match numel / block * block
    bytes; tensors are laid out in the given order, each at an offset that is a
    multiple of `alignment` (written as general.alignment when it is not 32 and
    the caller did not)."""
    meta = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", UINT32, alignment))
    head = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(meta)))
    for key, vtype, value in meta:
        head += _enc_str(key) + struct.pack("<I", vtype) + _enc_value(vtype, value)
    offsets, off = [], 0
    blobs = []
    for name, dims, ttype, data in tensors:
        block, nbytes = TYPE_LAYOUT[ttype]
        numel = int(np.prod(dims, dtype=np.uint64)) if dims else 1
        blob = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        if numel % block or blob.nbytes != numel // block * nbytes:
            raise ValueError(f"{name}: {blob.nbytes} bytes for {numel} elements of type {ttype}")
        offsets.append(off)
        blobs.append(blob)
        off = (off + blob.nbytes + alignment - 1) // alignment * alignment
    for (name, dims, ttype, _), o in zip(tensors, offsets):
        head += _enc_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        pos = 0
        for blob, o in zip(blobs, offsets):
            f.write(b"\0" * (o - pos))
            f.write(memoryview(blob))
            pos = o + blob.nbytes


# ---- Gemma-2 weights ------------------------------------------------------------

_LAYER_TENSORS = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "w_gate": "ffn_gate",
                  "w_up": "ffn_up", "w_down": "ffn_down"}
_LAYER_NORMS = {"attn_norm": "attn_norm", "post_attn_norm": "post_attention_norm", "ffn_norm": "ffn_norm",
                "post_ffw_norm": "post_ffw_norm"}


def _gemma2_shapes(cfg: dict) -> dict:
    d, qd = cfg["dim"], cfg["n_heads"] * cfg["head_dim"]
    kvd, f = cfg["n_kv_heads"] * cfg["head_dim"], cfg["ffn_dim"]
    return {"wq": (qd, d), "wk": (kvd, d), "wv": (kvd, d), "wo": (d, qd), "w_gate": (f, d), "w_up": (f, d),
            "w_down": (d, f)}


def write_gemma2(path: str | Path, model: dict) -> None:
    """Store a Gemma-2 weight set (the dict of synth.gemma2_model) as GGUF."""
    cfg = model["cfg"]
    meta = [("general.architecture", STRING, "gemma2"),
            ("gemma2.block_count", UINT32, cfg["n_layers"]),
            ("gemma2.embedding_length", UINT32, cfg["dim"]),
            ("gemma2.feed_forward_length", UINT32, cfg["ffn_dim"]),
            ("gemma2.attention.head_count", UINT32, cfg["n_heads"]),
            ("gemma2.attention.head_count_kv", UINT32, cfg["n_kv_heads"]),
            ("gemma2.attention.key_length", UINT32, cfg["head_dim"]),
            ("gemma2.context_length", UINT32, cfg["ctx_len"]),
            ("gemma2.rope.freq_base", FLOAT32, cfg["rope_base"]),
            ("gemma2.attention.layer_norm_rms_epsilon", FLOAT32, cfg["eps"]),
            ("gemma2.attention.scale", FLOAT32, cfg["attn_scale"])]
    ttype = Q8_0 if model["tie_q8"] else Q4_0
    tensors = [("token_embd.weight", [cfg["dim"], cfg["vocab"]], ttype, model["tok_embd"]),
               ("output_norm.weight", [cfg["dim"]], F32, model["output_norm"])]
    shapes = _gemma2_shapes(cfg)
    for li, L in enumerate(model["layers"]):
        for key, name in _LAYER_TENSORS.items():
            rows, cols = shapes[key]
            tensors.append((f"blk.{li}.{name}.weight", [cols, rows], Q4_0, L[key]))
        for key, name in _LAYER_NORMS.items():
            tensors.append((f"blk.{li}.{name}.weight", [cfg["dim"]], F32, L[key]))
    write_gguf(path, meta, tensors)


def read_gemma2(path: str | Path) -> dict:
    """Load a Gemma-2 weight set written by write_gemma2 (or any GGUF with those
    names and keys) into the dict form of synth.gemma2_model.  Shapes and types
    are checked against the metadata."""
    with GgufFile(path) as g:
        def need(v, what):
            if v is None:
                raise GgufError(-8, f"GGUF: missing {what}")
            return v

        te = need(g.tensors.get("token_embd.weight"), "token_embd.weight")
        cfg = {"n_layers": need(g.meta_u32("gemma2.block_count"), "gemma2.block_count"),
               "dim": need(g.meta_u32("gemma2.embedding_length"), "gemma2.embedding_length"),
               "n_heads": need(g.meta_u32("gemma2.attention.head_count"), "head_count"),
               "n_kv_heads": need(g.meta_u32("gemma2.attention.head_count_kv"), "head_count_kv"),
               "head_dim": need(g.meta_u32("gemma2.attention.key_length"), "key_length"),
               "ffn_dim": need(g.meta_u32("gemma2.feed_forward_length"), "feed_forward_length"),
               "vocab": te["dims"][1],
               "ctx_len": need(g.meta_u32("gemma2.context_length"), "context_length"),
               "rope_base": g.meta_f32("gemma2.rope.freq_base") or 10000.0,
               "eps": g.meta_f32("gemma2.attention.layer_norm_rms_epsilon") or 1e-6}
        scale = g.meta_f32("gemma2.attention.scale")
        cfg["attn_scale"] = scale if scale is not None else float(np.float32(cfg["head_dim"]) ** np.float32(-0.5))
        if te["type"] not in (Q4_0, Q8_0) or te["dims"][0] != cfg["dim"]:
            raise GgufError(-6, f"token_embd.weight: type {te['type']}, dims {te['dims'][:2]}")
        shapes = _gemma2_shapes(cfg)

        def matrix(name, rows, cols):
            t = need(g.tensors.get(name), name)
            if t["type"] != Q4_0 or t["dims"][:2] != [cols, rows]:
                raise GgufError(-6, f"{name}: type {t['type']}, dims {t['dims'][:2]}, want Q4_0 {[cols, rows]}")
            return g.read_tensor_bytes(name)

        def norm(name):
            t = need(g.tensors.get(name), name)
            if t["type"] != F32 or t["dims"][0] != cfg["dim"]:
                raise GgufError(-6, f"{name}: type {t['type']}, dims {t['dims'][:1]}, want F32 [{cfg['dim']}]")
            return g.read_tensor_bytes(name).view(np.float32)

        layers = []
        for li in range(cfg["n_layers"]):
            L = {key: matrix(f"blk.{li}.{name}.weight", *shapes[key]) for key, name in _LAYER_TENSORS.items()}
            L.update({key: norm(f"blk.{li}.{name}.weight") for key, name in _LAYER_NORMS.items()})
            layers.append(L)
        return {"cfg": cfg, "tie_q8": te["type"] == Q8_0, "tok_embd": g.read_tensor_bytes("token_embd.weight"),
                "output_norm": norm("output_norm.weight"), "layers": layers}
