"""Host-side mirror of the reference's GPU operator surface over the C ABI.

The reference (mitchellrenouf/QT_llama.cpp) drives its GPU path through
``CudaDevice`` / ``CudaBuffer`` in ``crates/mrml-tensor/src/cuda.rs``.  This
module gives the same surface -- ``HipDevice.new(0)``, ``HipBuffer.from_host``,
``dev.gemv_q4_0(w, x, y, rows, cols)``, ``dev.sync()`` ... -- over
``lib/libmrml_hip.so`` (``include/mrml_hip.h``) with ctypes and numpy, so
callers and tests read like the reference's own ``tests/ops_test.rs``.

Differences from the reference surface, all deliberate:

* Errors raise :class:`HipError` instead of panicking (the reference's op
  wrappers ``.expect()`` every launch, e.g. ``cuda.rs:2304``).
* Quantised weights are converted once to the backend layout
  (``HipBuffer.from_gguf``); ``gemv_q4_0_gguf`` reads raw GGUF bytes.
* Matvec outputs follow the reference CPU semantics (Q8_0-quantised
  activations, exact integer block dots, ordered f32 fold), not the
  reference CUDA kernels' f32 dequantise-and-FMA.

There is no CPU fallback: if the library or a gfx950 device is missing,
construction raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libmrml_hip.so"

Q4_0 = 2
Q8_0 = 8
Q4_K = 12

# bytes per block and weights per block, GGUF (types.rs:32-70)
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144}
BLOCK_WEIGHTS = {Q4_0: 32, Q8_0: 32, Q4_K: 256}

_STATUS = {
    0: "ok",
    -1: "invalid argument",
    -2: "allocation failed",
    -3: "HIP runtime error",
    -4: "unsupported",
    -5: "no gfx950 device",
    -6: "malformed GGUF file",
    -7: "file I/O error",
    -8: "not found",
}


class HipError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS.get(status, status)}: {message}")
        self.status = status


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("runtime_version", ctypes.c_int32),
        ("abi_version", ctypes.c_int32),
        ("total_memory", ctypes.c_uint64),
        ("l2_bytes", ctypes.c_uint64),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int32
_Z = ctypes.c_size_t
_F = ctypes.c_float


class Gemma2Config(ctypes.Structure):
    """mrml_hip_gemma2_config."""

    _fields_ = [(n, ctypes.c_int32) for n in
                ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "ctx_len")] + \
               [(n, ctypes.c_float) for n in ("rope_base", "eps", "attn_scale")] + \
               [("tie_type", ctypes.c_int32), ("numerics", ctypes.c_int32), ("sliding_window", ctypes.c_int32),
                ("swa_period", ctypes.c_int32)]


NUMERICS_EXACT = 0
NUMERICS_FAST = 1


GEMMA2_LAYER_TENSORS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
GEMMA2_LAYER_NORMS = ("attn_norm", "post_attn_norm", "ffn_norm", "post_ffw_norm")


class Gemma2Layer(ctypes.Structure):
    """mrml_hip_gemma2_layer: device pointers of one layer."""

    _fields_ = [(n, ctypes.c_void_p) for n in GEMMA2_LAYER_TENSORS + GEMMA2_LAYER_NORMS]

SCORE_CPU, SCORE_DEVICE = 0, 1


class Sampler(ctypes.Structure):
    """mrml_hip_sampler: the pick of the token step (model.rs:2842-2907)."""

    _fields_ = [("d_valid", ctypes.c_void_p), ("temperature", ctypes.c_float), ("top_k", ctypes.c_int32)]


# name -> argtypes; every function returns int status unless listed in _RESTYPE
_SIGNATURES = {
    "mrml_hip_device_count": [ctypes.POINTER(ctypes.c_int32)],
    "mrml_hip_create": [_I, ctypes.POINTER(_P)],
    "mrml_hip_destroy": [_P],
    "mrml_hip_last_error": [_P],
    "mrml_hip_status_string": [ctypes.c_int],
    "mrml_hip_sync": [_P],
    "mrml_hip_set_wait_limit": [_P, _I],
    "mrml_hip_device_info_get": [_P, ctypes.POINTER(DeviceInfo)],
    "mrml_hip_memory_info": [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "mrml_hip_stream": [_P],
    "mrml_hip_reserve_workspace": [_P, _Z],
    "mrml_hip_workspace_bytes": [_P, ctypes.POINTER(ctypes.c_size_t)],
    "mrml_hip_graph_begin": [_P],
    "mrml_hip_graph_end": [_P, ctypes.POINTER(_P)],
    "mrml_hip_graph_launch": [_P, _P],
    "mrml_hip_graph_destroy": [_P, _P],
    "mrml_hip_malloc": [_P, _Z, ctypes.POINTER(_P)],
    "mrml_hip_free": [_P, _P],
    "mrml_hip_memcpy_h2d": [_P, _P, _P, _Z],
    "mrml_hip_memcpy_d2h": [_P, _P, _P, _Z],
    "mrml_hip_memcpy_h2d_async": [_P, _P, _P, _Z],
    "mrml_hip_memcpy_d2d_async": [_P, _P, _P, _Z],
    "mrml_hip_zero_async": [_P, _P, _Z],
    "mrml_hip_copy_kernel": [_P, _P, _P, _Z],
    "mrml_hip_read_kernel": [_P, _P, _Z, _P],
    "mrml_hip_repack_q4_0": [_P, _P, _P, _I, _I],
    "mrml_hip_repack_q8_0": [_P, _P, _P, _I, _I],
    "mrml_hip_repack_q4_k": [_P, _P, _P, _I, _I],
    "mrml_hip_quantize_q8_0": [_P, _P, _P, _P, _I],
    "mrml_hip_q8_0_pack_bytes": [_I],
    "mrml_hip_gemv_q4_0": [_P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q4_0_q8": [_P, _P, _P, _P, _I, _I],
"mrml_hip_gemv_q4_0_q8_relaxed": [_P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q4_0_gguf": [_P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q4_0_geglu": [_P, _P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q4_0_qkv": [_P, _P, _P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemv_q4_0_geglu_q8": [_P, _P, _P, _P, _P, _I, _I],
    "mrml_hip_ffn_geglu_q4_0": [_P, _P, _P, _P, _P, _P, _P, _I, _I],
    "mrml_hip_ffn_split_geglu": [_P, _P, _P, _P, _P, _P, _P, _I, _I],
    "mrml_hip_ffn_split_down": [_P, _P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q4_0_geglu_pack": [_P, _P, _P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q4_0_qkv_q8": [_P, _P, _P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemv_q8_0": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemv_q4_k": [_P, _P, _P, _P, _I, _I],
    "mrml_hip_gemv_q8_0_q8": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemv_q4_k_q8": [_P, _P, _P, _P, _I, _I],
    "mrml_hip_gemm_q4_0": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemm_q4_0_q8": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemm_q4_0_noalloc": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemm_q4_0_relaxed": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_gemm_q4_0_qkv": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
    "mrml_hip_gemm_q4_0_geglu": [_P, _P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_rms_norm_batch": [_P, _P, _P, _P, _I, _I, _F],
    "mrml_hip_gemm_q4_0_noalloc_max_pack_bytes": [],
    "mrml_hip_gemm_pack_bytes": [_I, _I],
    "mrml_hip_quantize_q8_0_gemm": [_P, _P, _P, _I, _I],
    "mrml_hip_gemm_q4_0_gpack": [_P, _P, _P, _P, _I, _I, _I],
    "mrml_hip_argmax_f32": [_P, _P, _I, _P],
    "mrml_hip_vocab_topk": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I],
    "mrml_hip_vocab_select": [_P, _P, _I, _P, _P, _I, _I, _I, _F, ctypes.c_uint64, _I, _P, _P, _P],
    "mrml_hip_gemma2_set_sampler": [_P, _P, _P],
    "mrml_hip_rms_norm": [_P, _P, _P, _P, _P, _I, _F],
    "mrml_hip_residual_rms_norm": [_P, _P, _P, _P, _P, _P, _P, _I, _F],
    "mrml_hip_embedding": [_P, _P, _I, _I, _P, _P, _I, _I, _F],
    "mrml_hip_rope_table": [_P, _P, _I, _I, _F, _F],
    "mrml_hip_rope_kv_append_f16": [_P, _P, _P, _P, _I, _P, _I, _I, _I, _F, _F, _I, _P, _I],
    "mrml_hip_attn_decode_f16": [_P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _F, _I],
    "mrml_hip_attn_decode_f16_split": [_P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _F, _I],
    "mrml_hip_rope_kv_append_f16_batch": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _I, _I, _I, _P, _I],
    "mrml_hip_rope": [_P, _P, _I, _I, _I, _F, _F, _P, _I],
    "mrml_hip_geglu": [_P, _P, _P, _P, _I],
    "mrml_hip_swiglu": [_P, _P, _P, _P, _I],
    "mrml_hip_add": [_P, _P, _P, _P, _I],
    "mrml_hip_attention_prefill": [_P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I, _I],
    "mrml_hip_attention_causal": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _I],
    "mrml_hip_attention_causal_split": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _I],
    "mrml_hip_gemma2_create": [_P, _P, _P, _P, _P, ctypes.POINTER(_P)],
    "mrml_hip_gemma2_destroy": [_P, _P],
    "mrml_hip_gemma2_step": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I],
    "mrml_hip_gemma2_activations": [_P, _P, ctypes.POINTER(_P), ctypes.POINTER(_P)],
    "mrml_hip_gemma2_prefill": [_P, _P, _P, _I, _I, _P, _P, _P, _P],
    "mrml_hip_gemma2_reserve_prefill": [_P, _P],
}
_RESTYPE = {
    "mrml_hip_last_error": ctypes.c_char_p,
    "mrml_hip_status_string": ctypes.c_char_p,
    "mrml_hip_stream": _P,
    "mrml_hip_q8_0_pack_bytes": _Z,
    "mrml_hip_gemm_pack_bytes": _Z,
    "mrml_hip_gemm_q4_0_noalloc_max_pack_bytes": _Z,
}

_lib = None


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libmrml_hip.so and declare every exported C-ABI function."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise HipError(-4, f"{p} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    if path is None:
        _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def device_count() -> int:
    n = ctypes.c_int32(0)
    load_library().mrml_hip_device_count(ctypes.byref(n))
    return int(n.value)


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, HipBuffer):
        return x.ptr
    return int(x)


class HipBuffer:
    """A device allocation (CudaBuffer, cuda.rs:1243-1513).  Frees on close/GC."""

    def __init__(self, dev: "HipDevice", nbytes: int, dtype=np.uint8, shape=None):
        self.dev = dev
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = ctypes.c_void_p()
        dev._check(dev.lib.mrml_hip_malloc(dev.ctx, self.nbytes, ctypes.byref(p)))
        self.ptr = int(p.value)

    # CudaBuffer::alloc_on / from_host_on
    @classmethod
    def alloc(cls, dev: "HipDevice", count: int, dtype=np.float32) -> "HipBuffer":
        dt = np.dtype(dtype)
        return cls(dev, count * dt.itemsize, dt, (count,))

    @classmethod
    def from_host(cls, dev: "HipDevice", arr: np.ndarray) -> "HipBuffer":
        arr = np.ascontiguousarray(arr)
        b = cls(dev, arr.nbytes, arr.dtype, arr.shape)
        b.copy_from_host(arr)
        return b

    @classmethod
    def from_gguf(cls, dev: "HipDevice", gguf_bytes: np.ndarray, qtype: int, rows: int, cols: int) -> "HipBuffer":
        """Upload a GGUF-layout quantised matrix and convert it to the backend layout."""
        raw = cls.from_host(dev, np.ascontiguousarray(gguf_bytes, dtype=np.uint8).reshape(-1))
        try:
            out = cls(dev, raw.nbytes, np.uint8)
            fn = {Q4_0: dev.lib.mrml_hip_repack_q4_0, Q8_0: dev.lib.mrml_hip_repack_q8_0,
                  Q4_K: dev.lib.mrml_hip_repack_q4_k}[qtype]
            dev._check(fn(dev.ctx, raw.ptr, out.ptr, rows, cols))
            dev.sync()
        finally:
            raw.close()
        return out

    def copy_from_host(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {arr.nbytes} != {self.nbytes}")
        self.dev._check(self.dev.lib.mrml_hip_memcpy_h2d(self.dev.ctx, self.ptr, arr.ctypes.data, arr.nbytes))

    def copy_to_host(self, out: np.ndarray | None = None) -> np.ndarray:
        if out is None:
            out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {out.nbytes} != {self.nbytes}")
        self.dev._check(self.dev.lib.mrml_hip_memcpy_d2h(self.dev.ctx, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def numpy(self) -> np.ndarray:
        return self.copy_to_host()

    def close(self) -> None:
        if self.ptr and self.dev.ctx:
            self.dev.lib.mrml_hip_free(self.dev.ctx, self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipDevice:
    """One context = one device + one stream (CudaDevice, cuda.rs:1883-3112)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        ctx = ctypes.c_void_p()
        rc = self.lib.mrml_hip_create(device, ctypes.byref(ctx))
        if rc != 0:
            raise HipError(rc, f"mrml_hip_create({device})")
        self.ctx = ctx.value
        self.device = device

    @classmethod
    def new(cls, device: int = 0) -> "HipDevice":
        return cls(device)

    @staticmethod
    def is_available() -> bool:
        try:
            return device_count() > 0
        except Exception:
            return False

    def _check(self, rc: int) -> None:
        if rc != 0:
            msg = self.lib.mrml_hip_last_error(self.ctx) or b""
            raise HipError(rc, msg.decode(errors="replace"))

    def close(self) -> None:
        if self.ctx:
            self.lib.mrml_hip_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- lifecycle -----------------------------------------------------------
    def sync(self) -> None:
        self._check(self.lib.mrml_hip_sync(self.ctx))

    def set_wait_limit(self, polls: int) -> None:
        """Poll limit of the kernels' bounded waits on this device (< 0: the
        default; 0: every wait gives up, and the next sync() raises)."""
        self._check(self.lib.mrml_hip_set_wait_limit(self.ctx, polls))

    def device_info(self) -> dict:
        info = DeviceInfo()
        self._check(self.lib.mrml_hip_device_info_get(self.ctx, ctypes.byref(info)))
        return {f: (getattr(info, f).decode() if f == "name" else getattr(info, f)) for f, _ in info._fields_}

    def memory_info(self) -> tuple[int, int]:
        f, t = ctypes.c_uint64(), ctypes.c_uint64()
        self._check(self.lib.mrml_hip_memory_info(self.ctx, ctypes.byref(f), ctypes.byref(t)))
        return int(f.value), int(t.value)

    @property
    def stream(self) -> int:
        return int(self.lib.mrml_hip_stream(self.ctx) or 0)

    def reserve_workspace(self, nbytes: int) -> None:
        self._check(self.lib.mrml_hip_reserve_workspace(self.ctx, nbytes))

    def workspace_bytes(self) -> int:
        n = ctypes.c_size_t()
        self._check(self.lib.mrml_hip_workspace_bytes(self.ctx, ctypes.byref(n)))
        return int(n.value)

    def zero(self, buf, nbytes: int | None = None) -> None:
        self._check(self.lib.mrml_hip_zero_async(self.ctx, _ptr(buf), buf.nbytes if nbytes is None else nbytes))

    # ---- graphs (CudaDevice::capture / launch_graph, cuda.rs:1957-2003) -------
    def capture(self, fn) -> "HipGraph":
        """Record the ops `fn()` issues on this device into a replayable graph."""
        self._check(self.lib.mrml_hip_graph_begin(self.ctx))
        try:
            fn()
        except BaseException:
            g = ctypes.c_void_p()
            self.lib.mrml_hip_graph_end(self.ctx, ctypes.byref(g))
            if g.value:
                self.lib.mrml_hip_graph_destroy(self.ctx, g.value)
            raise
        g = ctypes.c_void_p()
        self._check(self.lib.mrml_hip_graph_end(self.ctx, ctypes.byref(g)))
        return HipGraph(self, g.value)

    def copy_kernel(self, dst, src, nbytes: int) -> None:
        self._check(self.lib.mrml_hip_copy_kernel(self.ctx, _ptr(dst), _ptr(src), nbytes))

    def read_kernel(self, src, nbytes: int, sink) -> None:
        """Streaming read of nbytes of src (the read-only floor of a matvec's weight stream)."""
        self._check(self.lib.mrml_hip_read_kernel(self.ctx, _ptr(src), nbytes, _ptr(sink)))

    # ---- ops (names follow CudaDevice) -----------------------------------------
    def quantize_q8_0(self, x, q8_gguf=None, pack=None, n: int | None = None) -> None:
        n = x.shape[0] if n is None else n
        self._check(self.lib.mrml_hip_quantize_q8_0(self.ctx, _ptr(x), _ptr(q8_gguf), _ptr(pack), n))

    def q8_0_pack_bytes(self, n: int) -> int:
        return int(self.lib.mrml_hip_q8_0_pack_bytes(n))

    def gemv_q4_0(self, w, x, y, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols))

    def gemv_q4_0_q8(self, w, xpack, y, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_q8(self.ctx, _ptr(w), _ptr(xpack), _ptr(y), rows, cols))

    def gemv_q4_0_q8_relaxed(self, w, xpack, y, rows: int, cols: int) -> None:
        """The tolerance path's matvec (tree-order row sums; mrml_hip_gemv_q4_0_q8_relaxed)."""
        self._check(self.lib.mrml_hip_gemv_q4_0_q8_relaxed(self.ctx, _ptr(w), _ptr(xpack), _ptr(y), rows, cols))

    def gemm_q4_0(self, w, x, y, rows: int, cols: int, batch: int) -> None:
        self._check(self.lib.mrml_hip_gemm_q4_0(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols, batch))

    def gemm_q4_0_relaxed(self, w, x, y, rows: int, cols: int, batch: int) -> None:
        """gemm_q4_0 with the one-FMA f32 fold (within 1e-5 of the exact product)."""
        self._check(self.lib.mrml_hip_gemm_q4_0_relaxed(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols, batch))

    def gemm_q4_0_qkv(self, wq, wk, wv, x, y, q_rows: int, kv_rows: int, cols: int, batch: int) -> None:
        self._check(self.lib.mrml_hip_gemm_q4_0_qkv(self.ctx, _ptr(wq), _ptr(wk), _ptr(wv), _ptr(x), _ptr(y),
                                                    q_rows, kv_rows, cols, batch))

    def gemm_q4_0_geglu(self, w_gate, w_up, x, act, rows: int, cols: int, batch: int) -> None:
        self._check(self.lib.mrml_hip_gemm_q4_0_geglu(self.ctx, _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(act),
                                                      rows, cols, batch))

    def rms_norm_batch(self, x, w, out, dim: int, batch: int, eps: float) -> None:
        self._check(self.lib.mrml_hip_rms_norm_batch(self.ctx, _ptr(x), _ptr(w), _ptr(out), dim, batch, eps))

    def gemm_q4_0_noalloc(self, w, x, y, rows: int, cols: int, batch: int) -> None:
        """gemm_q4_0 without any allocation: the activations' GEMM pack goes to
        the library's fixed per-GPU device scratch (calls overlapping on one
        GPU race)."""
        self._check(self.lib.mrml_hip_gemm_q4_0_noalloc(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols, batch))

    def gemm_q4_0_noalloc_max_pack_bytes(self) -> int:
        return int(self.lib.mrml_hip_gemm_q4_0_noalloc_max_pack_bytes())

    def gemm_q4_0_q8(self, w, xpack, y, rows: int, cols: int, batch: int) -> None:
        self._check(self.lib.mrml_hip_gemm_q4_0_q8(self.ctx, _ptr(w), _ptr(xpack), _ptr(y), rows, cols, batch))

    def gemm_pack_bytes(self, cols: int, batch: int) -> int:
        return int(self.lib.mrml_hip_gemm_pack_bytes(cols, batch))

    def quantize_q8_0_gemm(self, x, gpack, cols: int, batch: int) -> None:
        self._check(self.lib.mrml_hip_quantize_q8_0_gemm(self.ctx, _ptr(x), _ptr(gpack), cols, batch))

    def gemm_q4_0_gpack(self, w, gpack, y, rows: int, cols: int, batch: int) -> None:
        self._check(self.lib.mrml_hip_gemm_q4_0_gpack(self.ctx, _ptr(w), _ptr(gpack), _ptr(y), rows, cols, batch))

    def gemv_q4_0_gguf(self, w, x, y, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_gguf(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols))

    def gemv_q4_0_geglu(self, w_gate, w_up, x, act, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_geglu(self.ctx, _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(act),
                                                      rows, cols))

    def gemv_q4_0_qkv(self, wq, wk, wv, x, y, q_rows: int, kv_rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_qkv(self.ctx, _ptr(wq), _ptr(wk), _ptr(wv), _ptr(x), _ptr(y),
                                                    q_rows, kv_rows, cols))

    def gemv_q4_0_geglu_q8(self, w_gate, w_up, xpack, act, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_geglu_q8(self.ctx, _ptr(w_gate), _ptr(w_up), _ptr(xpack),
                                                         _ptr(act), rows, cols))

    def gemv_q4_0_geglu_pack(self, w_gate, w_up, x, act, act_pack, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_geglu_pack(self.ctx, _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(act),
                                                           _ptr(act_pack), rows, cols))

    def ffn_split_geglu(self, w_gate, w_up, x, act, act_pack, dim: int, ffn: int, w_down_next=None) -> None:
        """The split FFN's GeGLU launch: f32 act and the pack's whole blocks (mrml_hip_ffn_split_geglu);
        w_down_next (optional): the down projection launched next, read ahead into the caches."""
        self._check(self.lib.mrml_hip_ffn_split_geglu(self.ctx, _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(act),
                                                      _ptr(act_pack), _ptr(w_down_next), dim, ffn))

    def ffn_split_down(self, w_down, act_pack, act, y, dim: int, ffn: int) -> None:
        """The split FFN's down launch (mrml_hip_ffn_split_down)."""
        self._check(self.lib.mrml_hip_ffn_split_down(self.ctx, _ptr(w_down), _ptr(act_pack), _ptr(act), _ptr(y),
                                                     dim, ffn))

    def ffn_geglu_q4_0(self, w_gate, w_up, w_down, x, act, y, dim: int, ffn: int) -> None:
        self._check(self.lib.mrml_hip_ffn_geglu_q4_0(self.ctx, _ptr(w_gate), _ptr(w_up), _ptr(w_down), _ptr(x),
                                                     _ptr(act), _ptr(y), dim, ffn))

    def gemv_q4_0_qkv_q8(self, wq, wk, wv, xpack, y, q_rows: int, kv_rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_0_qkv_q8(self.ctx, _ptr(wq), _ptr(wk), _ptr(wv), _ptr(xpack),
                                                       _ptr(y), q_rows, kv_rows, cols))

    def gemv_q8_0(self, w, x, y, rows: int, cols: int, softcap: bool = False) -> None:
        self._check(self.lib.mrml_hip_gemv_q8_0(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols, int(softcap)))

    def gemv_q4_k(self, w, x, y, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_k(self.ctx, _ptr(w), _ptr(x), _ptr(y), rows, cols))

    def gemv_q8_0_q8(self, w, xpack, y, rows: int, cols: int, softcap: bool = False) -> None:
        self._check(self.lib.mrml_hip_gemv_q8_0_q8(self.ctx, _ptr(w), _ptr(xpack), _ptr(y), rows, cols,
                                                   int(softcap)))

    def gemv_q4_k_q8(self, w, xpack, y, rows: int, cols: int) -> None:
        self._check(self.lib.mrml_hip_gemv_q4_k_q8(self.ctx, _ptr(w), _ptr(xpack), _ptr(y), rows, cols))

    def argmax_f32(self, x, n: int, out) -> None:
        self._check(self.lib.mrml_hip_argmax_f32(self.ctx, _ptr(x), n, _ptr(out)))

    def vocab_topk(self, logits, valid, recent, scores, ids, vocab_size: int, n_recent: int, generated_count: int,
                   k: int, partitions: int) -> None:
        """CudaDevice::vocab_topk (cuda.rs:3052-3111): each partition's k best (score, id)."""
        self._check(self.lib.mrml_hip_vocab_topk(self.ctx, _ptr(logits), _ptr(valid), _ptr(recent), _ptr(scores),
                                                 _ptr(ids), vocab_size, n_recent, generated_count, k, partitions))

    def vocab_select(self, logits, vocab: int, valid=None, recent=None, n_recent: int = 0, generated_count: int = 0,
                     scoring: int = 0, temperature: float = 0.0, pos: int = 0, k: int = 40, token=None,
                     scores=None, ids=None) -> None:
        """step_generation's next-token pick (model.rs:2842-2907) on the device; scoring
        SCORE_CPU (softcap, -3.5 once) or SCORE_DEVICE (-1.8 per occurrence)."""
        self._check(self.lib.mrml_hip_vocab_select(self.ctx, _ptr(logits), vocab, _ptr(valid), _ptr(recent),
                                                   n_recent, generated_count, scoring, temperature, pos, k,
                                                   _ptr(token), _ptr(scores), _ptr(ids)))

    # ---- the rest of the token step ----------------------------------------------
    def rms_norm(self, x, w, out, dim: int, eps: float, pack=None) -> None:
        """CudaDevice::rms_norm (cuda.rs:2102-2180); `pack` also takes the Q8_0 pack."""
        self._check(self.lib.mrml_hip_rms_norm(self.ctx, _ptr(x), _ptr(w), _ptr(out), _ptr(pack), dim, eps))

    def residual_rms_norm(self, t, w_post, h, w_next, xn, dim: int, eps: float, pack=None) -> None:
        self._check(self.lib.mrml_hip_residual_rms_norm(self.ctx, _ptr(t), _ptr(w_post), _ptr(h), _ptr(w_next),
                                                        _ptr(xn), _ptr(pack), dim, eps))

    def embedding(self, table, qtype: int, token: int, out, dim: int, vocab: int, scale: float,
                  d_token=None) -> None:
        """CudaDevice::embedding_q8_0 (cuda.rs:2625-2656) for Q4_0 or Q8_0 tables."""
        self._check(self.lib.mrml_hip_embedding(self.ctx, _ptr(table), qtype, token, _ptr(d_token), _ptr(out),
                                                dim, vocab, scale))

    def rope_table(self, table, n_pos: int, head_dim: int, freq_base: float, freq_scale: float = 1.0) -> None:
        """Fill a (cos, sin) table for positions < n_pos with the host C library."""
        self._check(self.lib.mrml_hip_rope_table(self.ctx, _ptr(table), n_pos, head_dim, freq_base, freq_scale))

    def rope_kv_append_f16(self, qkv, k_cache, v_cache, pos: int, n_heads: int, n_kv_heads: int, head_dim: int,
                           freq_base: float, capacity: int, freq_scale: float = 1.0, d_pos=None, table=None,
                           n_table: int = 0) -> None:
        """CudaDevice::qkv_postprocess (cuda.rs:2438-2476) without head norms."""
        self._check(self.lib.mrml_hip_rope_kv_append_f16(self.ctx, _ptr(qkv), _ptr(k_cache), _ptr(v_cache), pos,
                                                         _ptr(d_pos), n_heads, n_kv_heads, head_dim, freq_base,
                                                         freq_scale, capacity, _ptr(table), n_table))

    def qkv_postprocess_batch(self, qkv, k_cache, v_cache, start_pos: int, cache_start: int, n_heads: int,
                              n_kv_heads: int, head_dim: int, freq_base: float, batch: int, capacity: int,
                              k_format: int = 0, v_format: int = 0, freq_scale: float = 1.0, table=None,
                              n_table: int = 0) -> None:
        """CudaDevice::qkv_postprocess_batch (cuda.rs:2478-2519) without head norms, the reference's argument
        order (mrml_hip_rope_kv_append_f16_batch)."""
        self._check(self.lib.mrml_hip_rope_kv_append_f16_batch(
            self.ctx, _ptr(qkv), _ptr(k_cache), _ptr(v_cache), start_pos, cache_start, batch, n_heads, n_kv_heads,
            head_dim, freq_base, freq_scale, capacity, k_format, v_format, _ptr(table), n_table))

    def rope_256k(self, vec, pos: int, head_dim: int, n_heads: int, freq_base: float, freq_scale: float = 1.0,
                  table=None, n_table: int = 0) -> None:
        """CudaDevice::rope_256k (cuda.rs:2248-2285): RoPE of n_heads heads of vec in place."""
        self._check(self.lib.mrml_hip_rope(self.ctx, _ptr(vec), pos, head_dim, n_heads, freq_base, freq_scale,
                                           _ptr(table), n_table))

    def geglu(self, gate, up, out, n: int) -> None:
        """CudaDevice::geglu (cuda.rs:2215-2246): out = gelu_tanh(gate) * up."""
        self._check(self.lib.mrml_hip_geglu(self.ctx, _ptr(gate), _ptr(up), _ptr(out), n))

    def swiglu(self, gate, up, out, n: int) -> None:
        """CudaDevice::swiglu (cuda.rs:2182-2213): out = silu(gate) * up."""
        self._check(self.lib.mrml_hip_swiglu(self.ctx, _ptr(gate), _ptr(up), _ptr(out), n))

    def add(self, a, b, out, n: int) -> None:
        """CudaDevice::add (cuda.rs:2579-2593): out = a + b."""
        self._check(self.lib.mrml_hip_add(self.ctx, _ptr(a), _ptr(b), _ptr(out), n))

    def attention_prefill(self, q, k_cache, v_cache, out, cache_start: int, batch: int, n_heads: int,
                          n_kv_heads: int, head_dim: int, scale: float, sliding_window, capacity: int,
                          k_format: int = 0, v_format: int = 0, q_stride: int | None = None) -> None:
        """CudaDevice::attention_prefill (cuda.rs:2727-2770): q_stride defaults to the reference's
        q.len() / batch (q a HipBuffer of f32)."""
        if q_stride is None:
            q_stride = (q.nbytes // 4) // batch
        self._check(self.lib.mrml_hip_attention_prefill(
            self.ctx, _ptr(q), q_stride, _ptr(k_cache), _ptr(v_cache), _ptr(out), cache_start, batch, n_heads,
            n_kv_heads, head_dim, scale, -1 if sliding_window is None else int(sliding_window), capacity, k_format,
            v_format))

    def attention_causal(self, q, k_cache, v_cache, out, n_past: int, n_heads: int, n_kv_heads: int,
                         head_dim: int, scale: float, capacity: int, pack=None, d_pos=None) -> None:
        """CudaDevice::attention_causal (cuda.rs:2658-2697) for one token, f16 cache."""
        self._check(self.lib.mrml_hip_attn_decode_f16(self.ctx, _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                                      _ptr(pack), n_past, _ptr(d_pos), n_heads, n_kv_heads,
                                                      head_dim, scale, capacity))


    def attention_causal_split(self, q, k_cache, v_cache, out, n_past: int, n_heads: int, n_kv_heads: int,
                               head_dim: int, scale: float, capacity: int, pack=None, d_pos=None) -> None:
        """attention_causal split over tiles of the window (the FAST numerics)."""
        self._check(self.lib.mrml_hip_attn_decode_f16_split(self.ctx, _ptr(q), _ptr(k_cache), _ptr(v_cache),
                                                            _ptr(out), _ptr(pack), n_past, _ptr(d_pos), n_heads,
                                                            n_kv_heads, head_dim, scale, capacity))

    def attention_causal_ref(self, q, k_cache, v_cache, out, n_past: int, n_heads: int, n_kv_heads: int,
                             head_dim: int, scale: float, sliding_window, capacity: int, k_format: int = 0,
                             v_format: int = 0, split: bool = False) -> None:
        """CudaDevice::attention_causal with its own arguments (cuda.rs:2658-2697): sliding_window None or an
        int (mrml_hip_attention_causal, or its split form)."""
        fn = self.lib.mrml_hip_attention_causal_split if split else self.lib.mrml_hip_attention_causal
        self._check(fn(self.ctx, _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), n_past, n_heads, n_kv_heads,
                       head_dim, scale, -1 if sliding_window is None else int(sliding_window), capacity, k_format,
                       v_format))


class Gemma2Model:
    """A Gemma-2-shape decoder bound to device weights (mrml_hip_gemma2_*).

    ``layers`` is a list of dicts with the keys of GEMMA2_LAYER_TENSORS (backend
    Q4_0 buffers) and GEMMA2_LAYER_NORMS (f32 buffers).  Weights are not copied;
    keep them alive while the model is used.
    """

    def __init__(self, dev: HipDevice, cfg: Gemma2Config, tok_embd, output_norm, layers):
        self.dev = dev
        self.cfg = cfg
        arr = (Gemma2Layer * cfg.n_layers)()
        for i, L in enumerate(layers):
            for name in GEMMA2_LAYER_TENSORS + GEMMA2_LAYER_NORMS:
                setattr(arr[i], name, _ptr(L[name]))
        h = ctypes.c_void_p()
        dev._check(dev.lib.mrml_hip_gemma2_create(dev.ctx, ctypes.byref(cfg), _ptr(tok_embd), _ptr(output_norm),
                                                  arr, ctypes.byref(h)))
        self.handle = h.value

    @classmethod
    def from_host(cls, dev: HipDevice, model: dict, numerics: int = NUMERICS_EXACT) -> "Gemma2Model":
        """Upload a model held as GGUF block bytes (the dict of synth.gemma2_model)
        and convert every matrix to the backend layout; the model keeps the
        device buffers alive.  numerics: NUMERICS_EXACT (bit-identical to the
        CPU step) or NUMERICS_FAST (tree-order norm sums, split-K attention)."""
        c = model["cfg"]
        cfg = Gemma2Config(c["n_layers"], c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ffn_dim"],
                           c["vocab"], c["ctx_len"], c["rope_base"], c["eps"], c["attn_scale"],
                           Q8_0 if model["tie_q8"] else Q4_0, numerics, c.get("sliding_window", 0),
                           c.get("swa_period", 0))
        qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
        shapes = {"wq": (qd, c["dim"]), "wk": (kvd, c["dim"]), "wv": (kvd, c["dim"]), "wo": (c["dim"], qd),
                  "w_gate": (c["ffn_dim"], c["dim"]), "w_up": (c["ffn_dim"], c["dim"]),
                  "w_down": (c["dim"], c["ffn_dim"])}
        keep = []
        layers = []
        for L in model["layers"]:
            d = {}
            for name in GEMMA2_LAYER_TENSORS:
                d[name] = HipBuffer.from_gguf(dev, L[name], Q4_0, *shapes[name])
            for name in GEMMA2_LAYER_NORMS:
                d[name] = HipBuffer.from_host(dev, L[name])
            layers.append(d)
            keep.extend(d.values())
        table = HipBuffer.from_gguf(dev, model["tok_embd"], cfg.tie_type, c["vocab"], c["dim"])
        out_norm = HipBuffer.from_host(dev, model["output_norm"])
        self = cls(dev, cfg, table, out_norm, layers)
        self.buffers = keep + [table, out_norm]
        return self

    def cache_elems(self) -> int:
        """f16 elements of one of the two KV caches."""
        c = self.cfg
        return c.n_layers * c.ctx_len * c.n_kv_heads * c.head_dim

    def step(self, state, k_cache, v_cache, logits=None, argmax=None, hist=None, hist_cap: int = 0,
             prompt=None, prompt_len: int = 0) -> None:
        """Enqueue one token step (model.rs forward_token + greedy pick); see mrml_hip_gemma2_step."""
        self.dev._check(self.dev.lib.mrml_hip_gemma2_step(self.dev.ctx, self.handle, _ptr(state), _ptr(k_cache),
                                                          _ptr(v_cache), _ptr(logits), _ptr(argmax), _ptr(hist),
                                                          hist_cap, _ptr(prompt), prompt_len))

    def prefill(self, tokens, n_tokens: int, pos0: int, k_cache, v_cache, logits=None, argmax=None) -> None:
        """Enqueue the prefill of n_tokens device tokens from position pos0 (prefill_cuda,
        model.rs:2395-2638); see mrml_hip_gemma2_prefill."""
        self.dev._check(self.dev.lib.mrml_hip_gemma2_prefill(self.dev.ctx, self.handle, _ptr(tokens), n_tokens, pos0,
                                                             _ptr(k_cache), _ptr(v_cache), _ptr(logits),
                                                             _ptr(argmax)))

    def reserve_prefill(self) -> None:
        """Allocate the prefill's chunk buffers now, so a later prefill can be captured."""
        self.dev._check(self.dev.lib.mrml_hip_gemma2_reserve_prefill(self.dev.ctx, self.handle))

    def set_sampler(self, temperature: float = 0.0, top_k: int = 40, valid=None) -> None:
        """Pick with the CPU path's scoring and draw (mrml_hip_gemma2_set_sampler)."""
        sp = Sampler(_ptr(valid), temperature, top_k)
        self.dev._check(self.dev.lib.mrml_hip_gemma2_set_sampler(self.dev.ctx, self.handle, ctypes.byref(sp)))

    def clear_sampler(self) -> None:
        """Back to the plain argmax."""
        self.dev._check(self.dev.lib.mrml_hip_gemma2_set_sampler(self.dev.ctx, self.handle, None))

    def activations(self) -> tuple[int, int]:
        h, lg = ctypes.c_void_p(), ctypes.c_void_p()
        self.dev._check(self.dev.lib.mrml_hip_gemma2_activations(self.dev.ctx, self.handle, ctypes.byref(h),
                                                                 ctypes.byref(lg)))
        return int(h.value), int(lg.value)

    def close(self) -> None:
        if self.handle and self.dev.ctx:
            self.dev.lib.mrml_hip_gemma2_destroy(self.dev.ctx, self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipGraph:
    """An instantiated graph (CudaGraphExec, cuda.rs:1841-1858)."""

    def __init__(self, dev: HipDevice, exec_ptr: int):
        self.dev = dev
        self.exec = exec_ptr

    def launch(self) -> None:
        self.dev._check(self.dev.lib.mrml_hip_graph_launch(self.dev.ctx, self.exec))

    def close(self) -> None:
        if self.exec and self.dev.ctx:
            self.dev.lib.mrml_hip_graph_destroy(self.dev.ctx, self.exec)
        self.exec = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = [
    "HipDevice", "HipBuffer", "HipGraph", "HipError", "load_library", "device_count", "exported_symbols",
    "Q4_0", "Q8_0", "Q4_K", "BLOCK_BYTES", "BLOCK_WEIGHTS", "LIB_PATH",
]
