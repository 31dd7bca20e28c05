"""C-ABI checks that need no GPU: the library loads, exports every function
include/mrml_hip.h declares, and fails cleanly where no gfx950 device exists."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "mrml_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mrml_(?:hip|gguf)_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_surface():
    names = declared_functions()
    for must in ("mrml_hip_create", "mrml_hip_gemv_q4_0", "mrml_hip_gemv_q4_0_geglu", "mrml_hip_gemv_q8_0",
                 "mrml_hip_gemv_q4_k", "mrml_hip_gemm_q4_0", "mrml_hip_gemm_q4_0_q8", "mrml_hip_gemm_q4_0_gpack", "mrml_hip_quantize_q8_0_gemm", "mrml_hip_quantize_q8_0", "mrml_hip_argmax_f32", "mrml_hip_repack_q4_0"):
        assert must in names


def test_library_exports_every_declared_symbol(backend):
    lib = backend.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python mirror binds exactly the declared surface
    import qt_llama_cpp_amd.gguf as gguf
    assert sorted(backend.exported_symbols() + gguf.exported_symbols()) == declared_functions()


def test_library_is_gfx950_only():
    so = (ROOT / "qt_llama.cpp_amd" / "lib" / "libmrml_hip.so").read_bytes()
    assert b"gfx950" in so
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in so


def test_status_strings_and_null_context(backend):
    lib = backend.load_library()
    assert lib.mrml_hip_status_string(0) == b"ok"
    assert lib.mrml_hip_status_string(-5) == b"no gfx950 device"
    assert lib.mrml_hip_last_error(None) == b"null context"
    assert lib.mrml_hip_sync(None) == -1
    assert lib.mrml_hip_gemv_q4_0(None, None, None, None, 1, 32) == -1
    assert lib.mrml_hip_q8_0_pack_bytes(2304) == 72 * 40
    assert lib.mrml_hip_gemma2_prefill(None, None, None, 1, 0, None, None, None, None) == -1


def test_no_device_fails_cleanly(backend):
    if backend.device_count() > 0:
        pytest.skip("a device is visible; covered by the GPU tests")
    ctx = ctypes.c_void_p()
    rc = backend.load_library().mrml_hip_create(0, ctypes.byref(ctx))
    assert rc == -5 and not ctx.value
    with pytest.raises(backend.HipError):
        backend.HipDevice.new(0)
