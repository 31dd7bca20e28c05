"""Shared test setup: the `gpu` marker, the backend package and the oracle.

The backend package lives in the folder ``qt_llama.cpp_amd`` (not an importable
identifier), so it is loaded by path under the module name ``qt_llama_cpp_amd``.
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_backend():
    name = "qt_llama_cpp_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "qt_llama.cpp_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


@pytest.fixture(scope="session")
def backend():
    return load_backend()


@pytest.fixture(scope="session")
def orc():
    from oracle import orc as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def synth():
    load_backend()
    import qt_llama_cpp_amd.synth as s
    return s


@pytest.fixture(scope="session")
def gguf():
    load_backend()
    import qt_llama_cpp_amd.gguf as g
    return g


@pytest.fixture(scope="session")
def dev(backend):
    """One context for the whole GPU session (GPU tests run in one process)."""
    if backend.device_count() < 1:
        pytest.fail("no GPU visible: GPU tests must run on the MI355X box")
    d = backend.HipDevice.new(0)
    yield d
    d.close()
