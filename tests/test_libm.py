"""The device's f32 tanh/exp/sin/cos (qt_llama.cpp_amd/csrc/libm_f32.h)
against the host C library the reference links (crates/mrml-math/src/lib.rs
binds glibc's tanhf/expf/sinf/cosf).  CPU only: the header is compiled for the host by g++ and every
97th float bit pattern (44M values, all exponent ranges) is compared bit for
bit.  An exhaustive pass over all 2^32 floats is `libm_check 1` (~20 s on 8
cores); it also reports 0 mismatches for tanhf and for the expf, sinf and
cosf forms this host's glibc selects."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

NATIVE = Path(__file__).resolve().parent / "native"


def host_expf_fused() -> bool:
    """glibc's x86-64 expf dispatch: the FMA build when the CPU has FMA and AVX2."""
    flags = set()
    for line in Path("/proc/cpuinfo").read_text().splitlines():
        if line.startswith("flags"):
            flags = set(line.split(":", 1)[1].split())
            break
    return "fma" in flags and "avx2" in flags


@pytest.fixture(scope="module")
def libm_check(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("libm") / "libm_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fopenmp", "-ffp-contract=off", str(NATIVE / "libm_check.cpp"),
                    "-o", str(exe), "-lm"], check=True)
    return exe


def test_tanhf_and_expf_match_host_libm(libm_check):
    out = subprocess.run([str(libm_check), "97"], check=True, capture_output=True, text=True).stdout
    fields = out.split()
    counts = {fields[i]: int(fields[i + 1]) for i in range(0, 16, 2)}
    assert counts["checked"] > 40_000_000
    assert counts["tanhf"] == 0, out
    form = "fused" if host_expf_fused() else "plain"
    for fn in ("expf", "sinf", "cosf"):
        assert counts[f"{fn}_{form}"] == 0, out


@pytest.fixture(scope="module")
def exact_sum_check(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("xsum") / "exact_sum_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", str(NATIVE / "exact_sum_check.cpp"),
                    "-o", str(exe)], check=True)
    return exe


@pytest.mark.parametrize("seed", [1, 2])
def test_exact_parallel_sum_matches_sequential_loop(exact_sum_check, seed):
    """qt_llama.cpp_amd/csrc/exact_sum.h: the run/event compression of the
    sequential f32 sum of non-negative terms (used for RMSNorm's sum of
    squares) reproduces the plain loop bit for bit on 20000 random vectors
    per seed: squares of normals over 16 decades, softmax terms, zeros and
    outliers, tie-rich multiples of 2^-12, constants, subnormals, wide ranges."""
    out = subprocess.run([str(exact_sum_check), "20000", str(seed)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout
    assert out.stdout.split()[1] == "0", out.stdout
