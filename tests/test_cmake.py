"""The in-tree CMake build (CPU only: configures and compiles, runs no GPU code).

* a CPU-only configure (XKSV_ENABLE_HIP off, the default, as the reference's
  XKSV_ENABLE_CUDA, CMakeLists.txt:35-40) builds the oracle the CPU tests use;
* -DXKSV_ENABLE_HIP=ON also builds libxksv_hip.so for gfx950, exporting the
  same symbols as the Makefile's library and loading through the binding.
"""
from __future__ import annotations

import shutil
import subprocess

import pytest

import xksv_hip
from conftest import PKG, ROOT
from oracle_lib import Oracle, raw_bytes
import xksv_synth as syn

pytestmark = pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not installed")


def _build(tmp_path, hip: bool):
    build = tmp_path / ("hip" if hip else "cpu")
    gen = ["-G", "Ninja"] if shutil.which("ninja") else []
    subprocess.run(["cmake", "-S", str(ROOT), "-B", str(build), *gen, f"-DXKSV_ENABLE_HIP={'ON' if hip else 'OFF'}"],
                   check=True, capture_output=True)
    subprocess.run(["cmake", "--build", str(build), "-j", "8"], check=True, capture_output=True)
    return build


def _exports(path) -> set:
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], check=True, capture_output=True, text=True)
    return {ln.split()[-1] for ln in out.stdout.splitlines() if " T " in ln and ln.split()[-1].startswith("xksv_")}


def test_cpu_only_configure_builds_the_oracle(tmp_path):
    build = _build(tmp_path, hip=False)
    assert not (build / "libxksv_hip.so").exists()
    oracle = Oracle(build / "liboracle.so")
    w = syn.normal_bf16(3, (16, 96))
    rc, blob = oracle.pack_parallel(raw_bytes(w), 16, 96)
    assert rc == 0 and oracle.unpack_parallel(blob) == (0, raw_bytes(w))


def test_hip_switch_builds_the_same_library(tmp_path):
    build = _build(tmp_path, hip=True)
    lib = build / "libxksv_hip.so"
    assert lib.exists()
    made = PKG / "libxksv_hip.so"
    assert _exports(lib) == _exports(made) == set(xksv_hip.EXPORTS)
    h = xksv_hip.Library(lib)
    assert h.lib.xksv_hip_version() >= 1
