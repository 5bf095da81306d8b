"""The library called from C++ as the reference engine calls libr4d (tests/cpp/engine_abi.cpp): through the C ABI of
include/r4d_mi355x.h, an illegal launch caught as std::runtime_error (third_party/libr4d/r4d.h:30-31), results
against the CPU oracle. The CPU part runs the checks that need no GPU; the GPU part all of them."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "engine_abi")


def _binary(build_if_missing):
    if not os.path.exists(BIN):
        if not build_if_missing:
            pytest.fail("tests/cpp/engine_abi is not built: run __graft_entry__.build()")
        subprocess.run(["sh", os.path.join(ROOT, "tests", "cpp", "build.sh")], check=True, timeout=300)
    return BIN


def test_engine_abi_cpu_contract():
    r = subprocess.run([_binary(True), "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout


@pytest.mark.gpu
def test_engine_abi_gpu():
    print("[gpu-step] engine_abi gpu", flush=True)
    r = subprocess.run([_binary(False), "gpu"], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout
