"""Runs the C++ restatement of the reference's unit tests (tests/cpp/tensor_tests.cpp)
against the gfx950 library through the host mirror, in one child process."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "tensor_tests.bin")


@pytest.mark.gpu
def test_reference_unit_tests_in_cpp():
    assert os.path.exists(BIN), "build first: python -m rustllm_amd.build"
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    print(res.stdout[-4000:])
    assert res.returncode == 0, res.stdout[-4000:] + res.stderr[-2000:]
    assert " 0 failed" in res.stdout


def test_cpp_mirror_is_built_and_links_the_library():
    host = os.path.join(ROOT, "rustllm_amd", "librustllm_tensor.so")
    assert os.path.exists(host) and os.path.exists(BIN)
    out = subprocess.run(["ldd", BIN], capture_output=True, text=True).stdout
    assert "librustllm_tensor.so" in out and "librustllm_hip.so" in out
    assert "not found" not in out
