"""Builds the gfx950 library in-tree with hipcc (no JIT, no cache outside the repo).

    python -m rustllm_amd.build          # rustllm_amd/librustllm_hip.so (+ host mirror, tests)

Every HIP source is compiled for gfx950 only, with packed-fp32 instructions
disabled and floating-point contraction off (the reference's expressions are
rounded operation by operation).  Objects go to rustllm_amd/_build/.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "librustllm_hip.so")
HOST_LIB = os.path.join(PKG, "librustllm_tensor.so")
CPP_TESTS = os.path.join(ROOT, "tests", "cpp", "tensor_tests.bin")
PROBE = os.path.join(PKG, "hbm_probe")

ARCH = "gfx950"
HIP_SOURCES = ["runtime.hip", "elementwise.hip", "movement.hip", "rmsnorm.hip", "softmax.hip",
               "rope.hip", "kvcache.hip", "embedding.hip", "attention.hip",
               "gqa.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def hip_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-I" + INCLUDE, "-I" + CSRC,
        "-ffp-contract=off", "-Wall",
        # Packed FP32 VALU ops stay off: hipcc would otherwise form them from float code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device feature above; that warning is noise.
    noise = ("packed-fp32-ops",)
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, *hip_flags(), "-c", os.path.join(CSRC, src), "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,--version-script=" + os.path.join(CSRC, "exports.map"), "-Wl,-z,defs"])
    os.replace(tmp, LIB)
    return LIB


def build_host() -> str | None:
    """C++ mirror of the reference's Tensor / ops / nn layer over the C ABI,
    plus its test program (the reference's own unit tests restated)."""
    src = os.path.join(HOST, "tensor.cpp")
    if not os.path.exists(src):
        return None
    cxx = shutil.which("g++") or "g++"
    flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-I" + INCLUDE, "-I" + HOST]
    rpath = "-Wl,-rpath,$ORIGIN"
    tmp = HOST_LIB + ".tmp"
    _run([cxx, *flags, "-shared", "-o", tmp, src, "-L" + PKG, "-lrustllm_hip", rpath])
    os.replace(tmp, HOST_LIB)
    test_src = os.path.join(ROOT, "tests", "cpp", "tensor_tests.cpp")
    if os.path.exists(test_src):
        tmp = CPP_TESTS + ".tmp"
        _run([cxx, *flags, "-o", tmp, test_src, "-L" + PKG, "-lrustllm_tensor", "-lrustllm_hip",
              "-Wl,-rpath,$ORIGIN/../../rustllm_amd"])
        os.replace(tmp, CPP_TESTS)
    return HOST_LIB


def build_probe() -> str:
    """The HBM streaming probe the bench compares each kernel with
    (rustllm_amd/hbm_probe, a plain executable: no library, no Python)."""
    tmp = PROBE + ".tmp"
    _run([hipcc(), *hip_flags(), "-o", tmp, os.path.join(CSRC, "hbm_probe.hip")])
    os.replace(tmp, PROBE)
    return PROBE


def build_all() -> None:
    build_hip()
    build_host()
    build_probe()


if __name__ == "__main__":
    build_all()
    print(LIB)
