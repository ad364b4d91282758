"""Ahead-of-time build of the gfx950 library ``axis_amd/libaxis_hip.so`` (HIP kernels + C ABI)
and of the C++ host layer ``axis_amd/_axis*.so`` (named-axis tensors, autograd tape, optimizers)
on top of it.  Runs on a machine without a GPU: hipcc cross-compiles for gfx950.

    python -m axis_amd.build            # build both
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(CSRC, "host")
BUILD = os.path.join(HERE, "_build")
HIP_LIB = os.path.join(HERE, "libaxis_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 VALU ops are disabled for every kernel (-packed-fp32-ops).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# Sources whose arithmetic must round exactly as written (no fused multiply-add contraction).
EXACT = {"device.hip", "finish.hip", "unfold.hip", "grouped.hip", "elementwise.hip", "pool.hip", "loss.hip",
         "optim.hip", "conv_small.hip", "gemm_bf16.hip"}
# Matrix-core kernels keep their accumulators in ordinary VGPRs: the MFMA VGPR form avoids the
# per-iteration AGPR<->VGPR copies the default allocation inserts around the K loop.
EXTRA = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "conv_small.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "gemm_bf16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIP_SOURCES = ["device.hip", "finish.hip", "gemm.hip", "gemm_bf16.hip", "conv_small.hip", "unfold.hip", "grouped.hip", "elementwise.hip",
               "pool.hip", "loss.hip", "optim.hip"]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in line and "not a recognized feature" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _compile_hip(src):
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    flags = list(HIP_FLAGS)
    if src in EXACT:
        flags.append("-ffp-contract=off")
    flags += EXTRA.get(src, [])
    _run([HIPCC, *flags, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile_hip, HIP_SOURCES))
    tmp = HIP_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def host_sources():
    if not os.path.isdir(HOST):
        return []
    return sorted(os.path.join(HOST, f) for f in os.listdir(HOST) if f.endswith(".cpp"))


def build_host(jobs: int = 8) -> str | None:
    """The pybind11 module `_axis` (C++ host layer), linked against libaxis_hip.so."""
    sources = host_sources()
    if not sources:
        return None
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    target = os.path.join(HERE, "_axis" + suffix)
    py_inc = sysconfig.get_paths()["include"]
    flags = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", "-ffp-contract=off",
             f"-I{pybind11.get_include()}", f"-I{py_inc}", f"-I{os.path.join(ROOT, 'include')}",
             f"-I{HOST}", "-fvisibility=hidden"]
    os.makedirs(BUILD, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(BUILD, "host_" + os.path.basename(src).replace(".cpp", ".o"))
        _run(["g++", *flags, "-c", src, "-o", obj])
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = target + ".tmp"
    _run(["g++", "-shared", "-o", tmp, *objs, f"-L{HERE}", "-laxis_hip",
          "-Wl,-rpath,$ORIGIN", "-Wl,--no-as-needed"])
    os.replace(tmp, target)
    return target


def build(jobs: int = 8):
    lib = build_hip(jobs)
    host = build_host(jobs)
    return lib, host


if __name__ == "__main__":
    for path in build():
        if path:
            print(path)
    sys.exit(0)
