"""Builds the hip backend's native libraries in-tree for gfx950.

  engine_amd/liblykuro_hip.so        kernels + the C ABI of include/lykuro_hip.h
                                     (hipcc, every .hip under csrc/kernels and
                                     the host-side packers under csrc/host)
  engine_amd/liblykuro_hip_model.so  the C++20 host model (QwenHipModel) and the
                                     model-level C ABI of include/lykuro_hip_model.h

Run as `python -m engine_amd.build` or through __graft_entry__.build(). It
always recompiles; objects go to engine_amd/_build/ (git-ignored).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

KERNEL_LIB = os.path.join(PKG, "liblykuro_hip.so")
MODEL_LIB = os.path.join(PKG, "liblykuro_hip_model.so")

# Every HIP translation unit: packed-FP32 instructions disabled (the compiler
# still uses packed fp16 and dot2), -O3, C++20.
HIP_FLAGS = ["-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function", "-I", INCLUDE,
             "-I", os.path.join(CSRC, "kernels"), "-I", os.path.join(CSRC, "host")]
# Host C++: ISO C++20, no FP contraction (quantizers must match the oracle's
# rounding bit for bit).
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra",
             "-Wno-unused-parameter", "-I", INCLUDE, "-I", os.path.join(CSRC, "host"),
             "-I", os.path.join(CSRC, "host", "iface"),
             "-I", os.path.join(ROCM, "include"), "-D__HIP_PLATFORM_AMD__"]

KERNEL_HOST_SOURCES = ["quant_pack.cpp"]  # C-ABI host helpers in the kernel lib


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{out}")
    return out


def _sources(sub, ext):
    d = os.path.join(CSRC, sub)
    return sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(ext))


def build(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    jobs = []
    for src in _sources("kernels", ".hip"):
        obj = os.path.join(OUT, os.path.basename(src) + ".o")
        jobs.append(("k", obj, [HIPCC, *HIP_FLAGS, "-c", src, "-o", obj]))
    host_srcs = _sources("host", ".cpp")
    for src in host_srcs:
        obj = os.path.join(OUT, os.path.basename(src) + ".o")
        kind = "k" if os.path.basename(src) in KERNEL_HOST_SOURCES else "m"
        jobs.append((kind, obj, ["g++", *CXX_FLAGS, "-c", src, "-o", obj]))
    workers = min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(workers) as ex:
        futs = {ex.submit(_run, cmd): (kind, obj) for kind, obj, cmd in jobs}
        for f in cf.as_completed(futs):
            out = f.result()
            if verbose and out.strip():
                print(out)
    kobjs = [o for k, o, _ in jobs if k == "k"]
    mobjs = [o for k, o, _ in jobs if k == "m"]
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", KERNEL_LIB + ".tmp",
          *kobjs, "-lpthread"])
    os.replace(KERNEL_LIB + ".tmp", KERNEL_LIB)
    if mobjs:
        _run(["g++", "-shared", "-fPIC", "-o", MODEL_LIB + ".tmp", *mobjs,
              "-L", PKG, "-llykuro_hip", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
              "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib"), "-lpthread"])
        os.replace(MODEL_LIB + ".tmp", MODEL_LIB)
    return KERNEL_LIB, MODEL_LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", KERNEL_LIB)
