"""Build recipe for the native parts of velo-mind_amd.

  libvmhip.so     HIP kernels + C ABI (include/vm_hip.h), hipcc, gfx950
  libvelomind.so  C++ VeloMind host layer with the DeviceType::HIP backend
                  (velo-mind_amd/core), linked against libvmhip.so

Run as ``python velo-mind_amd/build.py`` or through
``__graft_entry__.build()``.  Objects are rebuilt every time (the driver's
"does it build" check); compile units run in parallel.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shlex
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
CORE = os.path.join(PKG, "core")
OUT_DIR = os.path.join(PKG, "velomind_hip")
BUILD_DIR = os.path.join(PKG, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed-FP32 VALU forms stay disabled on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Bit-exact packing needs IEEE division and no fast-math rewriting.
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math",
    "-Wall", "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
]
# Phase timestamps in the one-launch decode step (profiling builds only).
if os.environ.get("VELOMIND_DECODE_TRACE") == "1":
    HIP_FLAGS.append("-DVM_DECODE_TRACE")
# Phase timestamps in the decode GEMV (profiling builds only).
if os.environ.get("VELOMIND_GEMV_TRACE") == "1":
    HIP_FLAGS.append("-DVM_GEMV_TRACE")
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-pthread", "-Wall", "-Wextra",
             f"-I{os.path.join(CORE, 'include')}", f"-I{os.path.join(CORE, 'src')}",
             f"-I{os.path.join(ROOT, 'include')}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("build step failed: " + " ".join(shlex.quote(c) for c in cmd))
    noise = "is not a recognized feature for this target"
    for line in (proc.stdout + proc.stderr).splitlines():
        if line.strip() and noise not in line:
            sys.stderr.write(line + "\n")


# Per-file additions.  qmm_gemm.hip: MFMA accumulators in ordinary VGPRs
# (with AGPR accumulators the register allocator rotates the loop-carried
# tiles through copies every iteration of the wide kernel's K loop).
FILE_FLAGS = {"qmm_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def build_vmhip(jobs: int = 8) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = []
    cmds = []
    for src in sources:
        obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    out = os.path.join(OUT_DIR, "libvmhip.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          "-Wl,-soname,libvmhip.so"])
    os.replace(tmp, out)
    return out


def build_core(jobs: int = 8) -> str | None:
    sources = sorted(glob.glob(os.path.join(CORE, "src", "**", "*.cpp"), recursive=True))
    if not sources:
        return None
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs, cmds = [], []
    for src in sources:
        rel = os.path.relpath(src, CORE).replace(os.sep, "_")
        obj = os.path.join(BUILD_DIR, rel + ".o")
        objs.append(obj)
        cmds.append([CXX, *CXX_FLAGS, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    out = os.path.join(OUT_DIR, "libvelomind.so")
    tmp = out + ".tmp"
    _run([CXX, "-shared", "-fPIC", "-pthread", *objs, "-o", tmp, f"-L{OUT_DIR}", "-lvmhip",
          "-Wl,-rpath,$ORIGIN", "-Wl,-soname,libvelomind.so"])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_vmhip()
    build_core()


if __name__ == "__main__":
    build_all()
    print("built:", ", ".join(sorted(os.path.basename(p) for p in glob.glob(os.path.join(OUT_DIR, "*.so")))))
