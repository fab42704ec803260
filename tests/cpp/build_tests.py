"""Builds the C++ test binary tests/cpp/velomind_tests (g++, links the
VeloMind host layer libvelomind.so and libvmhip.so; compiles the CPU oracle
in as the checker).

``--sanitize`` instead builds tests/cpp/velomind_tests_asan: the host layer's
sources compiled into the binary with AddressSanitizer and
UndefinedBehaviorSanitizer (g++ only, host code; the HIP kernels stay in
libvmhip.so).  Run it on the CPU tests: ``velomind_tests_asan "~[gpu]"``."""
from __future__ import annotations

import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PKG = os.path.join(ROOT, "velo-mind_amd")
LIBDIR = os.path.join(PKG, "velomind_hip")
OUT = os.path.join(HERE, "velomind_tests")


def build() -> str:
    objdir = os.path.join(PKG, "_build", "tests")
    os.makedirs(objdir, exist_ok=True)
    oracle_obj = os.path.join(objdir, "qmm_oracle.o")
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-c",
                    os.path.join(ROOT, "oracle", "qmm_oracle.c"), "-o", oracle_obj], check=True)
    srcs = sorted(glob.glob(os.path.join(HERE, "*.cpp")))
    cmd = ["g++", "-O1", "-std=c++20", "-Wall", "-pthread",
           f"-I{os.path.join(PKG, 'core', 'include')}", f"-I{os.path.join(PKG, 'core', 'src')}",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROOT, 'oracle')}", f"-I{HERE}",
           *srcs, oracle_obj, "-o", OUT + ".tmp", f"-L{LIBDIR}", "-lvelomind", "-lvmhip",
           f"-Wl,-rpath,{os.path.relpath(LIBDIR, HERE).join(['$ORIGIN/', ''])}", "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("C++ test build failed")
    os.replace(OUT + ".tmp", OUT)
    return OUT


def build_sanitized() -> str:
    objdir = os.path.join(PKG, "_build", "tests_asan")
    os.makedirs(objdir, exist_ok=True)
    san = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g"]
    oracle_obj = os.path.join(objdir, "qmm_oracle.o")
    subprocess.run(["gcc", "-O1", "-fPIC", "-std=c11", "-ffp-contract=off", *san, "-c",
                    os.path.join(ROOT, "oracle", "qmm_oracle.c"), "-o", oracle_obj], check=True)
    core = sorted(glob.glob(os.path.join(PKG, "core", "src", "**", "*.cpp"), recursive=True))
    srcs = sorted(glob.glob(os.path.join(HERE, "*.cpp")))
    out = OUT + "_asan"
    cmd = ["g++", "-O1", "-std=c++20", "-pthread", *san,
           f"-I{os.path.join(PKG, 'core', 'include')}", f"-I{os.path.join(PKG, 'core', 'src')}",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROOT, 'oracle')}", f"-I{HERE}",
           *core, *srcs, oracle_obj, "-o", out + ".tmp", f"-L{LIBDIR}", "-lvmhip",
           f"-Wl,-rpath,{os.path.relpath(LIBDIR, HERE).join(['$ORIGIN/', ''])}", "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("sanitized C++ test build failed")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build_sanitized() if "--sanitize" in sys.argv[1:] else build())
