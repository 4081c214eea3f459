"""Build the test oracle `oracle/liboracle_cpu.so` (test infrastructure only).

The oracle links against the product library for the shared front end (IR,
scheduler, rangeify) and supplies the CPU device: the reference's
upcast/unroll/symbolic passes, a C emitter with the reference's statement
structure and accumulation order, and `clang -shared -O3 -march=native`
+ dlopen at run time.

The reference itself (Rust, /root/reference) cannot be compiled here: no
cargo/rustc and its crates need a network fetch, so there is no oracle/_ref.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "ferrograd_amd")
LIB = os.path.join(HERE, "liboracle_cpu.so")

CXX = os.environ.get("FG_ORACLE_CXX", "/opt/rocm/llvm/bin/clang++")


def build() -> str:
    cmd = [CXX, "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall",
           "-I" + os.path.join(PKG, "csrc"), "-I" + os.path.join(ROOT, "include"),
           os.path.join(HERE, "cpu_backend.cpp"), "-o", LIB + ".tmp",
           "-L" + PKG, "-lferrograd_amd", "-Wl,-rpath," + PKG, "-ldl"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("oracle build failed")
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build())
