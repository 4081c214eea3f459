"""Build the native library `libferrograd_amd.so` in-tree with hipcc.

The library holds the C++ front end (IR, scheduler, rangeify, autograd),
the gfx950 lowering/codegen and the HIP runtime behind the C-ABI declared in
`include/`. Generated kernels are compiled at run time by hiprtc for gfx950.

Usage: python -m ferrograd_amd.build  (or `build()` from __graft_entry__).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libferrograd_amd.so")

SOURCES = ["ir.cpp", "device.cpp", "schedule.cpp", "tensor.cpp", "gpu_lower.cpp", "hip_device.cpp",
           "hip_runtime.cpp", "kernel_text.cpp", "hip_kernel.cpp", "dataset.cpp", "capi.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXXFLAGS = ["-O2", "-g0", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
            "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
LDFLAGS = ["-shared", "-L/opt/rocm/lib", "-lhiprtc", "-lamdhip64", "-lhsa-runtime64", "-ldl",
           "-Wl,-rpath,/opt/rocm/lib"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("command failed: " + " ".join(cmd))


def build_python_module() -> str:
    """The CPython extension `_fgc` (csrc/pymodule.c): the hot Tensor methods
    as one C call each, linked against the library next to it."""
    import sysconfig

    out = os.path.join(HERE, "_fgc" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out + ".tmp"
    _run(["gcc", "-O2", "-g0", "-fPIC", "-shared", "-Wall", "-I" + sysconfig.get_paths()["include"],
          "-I" + os.path.join(ROOT, "include"), os.path.join(CSRC, "pymodule.c"), "-o", tmp,
          "-L" + HERE, "-lferrograd_amd", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build(jobs: int = 8) -> str:
    """Compile every source (always), link the shared library and build the
    Python extension over it."""
    os.makedirs(OBJ, exist_ok=True)

    def compile_one(src: str) -> str:
        obj = os.path.join(OBJ, src.replace(".cpp", ".o"))
        _run([HIPCC, *CXXFLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, *objs, "-o", tmp, *LDFLAGS])
    os.replace(tmp, LIB)
    build_python_module()
    return LIB


if __name__ == "__main__":
    print(build())
