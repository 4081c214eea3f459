"""TEST INFRASTRUCTURE — the parity oracle for the MI355X path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (ferrograd_amd) never does. Two parts:

* `liboracle_cpu.so` (cpu_backend.cpp): registers a "cpu" device that restates
  the reference's clang backend (src/device/cpu.rs, src/codegen/clang.rs and
  the lane semantics of src/expand.rs + src/devectorize.rs), so any program
  built with ferrograd_amd runs on "cpu" exactly as the reference would run it.
  The tests pin it against the reference's known answers and against float64
  restatements of the benchmark configs.
* `cpu_bench.py`: the CPU baseline leg of bench.py (the device above, timed on
  one pinned core).

The reference (Rust) cannot be compiled here (no cargo/rustc, crates need a
network fetch), so there is no oracle/_ref build.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_cpu.so")

_loaded = None


def load() -> ctypes.CDLL:
    """Load the oracle library and register the "cpu" device (idempotent)."""
    global _loaded
    if _loaded is None:
        import ferrograd_amd  # the product library must be loaded first (shared registry)

        ferrograd_amd.lib()
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run python oracle/build.py)")
        l = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        l.fg_oracle_register.restype = ctypes.c_int
        if l.fg_oracle_register() != 0:
            raise RuntimeError("fg_oracle_register failed")
        _loaded = l
    return _loaded


def set_fuse(on: bool) -> bool:
    """Run the CPU device's realisations with the HIP device's fusions (True)
    or the reference partition (False, the default); returns the previous
    setting. Fused and unfused runs on this one device use the same lowering,
    so a fusion that preserves values gives the same bits."""
    l = load()
    l.fg_oracle_set_fuse.restype = ctypes.c_int
    l.fg_oracle_set_fuse.argtypes = [ctypes.c_int]
    return bool(l.fg_oracle_set_fuse(int(on)))


def plan_c(roots) -> list:
    """Oracle C source of every kernel the reference schedule makes for `roots`."""
    import json

    l = load()
    l.fg_oracle_plan_c.restype = ctypes.c_int
    l.fg_oracle_plan_c.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t,
                                   ctypes.POINTER(ctypes.c_size_t)]
    arr = (ctypes.c_void_p * max(1, len(roots)))(*[t._h for t in roots])
    need = ctypes.c_size_t()
    rc = l.fg_oracle_plan_c(arr, len(roots), None, 0, ctypes.byref(need))
    buf = ctypes.create_string_buffer(need.value + 1)
    l.fg_oracle_plan_c(arr, len(roots), buf, need.value + 1, ctypes.byref(need))
    out = json.loads(buf.value.decode())
    if rc != 0:
        raise RuntimeError(out.get("error", "fg_oracle_plan_c failed"))
    return out["kernels"]
