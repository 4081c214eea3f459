"""TEST INFRASTRUCTURE — the parity oracle for the MI355X path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (ferrograd_amd) never does. Two parts:

* `liboracle_cpu.so` (cpu_backend.cpp): registers a "cpu" device that restates
  the reference's clang backend (src/device/cpu.rs, src/codegen/clang.rs and
  the lane semantics of src/expand.rs + src/devectorize.rs), so any program
  built with ferrograd_amd runs on "cpu" exactly as the reference would run it.
* `reference.py`: closed-form numpy restatements of the benchmark configs and
  the reference's known-answer values, used to pin the CPU device.

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
