"""The C-ABI library loads and exports every entry point its headers declare.
No compute calls (CPU only)."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header: str) -> list:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fg_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", ["ferrograd_hip.h", "ferrograd.h"])
def test_library_exports_every_declared_symbol(fg, header):
    names = declared(header)
    assert len(names) > 10
    lib = fg.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_exports_are_c_linkage(fg):
    out = subprocess.run(["nm", "-D", "--defined-only", fg.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (fg_[a-z0-9_]+)$", out, flags=re.M))
    for h in ("ferrograd_hip.h", "ferrograd.h"):
        assert set(declared(h)) <= exported


def test_headers_compile_as_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "ferrograd_hip.h"\n#include "ferrograd.h"\nint main(void){return 0;}\n')
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), "-c", str(src),
                        "-o", str(tmp_path / "t.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_errors_cross_the_abi_as_status_codes(fg):
    import ctypes

    lib = fg.lib()
    out = ctypes.c_void_p()
    shape = (ctypes.c_int64 * 1)(3)
    rc = lib.fg_tensor_zeros(7, 0, shape, 1, ctypes.byref(out))  # unknown device
    assert rc != 0 and b"unknown device" in lib.fg_last_error()


def test_graph_threshold_knob(fg):
    # Host-side setting only: no device is touched.
    prev = fg.graph_min_launches(5)
    try:
        # The default: every plan launches kernel by kernel (FG_HIP_GRAPHS=1: 2).
        assert prev == (2 if os.environ.get("FG_HIP_GRAPHS") == "1" else 0)
        assert fg.graph_min_launches(3) == 5
        for bad in (1, -1):
            with pytest.raises(fg.FerrogradError, match="at least 2 launches"):
                fg.graph_min_launches(bad)
        assert fg.graph_min_launches(0) == 3  # a rejected value leaves the setting alone
        assert fg.graph_min_launches(2) == 0
    finally:
        fg.graph_min_launches(prev)


def test_bench_refuses_more_than_one_gpu():
    # Every config here runs on one GPU; --gpus N > 1 exits with a message
    # before touching a device.
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one MI355X" in r.stderr and r.stdout == ""
