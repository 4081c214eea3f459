"""The Rust shim crate (rust/ferrograd-hip-sys) against the C headers.

The crate cannot be compiled here (no Rust toolchain), so this checks what
can be checked from the text: every function include/ferrograd_hip.h and
include/ferrograd.h declare has an extern declaration in src/lib.rs with the
same name and number of parameters, and the crate declares nothing the
headers do not. The library exports every one of those symbols
(tests/test_abi.py checks the exports).
"""
from __future__ import annotations

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions() -> dict:
    out = {}
    for h in ("ferrograd_hip.h", "ferrograd.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^(?:const\s+)?[a-z_0-9]+\s*\**\s*(fg_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
            params = m.group(2).strip()
            out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def rust_functions() -> dict:
    text = open(os.path.join(ROOT, "rust", "ferrograd-hip-sys", "src", "lib.rs")).read()
    out = {}
    for block in re.findall(r'extern "C" \{(.*?)\n\}', text, flags=re.S):
        for m in re.finditer(r"pub fn (fg_\w+)\((.*?)\)\s*(?:->\s*[^;]+)?;", block, flags=re.S):
            params = m.group(2).strip().rstrip(",")
            out[m.group(1)] = 0 if not params else params.count(",") + 1
    return out


def test_headers_parse():
    h = header_functions()
    assert "fg_hip_render" in h and "fg_tensor_realize_many" in h and len(h) > 80


def test_rust_shim_declares_every_header_function_with_its_arity():
    h, r = header_functions(), rust_functions()
    assert sorted(set(h) - set(r)) == []
    assert sorted(set(r) - set(h)) == []
    assert {k: (h[k], r[k]) for k in h if h[k] != r[k]} == {}


def test_reference_side_module_uses_only_declared_functions():
    text = open(os.path.join(ROOT, "rust", "ferrograd-hip-sys", "reference", "src", "device", "hip.rs")).read()
    used = set(re.findall(r"sys::(fg_\w+)\(", text))
    assert used and used <= set(header_functions())
