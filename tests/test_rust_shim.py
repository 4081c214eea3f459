"""The Rust shim crate (rust/ferrograd-hip-sys) against the C headers.

The crate cannot be compiled here (no Rust toolchain), so this checks what
can be checked from the text: every function include/ferrograd_hip.h and
include/ferrograd.h declare has an extern declaration in src/lib.rs with the
same name, the same parameter types and the same return type (each C type
translated by the C ABI's rules: int -> i32, size_t -> usize, int64_t -> i64,
`const T*` -> `*const T`, `T* const*` -> `*const *mut T`, an array parameter
-> a pointer), and the crate declares nothing the headers do not. The library
exports every one of those symbols (tests/test_abi.py checks the exports).
"""
from __future__ import annotations

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# C base types and the Rust types the C ABI gives them (std::ffi for char/void).
C_BASE = {"int": "i32", "unsigned": "u32", "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64",
          "uint8_t": "u8", "size_t": "usize", "float": "f32", "double": "f64", "char": "c_char", "void": "c_void"}


def c_type_to_rust(decl: str, is_param: bool = True) -> str:
    """The Rust type of one C parameter declaration (name included) or, with
    is_param False, of a return type."""
    decl = " ".join(decl.replace("*", " * ").split())
    array = False
    if is_param:
        m = re.match(r"^(.*?)\s*(\w+)\s*(\[\s*\d*\s*\])?$", decl)
        assert m, decl
        decl, array = m.group(1), m.group(3) is not None
    toks = decl.split()
    const_base = False
    if toks and toks[0] == "const":
        const_base, toks = True, toks[1:]
    base, rest = toks[0], toks[1:]
    if rest and rest[0] == "const":  # `T const *`
        const_base, rest = True, rest[1:]
    rust = C_BASE.get(base, base)
    if base == "void" and not rest and not array:
        return "()"
    # pointer levels, innermost first: each level's pointee constness
    levels, pointee_const = [], const_base
    for t in rest:
        if t == "*":
            levels.append(pointee_const)
            pointee_const = False
        elif t == "const":
            pointee_const = True  # qualifies the pointer just written
        else:
            raise AssertionError(decl)
    if array:
        levels.append(pointee_const)
    for c in levels:
        rust = ("*const " if c else "*mut ") + rust
    return rust


def header_signatures() -> dict:
    """name -> (parameter types, return type), in Rust spelling."""
    out = {}
    for h in ("ferrograd_hip.h", "ferrograd.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^((?:const\s+)?[a-z_0-9]+\s*\**)\s*(fg_\w+)\s*\(([^;]*?)\)\s*;", text,
                             flags=re.M | re.S):
            params = m.group(3).strip()
            ps = [] if params in ("", "void") else [c_type_to_rust(p) for p in params.split(",")]
            out[m.group(2)] = (ps, c_type_to_rust(m.group(1), is_param=False))
    return out


def rust_signatures() -> dict:
    text = open(os.path.join(ROOT, "rust", "ferrograd-hip-sys", "src", "lib.rs")).read()
    out = {}
    for block in re.findall(r'extern "C" \{(.*?)\n\}', text, flags=re.S):
        for m in re.finditer(r"pub fn (fg_\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
            params = [p for p in (x.strip() for x in m.group(2).split(",")) if p]
            types = [" ".join(p.split(":", 1)[1].split()) for p in params]
            ret = " ".join(m.group(3).split()) if m.group(3) else "()"
            out[m.group(1)] = (types, ret)
    return out


def test_c_type_translation():
    assert c_type_to_rust("fg_prog* const* progs") == "*const *mut fg_prog"
    assert c_type_to_rust("const unsigned grid[3]") == "*const u32"
    assert c_type_to_rust("uint64_t out[5]") == "*mut u64"
    assert c_type_to_rust("const char** out") == "*mut *const c_char"
    assert c_type_to_rust("void* dptr") == "*mut c_void"
    assert c_type_to_rust("int64_t start") == "i64"
    assert c_type_to_rust("const char*", is_param=False) == "*const c_char"
    assert c_type_to_rust("int", is_param=False) == "i32"


def test_rust_shim_declares_every_header_function_with_its_types():
    h, r = header_signatures(), rust_signatures()
    assert sorted(set(h) - set(r)) == []
    assert sorted(set(r) - set(h)) == []
    assert {k: (h[k], r[k]) for k in h if h[k] != r[k]} == {}


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
