"""The 160-wide MFMA GEMM tiles on HIP against float64.

A side of 784 (an MLP's input width, the C5 train step's dW1 = dZ1ᵀ·X with
K = 8192) pads to 1024 columns in 256-wide tiles; a 256x160 workgroup tile
(four waves of 64x160, five 32-wide MFMA columns each) pads it to 800. Its
[k][row] operand stages cut the five tiles' interleaved rows into a chunk of
four (16-byte LDS reads) and one of one. These shapes are ones the tile model
gives a 160-wide tile, in all three orientations of a Linear's products
(forward x·Wᵀ, dX = G·W, dW = Gᵀ·X: gradient.rs:100-105, 165-176), with
ragged edges, split K, stream-K (each workgroup an equal share of the
(tile, k-tile) iterations, crossing tile boundaries; C5's dW1 runs so),
16-wide k-tiles (three LDS stages) and a 160-row tile (the chunked layout on
the A side). Each product is checked per element within 1e-4·Σ|terms| of
float64 on sampled output rows."""
from __future__ import annotations

import re

import numpy as np
import pytest

from conftest import rel_err_bound

# (B, in, out) -> the tile (BM, BN, stream-K) each product gets, from the tile model.
CASES = {
    (3000, 800, 600): {"fwd": (256, 160, False), "dx": (256, 160, False)},
    (4096, 4096, 784): {"fwd": (256, 160, True), "dw": (160, 256, True)},
    (2048, 784, 1000): {"dx": (256, 160, False), "dw": (256, 160, False)},
    (8192, 784, 4096): {"dx": (256, 160, True), "dw": (256, 160, True)},
}


def products(fg, dev, x, w, g):
    xt = fg.Tensor.new(x, list(x.shape), dev).with_requires_grad(True)
    wt = fg.Tensor.new(w, list(w.shape), dev).with_requires_grad(True)
    gt = fg.Tensor.new(g, list(g.shape), dev)
    y = xt.matmul(wt.permute([1, 0]))
    dx, dw = y.mul(gt).sum([0, 1]).gradient([xt, wt])
    return {"fwd": y, "dx": dx, "dw": dw}


def gemm_tile(fg, t):
    src = [it["source"] for it in fg.debug_plan([t], fuse=True, render_hip=True)["items"]
           if it["class"] == "gemm_mfma_f32"]
    assert len(src) == 1
    return tuple(int(re.search(r"#define %s (\d+)" % k, src[0]).group(1)) for k in ("BM", "BN")) + (
        "#define ITERS_" in src[0],)


@pytest.mark.parametrize("shape", sorted(CASES))
def test_tile_model_gives_160_wide_tiles(fg, cpu, shape):
    B, fi, fo = shape
    ones = np.ones
    p = products(fg, cpu, ones((B, fi), np.float32), ones((fo, fi), np.float32), ones((B, fo), np.float32))
    for name, tile in CASES[shape].items():
        assert gemm_tile(fg, p[name]) == tile, name


def _c_expr(text, env):
    """Evaluates one of the kernel's integer expressions (non-negative
    operands, so C's division is Python's floor division)."""
    return eval(text.replace("(long)", "").replace("/", "//"), {}, dict(env))


def test_stream_k_tile_order_groups_each_xcds_tiles(fg, cpu):
    # C5's dW1 (4096x784, K 8192): 80 tiles of 256x160, 256 k-tiles each, on
    # 256 workgroups of 80 k-tiles. Workgroups 16 apart start at the same k
    # position 5 tiles apart, and round-robin dispatch puts workgroups 8 apart
    # on one XCD. The kernel's own expressions, evaluated here: the row-major
    # slot is a bijection, the second pass inverts it, and the 16 tiles that
    # one XCD's workgroups start at one k position cover at most 4 of the 16
    # row blocks (the grouped order gave 16 distinct ones: no shared rows).
    B, fi, fo = 8192, 784, 4096
    ones = np.ones
    p = products(fg, cpu, ones((B, fi), np.float32), ones((fo, fi), np.float32), ones((B, fo), np.float32))
    (src,) = [it["source"] for it in fg.debug_plan([p["dw"]], fuse=True, render_hip=True)["items"]
              if it["class"] == "gemm_mfma_f32"]
    d = {k: int(v) for k, v in re.findall(r"#define (\w+) (\d+)L?\n", src)}
    assert (d["NTILES_"], d["KTT_"], d["G_"], d["SK_D_"]) == (80, 256, 256, 5)
    slot = re.search(r"const int sq = (.+?);", src).group(1)
    inv = re.search(r"const long t0 = \(long\)(.+?) \* KTT_;", src).group(1)
    nbn = (fi + d["BN"] - 1) // d["BN"]
    fwd = [_c_expr(slot, {**d, "bid": b}) for b in range(d["NTILES_"])]
    assert sorted(fwd) == list(range(d["NTILES_"]))
    assert all(_c_expr(inv, {**d, "sq": q}) == b for b, q in enumerate(fwd))
    share = d["NTILES_"] * d["KTT_"] // d["G_"]
    for x in range(8):
        starts = {}
        for w in range(x, d["G_"], 8):
            tile, k0 = divmod(w * share, d["KTT_"])
            starts.setdefault(k0, []).append(fwd[tile] // nbn)
        for rows in starts.values():
            assert len(rows) == 16 and len(set(rows)) <= 4, rows


@pytest.mark.gpu
@pytest.mark.parametrize("shape", sorted(CASES))
def test_160_wide_tiles_against_float64(fg, hip, shape):
    B, fi, fo = shape
    r = np.random.default_rng(B + fi + fo)
    x = r.uniform(-1, 1, (B, fi)).astype(np.float32)
    w = (r.standard_normal((fo, fi)) / np.sqrt(fi)).astype(np.float32)
    g = r.standard_normal((B, fo)).astype(np.float32)
    p = products(fg, hip, x, w, g)
    fg.Tensor.realize_many([p["fwd"], p["dx"], p["dw"]])
    x64, w64, g64 = (a.astype(np.float64) for a in (x, w, g))
    br = np.unique(np.concatenate([[0, B - 1], r.integers(0, B, 40)]))
    orow = np.unique(np.concatenate([[0, fo - 1], r.integers(0, fo, 40)]))
    checks = {
        "fwd": (p["fwd"].numpy().reshape(B, fo)[br], x64[br] @ w64.T, np.abs(x64[br]) @ np.abs(w64.T)),
        "dx": (p["dx"].numpy().reshape(B, fi)[br], g64[br] @ w64, np.abs(g64[br]) @ np.abs(w64)),
        "dw": (p["dw"].numpy().reshape(fo, fi)[orow], g64[:, orow].T @ x64, np.abs(g64[:, orow]).T @ np.abs(x64)),
    }
    for name, (got, want, scale) in checks.items():
        assert rel_err_bound(got, want, scale, 1e-4) <= 1.0, name


FORCED = r"""
import sys
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import numpy as np
import ferrograd_amd as fg
from conftest import rel_err_bound
from test_gemm_tiles import products
B, fi, fo = 1000, 784, 600
r = np.random.default_rng(5)
x = r.uniform(-1, 1, (B, fi)).astype(np.float32)
w = (r.standard_normal((fo, fi)) / np.sqrt(fi)).astype(np.float32)
g = r.standard_normal((B, fo)).astype(np.float32)
p = products(fg, "hip", x, w, g)
fg.Tensor.realize_many([p["fwd"], p["dx"], p["dw"]])
x64, w64, g64 = (a.astype(np.float64) for a in (x, w, g))
errs = {
    "fwd": rel_err_bound(p["fwd"].numpy().reshape(B, fo), x64 @ w64.T, np.abs(x64) @ np.abs(w64.T), 1e-4),
    "dx": rel_err_bound(p["dx"].numpy().reshape(B, fi), g64 @ w64, np.abs(g64) @ np.abs(w64), 1e-4),
    "dw": rel_err_bound(p["dw"].numpy().reshape(fo, fi), g64.T @ x64, np.abs(g64.T) @ np.abs(x64), 1e-4),
}
print(errs, flush=True)
sys.exit(0 if max(errs.values()) <= 1.0 else 1)
"""


@pytest.mark.gpu
@pytest.mark.parametrize("tile", ["256,160,16,4,1,3,3", "160,256,32,1,4,2", "256,160,16,4,1,0,3", "128,128,32,2,2,0",
                                  "192,96,32,2,1,2", "96,192,32,1,2,0", "256,256,8,2,2,1", "64,64,24,2,2,1"])
def test_forced_160_wide_tiles_against_float64(tile):
    # Tiles the model rarely picks (16-wide k-tiles with three LDS stages; a
    # 160-row tile on every orientation; stream-K, split count 0, with those
    # stages and with two workgroups per CU on ragged 128x128 tiles; waves of
    # three 32-wide tiles, [k][row] stages as a chunk of two and one of one;
    # k-tiles of one and of three 8-k groups),
    # fixed with the FG_GEMM_TILE tuning override in a process of their own,
    # as it holds for every GEMM.
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, FG_GEMM_TILE=tile)
    r = subprocess.run([sys.executable, "-c", FORCED, root], env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr


# One-pass small GEMMs (M*N*K <= 2^26): forward x·Wᵀ, dX = G·W and dW = Gᵀ·X
# of Linear layers at these (B, in, out), covering K a multiple of 4 (16-byte
# loads of a lane's four k) and not (one element per step), ragged 16x16
# tiles, one to sixteen waves per workgroup, and a K range long enough that
# each wave folds its groups in rolled chunks of four ((16, 20000, 16): dW's
# K is 16, forward's 20000).
SMALL = [(256, 784, 128), (256, 128, 10), (65, 129, 47), (100, 8192, 20), (16, 20000, 16), (250, 96, 64)]


def small_gemm_sources(fg, p):
    out = {}
    for name, t in p.items():
        items = [it for it in fg.debug_plan([t], fuse=True, render_hip=True)["items"]
                 if it["class"] == "gemm_mfma_f32"]
        out[name] = items[0]["source"] if items else None
    return out


@pytest.mark.parametrize("shape", SMALL)
def test_small_gemm_forms(fg, cpu, shape):
    from hipcompile import compile_sources

    B, fi, fo = shape
    ones = np.ones
    p = products(fg, cpu, ones((B, fi), np.float32), ones((fo, fi), np.float32), ones((B, fo), np.float32))
    srcs = {k: v for k, v in small_gemm_sources(fg, p).items() if v}
    assert srcs, "no product took the GEMM path"
    for name, src in srcs.items():
        assert "mfma_f32_16x16x4f32" in src and "_part(" not in src, name
    if shape == (16, 20000, 16):
        assert "for (int c0 = 0; c0 <" in srcs["fwd"]
    compile_sources({v: k for k, v in srcs.items()}, limit_s=120)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", SMALL)
def test_small_gemms_against_float64(fg, hip, shape):
    B, fi, fo = shape
    print(f"small gemm products {shape}", flush=True)
    r = np.random.default_rng(sum(shape))
    x = r.uniform(-1, 1, (B, fi)).astype(np.float32)
    w = r.uniform(-1, 1, (fo, fi)).astype(np.float32)
    g = r.uniform(-1, 1, (B, fo)).astype(np.float32)
    p = products(fg, hip, x, w, g)
    fg.Tensor.realize_many(list(p.values()))
    x64, w64, g64 = (a.astype(np.float64) for a in (x, w, g))
    want = {"fwd": (x64 @ w64.T, np.abs(x64) @ np.abs(w64).T), "dx": (g64 @ w64, np.abs(g64) @ np.abs(w64)),
            "dw": (g64.T @ x64, np.abs(g64).T @ np.abs(x64))}
    for name, t in p.items():
        v, sc = want[name]
        got = t.numpy().astype(np.float64).reshape(v.shape)
        assert rel_err_bound(got, v, sc, 1e-4) <= 1.0, name
