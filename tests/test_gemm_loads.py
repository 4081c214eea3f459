"""How the MFMA GEMM's operand stages read memory, on HIP against float64.

The stages load through raw buffer loads: each lane's 32-bit byte offset is
the same in every k-tile and the k-tile's start goes in the scalar offset.
That needs every term of the operand's index to be a range with a
non-negative coefficient and the buffer to stay under 2 GiB; otherwise the
stage keeps 64-bit global loads. These cases cover an operand read through
narrow() views (its starts are kernel scalars, whose sign the renderer does
not know, so it keeps global loads, one element at a time for a start that
is not a multiple of 4) beside a contiguous one that takes buffer loads, the
same view read transposed (the [k][row] stage), and an operand of exactly
2 GiB. Each product is checked per element within 1e-4·Σ|terms| of
float64 (matmul as tensor.rs:771-777)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err_bound


def _sources(fg, t):
    return [it["source"] for it in fg.debug_plan([t], fuse=True, render_hip=True)["items"]
            if it["class"] == "gemm_mfma_f32"]


def _narrowed(fg, dev, X, W):
    x = fg.Tensor.new(X, list(X.shape), dev).narrow(0, 37, 2600).narrow(1, 5, 1024)
    w = fg.Tensor.new(W, list(W.shape), dev)
    return x, w


def test_narrowed_operand_keeps_global_loads(fg, cpu):
    X = np.ones((3000, 1100), np.float32)
    W = np.ones((768, 1024), np.float32)
    x, w = _narrowed(fg, cpu, X, W)
    (src,) = _sources(fg, x.matmul(w.permute([1, 0])))
    # The row and column starts are kernel scalars: data1 keeps global loads.
    assert "fg_rs_data1" not in src and "data1[" in src
    assert "__builtin_amdgcn_raw_buffer_load_b128(fg_rs_" in src  # the contiguous operand


def test_two_gib_operand_keeps_global_loads(fg, cpu):
    # An operand of 2^29 floats (2 GiB) is past the 32-bit offsets' limit.
    a = fg.Tensor.new(np.ones((65536, 1), np.float32), [65536, 1], cpu)
    b = fg.Tensor.new(np.ones((1, 8192), np.float32), [1, 8192], cpu)
    w = fg.Tensor.new(np.ones((32, 8192), np.float32), [32, 8192], cpu)
    (src,) = _sources(fg, a.mul(b).contiguous().matmul(w.permute([1, 0])))
    loads = [l for l in src.split("\n") if "const fg_f4 vec0 =" in l]
    assert any("raw_buffer_load" not in l for l in loads)  # the 2 GiB operand
    assert any("raw_buffer_load" in l for l in loads)      # the 1 MiB one


@pytest.mark.gpu
def test_narrowed_operands_against_float64(fg, hip):
    r = np.random.default_rng(17)
    X = r.standard_normal((3000, 1100)).astype(np.float32)
    W = (r.standard_normal((768, 1024)) / 32).astype(np.float32)
    x, w = _narrowed(fg, hip, X, W)
    y = x.matmul(w.permute([1, 0]))
    # The same view as the left operand of a transposed product: dW-shaped,
    # x read along its rows ([k][row] stage).
    g = fg.Tensor.new(r.standard_normal((2600, 256)).astype(np.float32), [2600, 256], hip)
    z = x.permute([1, 0]).matmul(g)
    fg.Tensor.realize_many([y, z])
    xs = X[37:2637, 5:1029].astype(np.float64)
    w64 = W.astype(np.float64)
    assert rel_err_bound(y.numpy(), xs @ w64.T, np.abs(xs) @ np.abs(w64.T), 1e-4) <= 1.0
    g64 = g.numpy().astype(np.float64)
    assert rel_err_bound(z.numpy(), xs.T @ g64, np.abs(xs.T) @ np.abs(g64), 1e-4) <= 1.0


@pytest.mark.gpu
def test_two_gib_operand_against_float64(fg, hip):
    # y = (a bᵀ) Wᵀ with a 2 GiB left operand built on the device: y[m, n] =
    # a[m] · (b · W[n]), checked on sampled rows.
    r = np.random.default_rng(18)
    A = r.uniform(0.5, 1.5, (65536, 1)).astype(np.float32)
    B = r.uniform(-1, 1, (1, 8192)).astype(np.float32)
    W = (r.standard_normal((32, 8192)) / 90).astype(np.float32)
    a, b, w = (fg.Tensor.new(v, list(v.shape), hip) for v in (A, B, W))
    y = a.mul(b).contiguous().matmul(w.permute([1, 0]))
    got = y.numpy()
    rows = np.unique(np.concatenate([[0, 65535], r.integers(0, 65536, 64)]))
    xr = A[rows].astype(np.float64) * B.astype(np.float64)
    xr32 = (A[rows] * B).astype(np.float64)  # the rows of a·bᵀ as the device stores them (one f32 rounding)
    want = xr32 @ W.astype(np.float64).T
    scale = np.abs(xr) @ np.abs(W.astype(np.float64).T)
    assert rel_err_bound(got[rows], want, scale, 1e-4) <= 1.0
