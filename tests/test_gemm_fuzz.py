"""Seeded random products on the MFMA GEMM path, on HIP against float64.

Each case draws M, N > 16 and K, with M·N·K above the one-pass small-GEMM
limit (2^26), so the tiled kernel runs: ragged edges on every side, K not a
multiple of the k-tile (bounds-checked k, no buffer loads) or one (buffer
loads), operands read through narrow() views with random starts, stored
transposed (the [k][row] stage), or through a relu (an operand expression
evaluated at the LDS write), and epilogues with a bias or a relu mask. Every
element of 24 sampled output rows is checked within 1e-4·Σ|terms| of float64
on the device's own operand values (matmul as tensor.rs:771-777)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err_bound

SEEDS = list(range(7100, 7140))


def draw(seed):
    r = np.random.default_rng(seed)
    while True:
        M, N = (int(v) for v in r.integers(17, 2600, 2))
        K = int(r.choice([int(r.integers(5, 3000)), 32 * int(r.integers(1, 90))]))
        if M * N * K > (1 << 26) and M * N * K < (1 << 32):
            break
    return r, M, N, K


def build(fg, dev, seed):
    """The product's tensors on `dev` and what float64 needs to check it."""
    r, M, N, K = draw(seed)
    form = r.choice(["plain", "narrow", "transposed", "relu"])
    pad = (int(r.integers(0, 40)), int(r.integers(0, 40)))
    if form == "narrow":
        X = r.standard_normal((M + pad[0] + 3, K + pad[1] + 3)).astype(np.float32)
        x = fg.Tensor.new(X, list(X.shape), dev).narrow(0, pad[0], M).narrow(1, pad[1], K)
        xv = X[pad[0]:pad[0] + M, pad[1]:pad[1] + K]
    elif form == "transposed":
        XT = r.standard_normal((K, M)).astype(np.float32)
        x = fg.Tensor.new(XT, [K, M], dev).permute([1, 0])
        xv = XT.T
    elif form == "relu":
        Z = r.standard_normal((M, K)).astype(np.float32)
        x = fg.Tensor.new(Z, [M, K], dev).relu()
        xv = np.where(Z > 0, Z, np.float32(0))
    else:
        xv = r.standard_normal((M, K)).astype(np.float32)
        x = fg.Tensor.new(xv, [M, K], dev)
    W = (r.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    y = x.matmul(fg.Tensor.new(W, [N, K], dev).permute([1, 0]))
    epi = r.choice(["none", "bias", "mask"])
    B = Zm = None
    if epi == "bias":
        B = r.standard_normal(N).astype(np.float32)
        y = y.add(fg.Tensor.new(B, [N], dev))
    elif epi == "mask":
        Zm = r.standard_normal((M, N)).astype(np.float32)
        zt = fg.Tensor.new(Zm, [M, N], dev)
        y = zt.relu().mul(y) if r.random() < 0.5 else y.mul(zt.relu())
    rows = np.unique(np.concatenate([[0, M - 1], r.integers(0, M, 22)]))
    return (M, N, K, form, epi), y, xv, W, B, Zm, rows


@pytest.mark.parametrize("seed", SEEDS[:8])
def test_fuzz_cases_take_the_tiled_kernel(fg, cpu, seed):
    (M, N, K, form, epi), y, *_ = build(fg, cpu, seed)
    classes = [it["class"] for it in fg.debug_plan([y], fuse=True, render_hip=True)["items"]]
    assert "gemm_mfma_f32" in classes, (M, N, K, form, epi, classes)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", SEEDS)
def test_random_products_against_float64(fg, hip, seed):
    (M, N, K, form, epi), y, xv, W, B, Zm, rows = build(fg, hip, seed)
    got = y.numpy().reshape(M, N)[rows]
    x64, w64 = xv[rows].astype(np.float64), W.astype(np.float64)
    want, scale = x64 @ w64.T, np.abs(x64) @ np.abs(w64.T)
    if B is not None:
        want, scale = want + B, scale + np.abs(B)
    if Zm is not None:
        m = np.where(Zm[rows] > 0, Zm[rows], np.float32(0)).astype(np.float64)
        want, scale = want * m, scale * np.abs(m)
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0, (M, N, K, form, epi)
