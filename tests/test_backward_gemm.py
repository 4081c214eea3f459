"""The backward products of nn::Linear on HIP, standalone, at the train steps'
shapes (C4: B=256, 784->128->10; C5: B=8192, 784->4096->4096->10).

A Linear forward y = h·Wᵀ (nn.rs:97-104) with upstream gradient G gives, by
gradient.rs's Mul and Expand rules (gradient.rs:100-105, 165-176):
  dH = G·W     [B, in]  ("NN": G k-contiguous, W contiguous along the output)
  dW = Gᵀ·H    [out, in] ("TN": both operands contiguous along the outputs)
The MFMA GEMM stages each orientation differently, and the train step runs
them with epilogues: the relu mask of the layer below on dH
(Where(0 < z, G·W, 0)), and the SGD update W - lr·dW on dW, which at K = B =
8192 is split over K with the update in the finishing pass. Each is checked
against float64 on the same inputs, per element within 1e-4 · Σ|terms| (the
update through its effective gradient, tests/f64ref.py), on sampled output
rows at the C5 shapes, and against the CPU oracle where the oracle finishes
in seconds."""
from __future__ import annotations

import numpy as np
import pytest

import f64ref
from conftest import rel_err_bound

pytestmark = pytest.mark.gpu

LR = 0.01


def inputs(B, fan_in, fan_out, seed):
    r = np.random.default_rng(seed)
    h = r.uniform(0, 1, (B, fan_in)).astype(np.float32)
    z = r.standard_normal((B, fan_in)).astype(np.float32)  # pre-activation for the relu case
    w = (r.standard_normal((fan_out, fan_in)) * np.sqrt(2.0 / fan_in)).astype(np.float32)
    g = (r.standard_normal((B, fan_out)) / B).astype(np.float32)  # a mean-loss gradient's scale
    return h, z, w, g


def backward_products(fg, dev, h, w, g, relu_input=None):
    """(dH, dW) of sum(G ⊙ (h·Wᵀ)) on `dev`; with relu_input, h = relu(z) and
    the first product is dZ = Where(0 < z, G·W, 0)."""
    x = fg.Tensor.new(relu_input if relu_input is not None else h, list(h.shape), dev).with_requires_grad(True)
    wt = fg.Tensor.new(w, list(w.shape), dev).with_requires_grad(True)
    gt = fg.Tensor.new(g, list(g.shape), dev)
    xin = x.relu() if relu_input is not None else x
    loss = xin.matmul(wt.permute([1, 0])).mul(gt).sum([0, 1])
    dx, dw = loss.gradient([x, wt])
    fg.Tensor.realize_many([dx, dw])
    return dx.numpy().reshape(h.shape), dw.numpy().reshape(w.shape)


def sgd_through_dw(fg, dev, h, w, g):
    """W after W.assign(W - lr · dW) with dW = Gᵀ·h fused into the update."""
    x = fg.Tensor.new(h, list(h.shape), dev)
    wt = fg.Tensor.new(w, list(w.shape), dev).with_requires_grad(True)
    gt = fg.Tensor.new(g, list(g.shape), dev)
    loss = x.matmul(wt.permute([1, 0])).mul(gt).sum([0, 1])
    (dw,) = loss.gradient([wt])
    wt.assign(wt.detach().sub(dw.mul(fg.Tensor.scalar(LR, dev))))
    fg.Tensor.realize_many([wt])
    return wt.numpy().reshape(w.shape)


def rows_of(n, k, seed):
    r = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, n - 1], r.integers(0, n, k)]))


# (B, in, out): C4's two layers and C5's three.
SHAPES = {"c4_l1": (256, 784, 128), "c4_l2": (256, 128, 10),
          "c5_l1": (8192, 784, 4096), "c5_l2": (8192, 4096, 4096), "c5_l3": (8192, 4096, 10)}


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_dh_nn_and_dw_tn_against_float64(fg, hip, name):
    B, fi, fo = SHAPES[name]
    h, z, w, g = inputs(B, fi, fo, 31)
    relu = name in ("c4_l2", "c5_l2", "c5_l3")  # layers with a hidden layer below them
    dx, dw = backward_products(fg, hip, h, w, g, relu_input=z if relu else None)
    hh = np.where(z > 0, z, np.float32(0)) if relu else h
    g64, w64 = g.astype(np.float64), w.astype(np.float64)
    # dH (or dZ with the relu mask), on sampled batch rows.
    br = rows_of(B, 48, 1)
    want = g64[br] @ w64
    scale = np.abs(g64[br]) @ np.abs(w64)
    if relu:
        want, scale = np.where(z[br] > 0, want, 0.0), np.where(z[br] > 0, scale, 0.0)
    assert rel_err_bound(dx[br], want, scale, 1e-4) <= 1.0
    if relu:
        assert np.all(dx[br][z[br] <= 0] == 0)  # the mask's zeros are exact
    # dW, on sampled output rows.
    orow = rows_of(fo, 48, 2)
    h64 = hh.astype(np.float64)
    want = g64[:, orow].T @ h64
    scale = np.abs(g64[:, orow]).T @ np.abs(h64)
    assert rel_err_bound(dw[orow], want, scale, 1e-4) <= 1.0


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_sgd_update_fused_with_dw(fg, hip, name):
    # At C5's K = 8192 the dW products are split over K (784 and 4096 wide
    # outputs in 4 splits, the 10-row one in 32), with the update applied
    # after the partials are summed.
    B, fi, fo = SHAPES[name]
    h, _, w, g = inputs(B, fi, fo, 37)
    w1 = sgd_through_dw(fg, hip, h, w, g)
    orow = rows_of(fo, 48, 3)
    g64, h64 = g.astype(np.float64)[:, orow], h.astype(np.float64)
    err = f64ref.sgd_effective_gradient_err(w[orow], w1[orow], g64.T @ h64, np.abs(g64).T @ np.abs(h64), LR)
    assert err <= 1.0


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_sgd_update_fused_with_dw_at_full_precision(fg, hip, name):
    # With W at the scale of an initialised layer the update's own rounding,
    # ulp(W1)/lr, is tens of times the product's error bound and hides it.
    # With W a millionth of that, W1 is about -lr·dW and that rounding is
    # about 2^-24 of the gradient: the fused kernel's effective gradient is
    # then held to 1e-4·Σ|terms| of the exact product (plus 2^-22 |dW| for
    # the f32 roundings of dW, lr·dW and the update).
    B, fi, fo = SHAPES[name]
    h, _, w, g = inputs(B, fi, fo, 43)
    w = (w * np.float32(1e-6)).astype(np.float32)
    w1 = sgd_through_dw(fg, hip, h, w, g)
    orow = rows_of(fo, 48, 4)
    g64, h64 = g.astype(np.float64)[:, orow], h.astype(np.float64)
    want, scale = g64.T @ h64, np.abs(g64).T @ np.abs(h64)
    lr32 = float(np.float32(LR))
    geff = (w[orow].astype(np.float64) - w1[orow].astype(np.float64)) / lr32
    ulp_term = np.spacing(np.abs(w1[orow])).astype(np.float64) / lr32
    assert np.median(ulp_term / (1e-4 * scale)) < 0.01  # the product's own bound dominates
    bound = 1e-4 * scale + 2.0 ** -22 * np.abs(want) + ulp_term
    assert float(np.max(np.abs(geff - want) / bound)) <= 1.0


@pytest.mark.parametrize("name", ["c4_l1", "c4_l2"])
def test_backward_products_against_the_oracle(fg, cpu, name):
    B, fi, fo = SHAPES[name]
    h, z, w, g = inputs(B, fi, fo, 41)
    relu = name == "c4_l2"
    (dx_c, dw_c), (dx_h, dw_h) = (backward_products(fg, d, h, w, g, relu_input=z if relu else None)
                                  for d in (cpu, "hip"))
    hh = np.where(z > 0, z, np.float32(0)) if relu else h
    sx = np.abs(g.astype(np.float64)) @ np.abs(w.astype(np.float64))
    sw = np.abs(g.astype(np.float64)).T @ np.abs(hh.astype(np.float64))
    assert rel_err_bound(dx_h, dx_c, sx, 1e-4) <= 1.0
    assert rel_err_bound(dw_h, dw_c, sw, 1e-4) <= 1.0
    # The two updates' effective gradients: each within 1e-4 · Σ|terms| of
    # the exact product, plus the rounding of its own update (f64ref).
    w_c, w_h = (sgd_through_dw(fg, d, h, w, g) for d in (cpu, "hip"))
    lr32 = float(np.float32(LR))
    g_c, g_h = ((w.astype(np.float64) - v) / lr32 for v in (w_c, w_h))
    bound = 2e-4 * sw + 2.0 ** -22 * np.abs(g_c) + (np.spacing(np.abs(w_c)) + np.spacing(np.abs(w_h))) / lr32
    assert np.all(np.abs(g_h - g_c) <= bound)
