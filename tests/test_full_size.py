"""The HIP path at BASELINE's full sizes, checked through properties that do
not need the oracle to finish at that size:

- C2 over 2^26 elements, bit for bit against IEEE f32 per-operation rounding
  restated in numpy;
- C3 at 4096^3 with the bench's inputs: 64 sampled output rows against
  float64, within 1e-4 * sum|terms| per element;
- one train step of C5's layer shapes (784 -> 4096 -> 4096 -> 10) at batch
  1024 against a float64 forward and hand-derived backward pass. The loss must
  agree within 1e-4 relative, every parameter after the SGD update within
  1e-4 * (|p| + lr * (|g| + 1e-3)). At this size some pre-activations lie
  within f32 rounding of 0, where f32 and f64 take different relu branches and
  the gradient jumps; the float64 backward therefore uses the relu masks of the
  pre-activations the device computed, and the test checks separately that
  those masks differ from float64's only where |z| <= 1e-5 * sum|terms|.

The C1 row reduce runs at [4096, 4096] against the oracle in test_parity.py."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err_bound


@pytest.mark.gpu
def test_c2_full_size_bit_exact(fg, hip):
    n = 1 << 26
    r = np.random.default_rng(2)
    a, b, c = (r.uniform(-1, 1, n).astype(np.float32) for _ in range(3))
    ta, tb, tc = (fg.Tensor.new(v, [n], hip) for v in (a, b, c))
    got = ta.mul(tb).add(tc).relu().numpy()
    ab = (a.astype(np.float64) * b).astype(np.float32)  # each operation rounded once
    s = (ab.astype(np.float64) + c).astype(np.float32)
    want = np.where(np.float32(0) < s, s, np.float32(0)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_c3_full_size_sampled_rows(fg, hip):
    x = np.random.default_rng(5).standard_normal((4096, 4096)).astype(np.float32)
    w = np.random.default_rng(6).uniform(-1 / 64, 1 / 64, (4096, 4096)).astype(np.float32)
    tx, tw = fg.Tensor.new(x, [4096, 4096], hip), fg.Tensor.new(w, [4096, 4096], hip)
    tb = fg.Tensor.zeros([4096], hip)
    y = tx.matmul(tw.permute([1, 0])).add(tb).numpy().reshape(4096, 4096)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, 4095], np.random.default_rng(9).integers(0, 4096, 59)]))
    xs, wd = x[rows].astype(np.float64), w.astype(np.float64)
    want = xs @ wd.T
    scale = np.abs(xs) @ np.abs(wd).T
    assert rel_err_bound(y[rows], want, scale, 1e-4) <= 1.0
    assert np.isfinite(y).all()


def mlp_step_f64(x, t, params, lr, masks=None):
    """One train step of a Linear/ReLU stack in float64: forward, mean
    softmax cross-entropy, backward by hand ((softmax - t)/B propagated through
    the layers, relu masks from the pre-activations, or `masks[i]` for hidden
    layer i when given), SGD."""
    ws = [p.astype(np.float64) for p in params[0::2]]
    bs = [p.astype(np.float64) for p in params[1::2]]
    h, t = x.astype(np.float64), t.astype(np.float64)
    ins, gates = [], []
    for i, (w, b) in enumerate(zip(ws, bs)):
        ins.append(h)
        z = h @ w.T + b
        if i + 1 < len(ws):
            gates.append(z > 0 if masks is None else masks[i])
            h = np.where(gates[-1], z, 0.0)
        else:
            h = z
    zs = h - h.max(1, keepdims=True)
    logp = zs - np.log(np.exp(zs).sum(1, keepdims=True))
    loss = -np.mean((t * logp).sum(1))
    dz = (np.exp(logp) - t) / x.shape[0]
    grads = [None] * len(params)
    for i in reversed(range(len(ws))):
        grads[2 * i] = dz.T @ ins[i]
        grads[2 * i + 1] = dz.sum(0)
        if i > 0:
            dz = (dz @ ws[i]) * gates[i - 1]
    new = [p.astype(np.float64) - lr * g for p, g in zip(params, grads)]
    return loss, new, grads


@pytest.mark.gpu
def test_wide_mlp_train_step_against_float64(fg, hip):
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    batch, dims, lr = 1024, (784, 4096, 4096, 10), 0.01
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 9, 10)
    fg.reset_init_seed(42)
    model = Mlp(dims, hip)
    params = model.parameters()
    p0 = [p.numpy().copy() for p in params]
    opt = fg.Sgd(params, lr)
    x, t = fg.Tensor.new(xs, list(xs.shape), hip), fg.Tensor.new(ts, list(ts.shape), hip)
    # The hidden pre-activations as the device computes them (the same
    # deterministic kernels the train step runs), and their relu masks.
    z1 = model.layers[0](x)
    z2 = model.layers[1](z1.relu())
    z1d, z2d = (z.numpy().reshape(batch, -1) for z in (z1, z2))
    masks = [z1d > 0, z2d > 0]
    w1, b1, w2, b2 = (p.astype(np.float64) for p in p0[:4])
    x64 = xs.astype(np.float64)
    z1r = x64 @ w1.T + b1
    h1r = np.where(masks[0], np.maximum(z1r, 0.0), 0.0)
    z2r = h1r @ w2.T + b2
    for zd, zr, s in ((z1d, z1r, np.abs(x64) @ np.abs(w1).T + np.abs(b1)), (z2d, z2r, h1r @ np.abs(w2).T + np.abs(b2))):
        assert rel_err_bound(zd, zr, s, 1e-4) <= 1.0
        flips = (zd > 0) != (zr > 0)
        assert np.all(np.abs(zr[flips]) <= 1e-5 * s[flips]), "a relu mask flipped away from 0"
    loss = model.forward(x).cross_entropy(t)
    opt.zero_grad()
    loss.backward()
    opt.step()
    got_loss = loss.to_vec()[0]
    got = [p.numpy() for p in params]
    want_loss, want, grads = mlp_step_f64(xs, ts, p0, lr, masks)
    assert abs(got_loss - want_loss) <= 1e-4 * abs(want_loss), (got_loss, want_loss)
    for i, (g, w, p, gr) in enumerate(zip(got, want, p0, grads)):
        scale = np.abs(p.astype(np.float64)) + lr * (np.abs(gr) + 1e-3)
        assert rel_err_bound(g, w, scale, 1e-4) <= 1.0, i


def test_float64_step_matches_the_golden_two_layer_reference():
    # The N-layer float64 step above must reduce to the committed fixtures'
    # two-layer reference (tests/golden/make_golden.py), and fail on a planted
    # mistake (a relu mask taken after the activation instead of before).
    import os
    import sys

    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    sys.path.insert(0, golden)
    import make_golden as mg

    with np.load(os.path.join(golden, "c4_step_b8.npz")) as z:
        f = {k: z[k] for k in z.files}
    p0 = [f[n + "_0"] for n in ("w1", "b1", "w2", "b2")]
    l1, n1, g1 = mlp_step_f64(f["x"], f["t"], p0, 0.01)
    l2, n2, g2 = mg.mlp_step_f64(f["x"], f["t"], p0)
    assert l1 == l2
    assert all(np.array_equal(a, b) for a, b in zip(n1 + g1, n2 + g2))
    mg.check_c4(f, p0, float(f["loss"][0]), [p.astype(np.float32) for p in n1])
