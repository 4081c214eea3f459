"""The HIP path at BASELINE's full sizes, checked through properties that do
not need the oracle to finish at that size:

- C2 over 2^26 elements, bit for bit against IEEE f32 per-operation rounding
  restated in numpy;
- C3 at 4096^3 with the bench's inputs: 64 sampled output rows against
  float64, within 1e-4 * sum|terms| per element;
- one train step of C5's layer shapes (784 -> 4096 -> 4096 -> 10) at the
  benched batch 8192 and at 1024, product by product on the device's own
  intermediate values (held pre-activations). Evaluating float64 on the
  device's forward values matters: some pre-activations lie within f32
  rounding of 0, where f32 and f64 take different relu branches and the
  gradient jumps.

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


@pytest.mark.gpu
@pytest.mark.parametrize("batch,lr", [(1024, 0.01), (8192, 0.01), (8192, 1.0)])
def test_wide_mlp_train_step_product_by_product(fg, hip, batch, lr):
    """One C5 train step (784 -> 4096 -> 4096 -> 10) at the benched B=8192 and
    at 1024, where the GEMM tile and split-K choices differ (choose_gemm_tile
    picks them from M, N and K). The step's own pre-activations are read from
    the held tensors afterwards; every forward product is checked on sampled
    batch rows, the loss against float64 cross-entropy of the device's
    logits, and each parameter's effective gradient (p0 - p1)/lr against
    float64 backward products on the device's forward values, for sampled
    rows of W1 and W2 and all of W3 and every bias
    (tests/f64ref.py: check_mlp_step).

    The effective gradient carries the update's own rounding, ulp(p1)/lr:
    at lr 0.01 that term dominates the bound for W1 and W2 (|p| about 0.05).
    At lr 1 it is 100 times smaller, so the fused weight-gradient + SGD
    kernels are held to the 1e-4 * sum|terms| of their products."""
    import f64ref
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    print(f"C5 step B={batch} lr={lr}", flush=True)
    dims = (784, 4096, 4096, 10)
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 9, 10)
    fg.reset_init_seed(42)
    model = Mlp(dims, hip)
    params = model.parameters()
    p0 = [p.numpy().copy() for p in params]
    opt = fg.Sgd(params, lr)
    x, t = fg.Tensor.new(xs, list(xs.shape), hip), fg.Tensor.new(ts, list(ts.shape), hip)
    z1 = model.layers[0](x)
    z2 = model.layers[1](z1.relu())
    logits = model.layers[2](z2.relu())
    loss = logits.cross_entropy(t)
    opt.zero_grad()
    loss.backward()
    opt.step()
    got_loss = loss.to_vec()[0]
    assert z1.is_realized() and z2.is_realized() and logits.is_realized()
    hidden = [z.numpy().reshape(batch, -1) for z in (z1, z2)]
    rep = f64ref.check_mlp_step(xs, ts, p0, [p.numpy() for p in params], got_loss, hidden,
                                logits.numpy().reshape(batch, -1), lr,
                                rows=[np.random.default_rng(4).choice(4096, 64, replace=False),
                                      np.random.default_rng(5).choice(4096, 64, replace=False)],
                                batch_rows=np.random.default_rng(6).choice(batch, 64, replace=False))
    assert rep["ok"], rep
