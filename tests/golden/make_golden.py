#!/usr/bin/env python3
"""Writes the committed golden fixtures for the parity tests.

Each fixture holds seeded inputs and the outputs of the CPU oracle (the
restated reference clang backend, src/device/cpu.rs + src/codegen/clang.rs),
at sizes small enough to store:

  c1_64x64.npz    ((x*0.5)+1).relu().sum(1), x [64,64] ~ N(0,1)
  c2_4096.npz     (a*b + c).relu(), a,b,c [4096] ~ U(-1,1)
  c3_64.npz       x@W^T + b, x [64,64] ~ N(0,1), W [64,64] ~ U(-1/64,1/64), b ~ N(0,1)
  c4_step_b8.npz  one MLP train step (mnist.rs:84-97 order), 784->16->10,
                  B=8, LCG init seed 42 (nn.rs:13-47), lr 0.01

Before a fixture is written its outputs are checked against an independent
float64 computation in numpy (the elementwise case per operation, rounded to
f32 after each op as IEEE arithmetic fixes it; reductions and products within
1e-4 * sum|terms|; the train step by the textbook softmax-cross-entropy
gradient (softmax - t)/B propagated by hand, each parameter's effective
gradient (p0 - p1)/lr held to 1e-4 of the gradient's condition scale), so a
fixture never records an oracle mistake. Run from the repository root:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))
import f64ref  # noqa: E402  (tests/f64ref.py)


def c1_inputs():
    return {"x": np.random.default_rng(101).standard_normal((64, 64)).astype(np.float32)}


def c2_inputs():
    r = np.random.default_rng(102)
    return {k: r.uniform(-1, 1, 4096).astype(np.float32) for k in ("a", "b", "c")}


def c3_inputs():
    r = np.random.default_rng(103)
    return {"x": r.standard_normal((64, 64)).astype(np.float32),
            "w": r.uniform(-1 / 64, 1 / 64, (64, 64)).astype(np.float32),
            "b": r.standard_normal(64).astype(np.float32)}


def c4_inputs():
    r = np.random.default_rng(104)
    x = r.uniform(0, 1, (8, 784)).astype(np.float32)
    labels = np.minimum(np.floor(r.uniform(0, 1, 8) * 10).astype(np.int64), 9)
    return {"x": x, "t": np.eye(10, dtype=np.float32)[labels]}


# ── the path under test, on any device ──────────────────────────────────────

def run_c1(fg, dev, x):
    t = fg.Tensor.new(x, list(x.shape), dev)
    return t.mul(fg.Tensor.scalar(0.5, dev)).add(fg.Tensor.scalar(1.0, dev)).relu().sum([1]).numpy().reshape(-1)


def run_c2(fg, dev, a, b, c):
    ta, tb, tc = (fg.Tensor.new(v, [v.size], dev) for v in (a, b, c))
    return ta.mul(tb).add(tc).relu().numpy()


def run_c3(fg, dev, x, w, b):
    tx, tw, tb = (fg.Tensor.new(v, list(v.shape), dev) for v in (x, w, b))
    return tx.matmul(tw.permute([1, 0])).add(tb).numpy()


def run_c4(fg, dev, x, t):
    """Returns initial params, loss and params after one step."""
    fg.reset_init_seed(42)
    l1, l2 = fg.Linear(784, 16, dev), fg.Linear(16, 10, dev)
    params = l1.parameters() + l2.parameters()
    p0 = [p.numpy().copy() for p in params]
    opt = fg.Sgd(params, 0.01)
    tx, tt = fg.Tensor.new(x, list(x.shape), dev), fg.Tensor.new(t, list(t.shape), dev)
    loss = l2(l1(tx).relu()).cross_entropy(tt)
    opt.zero_grad()
    loss.backward()
    opt.step()
    return p0, float(loss.to_vec()[0]), [p.numpy() for p in params]


# ── float64 references ──────────────────────────────────────────────────────

def within(got, want, scale, tol):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    return bool(np.all(err <= tol * np.maximum(np.asarray(scale, np.float64), 1e-30)))


def check_c1(inp, out):
    y = np.maximum(inp["x"].astype(np.float64) * 0.5 + 1.0, 0.0)
    assert within(out, y.sum(1), y.sum(1), 1e-5), "c1 vs float64"


def check_c2(inp, out):
    f = np.float32
    a, b, c = inp["a"], inp["b"], inp["c"]
    ab = (a.astype(np.float64) * b).astype(f)          # each op rounded once
    s = (ab.astype(np.float64) + c).astype(f)
    want = np.where(np.float32(0) < s, s, np.float32(0))
    assert np.array_equal(out.view(np.uint32), want.astype(f).view(np.uint32)), "c2 not bit-exact vs IEEE f32"


def check_c3(inp, out):
    x, w, b = (inp[k].astype(np.float64) for k in ("x", "w", "b"))
    scale = np.abs(x) @ np.abs(w).T + np.abs(b)
    assert within(out, x @ w.T + b, scale, 1e-4), "c3 vs float64"


def mlp_step_f64(x, t, p0, lr=0.01):
    """The two-layer step by hand, in float64: loss, params after SGD, the
    gradients, and each gradient's condition scale (the same sum over its
    terms with every input replaced by its absolute value, carried through
    the layers: |x| -> |x|·|W1|ᵀ + |b1| -> ...)."""
    w1, b1, w2, b2 = (p.astype(np.float64) for p in p0)
    x, t = x.astype(np.float64), t.astype(np.float64)
    h_pre = x @ w1.T + b1
    mask = h_pre > 0
    h = np.maximum(h_pre, 0)
    h_s = np.where(mask, np.abs(x) @ np.abs(w1).T + np.abs(b1), 0.0)
    z = h @ w2.T + b2
    zs = z - z.max(1, keepdims=True)
    logp = zs - np.log(np.exp(zs).sum(1, keepdims=True))
    loss = -np.mean((t * logp).sum(1))
    B = x.shape[0]
    dz = (np.exp(logp) - t) / B
    dw2, db2 = dz.T @ h, dz.sum(0)
    dh = (dz @ w2) * mask
    dw1, db1 = dh.T @ x, dh.sum(0)
    dh_s = (np.abs(dz) @ np.abs(w2)) * mask
    grads = [dw1, db1, dw2, db2]
    scales = [dh_s.T @ np.abs(x), dh_s.sum(0), np.abs(dz).T @ h_s, np.abs(dz).sum(0)]
    lr32 = float(np.float32(lr))
    return loss, [p - lr32 * g for p, g in zip((w1, b1, w2, b2), grads)], grads, scales


def check_c4(inp, p0, loss, p1):
    """Loss within 1e-5 relative; each parameter's effective gradient
    (p0 - p1)/lr within 1e-4 of its condition scale plus the roundings of the
    update itself (tests/f64ref.py: sgd_effective_gradient_err)."""
    want_loss, _, grads, scales = mlp_step_f64(inp["x"], inp["t"], p0)
    assert abs(loss - want_loss) <= 1e-5 * abs(want_loss), ("c4 loss", loss, want_loss)
    for name, a, b, g, s in zip(("w1", "b1", "w2", "b2"), p0, p1, grads, scales):
        worst = f64ref.sgd_effective_gradient_err(a, b, g, s)
        assert worst <= 1.0, f"c4 {name}: effective gradient off by {worst:.3g} x bound"


def main():
    import ferrograd_amd as fg
    import oracle

    oracle.load()
    dev = "cpu"
    out = {}
    i1 = c1_inputs(); o1 = run_c1(fg, dev, **i1); check_c1(i1, o1); out["c1_64x64"] = {**i1, "out": o1}
    i2 = c2_inputs(); o2 = run_c2(fg, dev, **i2); check_c2(i2, o2); out["c2_4096"] = {**i2, "out": o2}
    i3 = c3_inputs(); o3 = run_c3(fg, dev, **i3); check_c3(i3, o3); out["c3_64"] = {**i3, "out": o3}
    i4 = c4_inputs()
    p0, loss, p1 = run_c4(fg, dev, **i4)
    check_c4(i4, p0, loss, p1)
    names = ["w1", "b1", "w2", "b2"]
    out["c4_step_b8"] = {**i4, **{n + "_0": p for n, p in zip(names, p0)}, "loss": np.array([loss], np.float32),
                         **{n + "_1": p for n, p in zip(names, p1)}}
    for name, arrays in out.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
