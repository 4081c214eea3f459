"""Shared test setup: the `gpu` marker, the oracle CPU device and helpers."""
from __future__ import annotations

import contextlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def fg():
    import ferrograd_amd

    ferrograd_amd.lib()
    return ferrograd_amd


@pytest.fixture(scope="session")
def cpu(fg):
    """Registers the oracle's CPU device ("cpu") and returns its device name."""
    import oracle

    oracle.load()
    return "cpu"


@pytest.fixture(scope="session")
def hip(fg):
    """The HIP device name. Opens the device's HIP context first and fails
    with the runtime's error when the native HIP path is unusable."""
    from ferrograd_amd.hip import Context

    try:
        Context.of_device().info()
    except Exception as e:  # noqa: BLE001
        pytest.fail(f"HIP device unusable: {e}")
    return "hip"


def seeded(seed: int):
    return np.random.default_rng(seed)


def rel_err_bound(got: np.ndarray, want: np.ndarray, scale: np.ndarray, tol: float) -> float:
    """max |got-want| / (tol * scale) — <= 1 passes (scale = sum |terms|)."""
    denom = np.maximum(scale.astype(np.float64), np.finfo(np.float32).tiny) * tol
    return float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)) / denom))


def recorded_steps(fg, dev, xs, ts, dims, steps=1, starts=None, batch=None, lr=0.01, seed=42):
    """`steps` SGD train steps of an MLP with layer widths `dims` (with
    `starts`, step i trains on rows [starts[i], starts[i] + batch) through
    narrow(), the batching of examples/mnist.rs:46-62). Each step holds its
    pre-activations; returns per step what f64ref.check_mlp_step takes:
    (x, t, p0, p1, loss, hidden pre-activations, logits)."""
    from ferrograd_amd.mlp import Mlp, train_step

    fg.reset_init_seed(seed)
    model = Mlp(dims, dev)
    params = model.parameters()
    opt = fg.Sgd(params, lr)
    tx = fg.Tensor.new(xs, list(xs.shape), dev)
    tt = fg.Tensor.new(ts, list(ts.shape), dev)
    out = []
    for i in range(steps if starts is None else len(starts)):
        x = tx if starts is None else tx.narrow(0, starts[i], batch)
        t = tt if starts is None else tt.narrow(0, starts[i], batch)
        hx = xs if starts is None else xs[starts[i]:starts[i] + batch]
        ht = ts if starts is None else ts[starts[i]:starts[i] + batch]
        p0 = [p.numpy().copy() for p in params]
        zs = []
        loss = train_step(model, opt, x, t, zs).to_vec()[0]
        B = hx.shape[0]
        out.append((hx, ht, p0, [p.numpy() for p in params], loss, [z.numpy().reshape(B, -1) for z in zs[:-1]],
                    zs[-1].numpy().reshape(B, -1)))
    return out


def check_recorded_steps(steps, lr=0.01):
    """Every recorded step, product by product against float64
    (f64ref.check_mlp_step); returns the losses."""
    import f64ref

    for i, (x, t, p0, p1, loss, hidden, logits) in enumerate(steps):
        rep = f64ref.check_mlp_step(x, t, p0, p1, loss, hidden, logits, lr)
        assert rep["ok"], (i, rep)
    return [s[4] for s in steps]


@contextlib.contextmanager
def graphs_on(fg, n=2):
    """HIP-graph replay of sequences of `n` or more launches (the device's
    default launches them one by one), restored afterwards."""
    prev = fg.graph_min_launches(n)
    try:
        yield
    finally:
        fg.graph_min_launches(prev)


@pytest.fixture
def graphs(fg):
    with graphs_on(fg):
        yield
