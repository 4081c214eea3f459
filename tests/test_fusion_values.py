"""The HIP schedule's fusions leave every value unchanged.

The oracle CPU device can schedule with the HIP device's fusions
(`oracle.set_fuse`). Fused and reference partitions then run on one device
with the same lowering, so each program below must give the same bits both
ways. The cases are the fusion rules of ferrograd_amd/csrc/schedule.cpp,
alone and around in-place stores in the same realize_many (the reference
materialises shared nodes and ALU-consumed reduces in phase 1, before any
root's store, schedule.rs:88-121), and the benchmark programs."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import seeded


@pytest.fixture
def fused(cpu):
    import oracle

    yield lambda on: oracle.set_fuse(on)
    oracle.set_fuse(False)


def both_partitions(fused, fn):
    """fn(device) with the reference partition, then with the fused one."""
    out = []
    for on in (False, True):
        fused(on)
        out.append(fn("cpu"))
    return out


def assert_same_bits(a, b):
    if isinstance(a, (list, tuple)):
        assert len(a) == len(b)
        for x, y in zip(a, b):
            assert_same_bits(x, y)
        return
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def store_then(fg, dev, build, store_first=True):
    """realize_many over w.assign(w + 1) and y = build(w), in either order;
    returns (y, w)."""
    ws = np.linspace(-2.0, 3.0, 80, dtype=np.float32).reshape(8, 10)
    w = fg.Tensor.new(ws, [8, 10], dev)
    y = build(fg, dev, w)
    w.assign(w.add(fg.Tensor.scalar(1.0, dev)))
    fg.Tensor.realize_many([w, y] if store_first else [y, w])
    return y.numpy(), w.numpy()


READERS = {
    # A reduce consumed by ALU: deferred into its consumer's kernel as an epilogue.
    "reduce_epilogue": lambda fg, d, w: w.sum([0]).mul(fg.Tensor.scalar(2.0, d)),
    # A reduction over 10 elements: recomputed by each consumer.
    "small_reduce": lambda fg, d, w: w.max([1]).mul(fg.Tensor.scalar(2.0, d)).expand([8, 10]).add(w),
    # One op over one loaded value, read by two consumers: recomputed.
    "cheap_node": lambda fg, d, w: (lambda c: c.add(fg.Tensor.scalar(1.0, d)).mul(c.sum([1]).expand([8, 10])))(
        w.mul(fg.Tensor.scalar(3.0, d))),
    # exp(w) feeds two nodes that reconverge in one: inlined.
    "reconverging": lambda fg, d, w: (lambda e: e.add(e.mul(e)))(w.exp()),
    # matmul's identity copy of w: read in place.
    "identity_copy": lambda fg, d, w: fg.Tensor.new(np.ones((4, 10), np.float32), [4, 10], d).matmul(
        w.permute([1, 0])),
}


@pytest.mark.parametrize("store_first", [True, False])
@pytest.mark.parametrize("reader", sorted(READERS))
def test_fused_node_read_around_an_in_place_store(fg, fused, reader, store_first):
    ref, got = both_partitions(fused, lambda d: store_then(fg, d, READERS[reader], store_first))
    assert_same_bits(ref, got)


def test_reduce_read_after_store_uses_the_old_values(fg, fused):
    # The reference's answer, by hand: y = 2 * column sums of w before w += 1.
    fused(True)
    y, w = store_then(fg, "cpu", READERS["reduce_epilogue"])
    ws = np.linspace(-2.0, 3.0, 80, dtype=np.float32).reshape(8, 10)
    np.testing.assert_allclose(y.reshape(-1), 2 * ws.sum(0), rtol=1e-6)
    assert np.array_equal(w, ws + np.float32(1.0))


def test_benchmark_programs(fg, fused):
    r = seeded(21)
    x = r.standard_normal((64, 96)).astype(np.float32)
    a, b, c = (r.uniform(-1, 1, 1000).astype(np.float32) for _ in range(3))
    w = r.uniform(-1 / 64, 1 / 64, (48, 96)).astype(np.float32)
    bias = r.standard_normal(48).astype(np.float32)

    def run(d):
        T = lambda v: fg.Tensor.new(v, list(v.shape), d)
        c1 = T(x).mul(fg.Tensor.scalar(0.5, d)).add(fg.Tensor.scalar(1.0, d)).relu().sum([1]).numpy()
        c2 = T(a).mul(T(b)).add(T(c)).relu().numpy()
        c3 = T(x).matmul(T(w).permute([1, 0])).add(T(bias)).numpy()
        return [c1, c2, c3]

    ref, got = both_partitions(fused, run)
    assert_same_bits(ref, got)


@pytest.mark.parametrize("hidden", [(16,), (24, 20)])
def test_mlp_train_steps(fg, fused, hidden):
    from ferrograd_amd.mlp import Mlp, synthetic_batch, train_step

    xs, ts = synthetic_batch(12, 40, 10, 3, 4)

    def run(d):
        fg.reset_init_seed(42)
        model = Mlp((40,) + hidden + (10,), d)
        opt = fg.Sgd(model.parameters(), 0.01)
        x, t = fg.Tensor.new(xs, list(xs.shape), d), fg.Tensor.new(ts, list(ts.shape), d)
        losses = [train_step(model, opt, x, t).to_vec()[0] for _ in range(3)]
        return [np.array(losses, np.float32)] + [p.numpy() for p in model.parameters()]

    ref, got = both_partitions(fused, run)
    assert_same_bits(ref, got)
