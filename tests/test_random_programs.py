"""Random Tensor programs (tests/randprog.py) against an independent float64
numpy interpreter: on the oracle CPU device, and on HIP. The interpreter
restates each op from the reference's definitions, so this checks the C++
front end (schedule, rangeify, index rules, the HIP fusions) that the oracle
and the HIP path share, not just the kernels."""
from __future__ import annotations

import pytest

import randprog

SEEDS = list(range(80))


@pytest.mark.parametrize("seed", SEEDS)
def test_random_program_on_the_oracle(fg, cpu, seed):
    nodes = randprog.random_program(fg, cpu, seed)
    assert randprog.check(nodes, fg) <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("seed", SEEDS)
def test_random_program_on_hip(fg, hip, seed):
    nodes = randprog.random_program(fg, hip, seed)
    assert randprog.check(nodes, fg) <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("consumer_first", [True, False])
def test_a_reduction_root_read_by_another_root_on_hip(fg, hip, consumer_first):
    # Listed after the root that reads it, a reduction root is inlined into
    # that root's kernel as a nested reduction (schedule.rs:118-133;
    # test_schedule.py::test_roots_are_compiled_in_the_order_given). The
    # oracle cannot emit that kernel; the HIP device folds it serially per
    # output, in the reference's loop order. Both orders against float64.
    import numpy as np

    from conftest import rel_err_bound

    r = np.random.default_rng(3)
    xa = r.uniform(-1, 1, (8, 16)).astype(np.float32)
    wa = r.uniform(-1, 1, (16, 8)).astype(np.float32)
    x = fg.Tensor.new(xa, [8, 16], hip)
    w = fg.Tensor.new(wa, [16, 8], hip)
    s = x.sum([0])
    m = s.matmul(w)
    fg.Tensor.realize_many([m, s] if consumer_first else [s, m])
    x64, w64 = xa.astype(np.float64), wa.astype(np.float64)
    s64 = x64.sum(axis=0, keepdims=True)
    assert rel_err_bound(s.numpy().reshape(1, 16), s64, np.abs(x64).sum(axis=0, keepdims=True), 1e-4) <= 1.0
    assert rel_err_bound(m.numpy().reshape(1, 8), s64 @ w64, np.abs(x64).sum(axis=0, keepdims=True) @ np.abs(w64),
                         1e-4) <= 1.0
