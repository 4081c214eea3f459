"""Realisation-plan replay: a recurring lazy-graph structure replays its
recorded kernels instead of being rescheduled. Replays must be
indistinguishable from scheduling afresh: same results bit for bit, and every
input that changes the schedule (buffer sharing, leaves still holding zeros,
literal values) must select a different plan."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import seeded


@pytest.fixture
def fresh_plans(fg):
    fg.plan_cache(False)
    fg.plan_cache(True)
    yield
    fg.plan_cache(True)


def train(fg, dev, steps, enabled):
    fg.plan_cache(enabled)
    r = seeded(7)
    x = r.uniform(0, 1, (16, 784)).astype(np.float32)
    t = np.eye(10, dtype=np.float32)[np.floor(r.uniform(0, 1, 16) * 10).astype(int)]
    fg.reset_init_seed(42)
    l1, l2 = fg.Linear(784, 32, dev), fg.Linear(32, 10, dev)
    params = l1.parameters() + l2.parameters()
    opt = fg.Sgd(params, 0.01)
    tx, tt = fg.Tensor.new(x, [16, 784], dev), fg.Tensor.new(t, [16, 10], dev)
    losses = []
    for _ in range(steps):
        loss = l2(l1(tx).relu()).cross_entropy(tt)
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.to_vec()[0])
    return losses, [p.numpy() for p in params]


def check_replay_matches_fresh(fg, dev):
    before = fg.plan_stats()["hits"]
    l_on, p_on = train(fg, dev, 4, True)
    hits = fg.plan_stats()["hits"] - before
    l_off, p_off = train(fg, dev, 4, False)
    fg.plan_cache(True)
    assert hits >= 4  # steps 2..4 replay both realisations of the step
    assert l_on == l_off
    for a, b in zip(p_on, p_off):
        assert np.array_equal(a, b)


def test_replayed_train_steps_match_fresh_scheduling(fg, cpu, fresh_plans):
    check_replay_matches_fresh(fg, cpu)


@pytest.mark.gpu
def test_replayed_train_steps_match_fresh_scheduling_hip(fg, hip, fresh_plans):
    check_replay_matches_fresh(fg, hip)


def test_zero_leaf_then_written_selects_new_plan(fg, cpu, fresh_plans):
    x = fg.Tensor.new([1.0, 2.0, 3.0, 4.0], [4], cpu)
    z = fg.Tensor.zeros([4], cpu)
    assert x.add(z).relu().to_vec() == [1.0, 2.0, 3.0, 4.0]  # z folded to a literal 0
    z.assign(fg.Tensor.new([10.0, 20.0, 30.0, 40.0], [4], cpu))
    fg.Tensor.realize_many([z])
    # Same structure over the same buffers, but z no longer holds zeros.
    assert x.add(z).relu().to_vec() == [11.0, 22.0, 33.0, 44.0]


def test_buffer_sharing_is_part_of_the_key(fg, cpu, fresh_plans):
    a = fg.Tensor.new([1.0, 2.0], [2], cpu)
    b = fg.Tensor.new([5.0, 7.0], [2], cpu)
    assert a.mul(a).add(b).to_vec() == [6.0, 11.0]
    assert a.mul(b).add(b).to_vec() == [10.0, 21.0]
    assert b.mul(b).add(a).to_vec() == [26.0, 51.0]  # same sharing as the first: replay, new buffers


def test_new_leaf_values_replay_with_new_buffers(fg, cpu, fresh_plans):
    x = fg.Tensor.new(np.arange(8, dtype=np.float32), [8], cpu)
    outs = []
    for s in (0.5, 2.0, -1.0):
        outs.append(x.mul(fg.Tensor.scalar(s, cpu)).sum([0]).to_vec()[0])
    assert outs == [14.0, 56.0, -28.0]
    assert fg.plan_stats()["hits"] >= 2


def test_narrow_starts_replay_as_kernel_scalars(fg, cpu, fresh_plans):
    # Shrink starts become ParamScalar arguments (schedule.rs:217-239): one
    # plan serves every batch offset and each replay passes the new start.
    x = fg.Tensor.new(np.arange(12, dtype=np.float32).reshape(6, 2), [6, 2], cpu)
    before = fg.plan_stats()["hits"]
    got = [x.narrow(0, s, 2).mul(fg.Tensor.scalar(2.0, cpu)).to_vec() for s in (0, 1, 3, 4)]
    assert got == [[0.0, 2.0, 4.0, 6.0], [4.0, 6.0, 8.0, 10.0], [12.0, 14.0, 16.0, 18.0], [16.0, 18.0, 20.0, 22.0]]
    assert fg.plan_stats()["hits"] - before >= 2


def test_same_inputs_different_ops_select_different_plans(fg, cpu, fresh_plans):
    x = fg.Tensor.new(np.arange(4, dtype=np.float32), [4], cpu)
    assert x.add(x).exp2().to_vec() == [1.0, 4.0, 16.0, 64.0]
    assert x.add(x).log2().to_vec()[1:] == [1.0, 2.0, np.log2(6.0).astype(np.float32)]


def test_disabling_drops_recorded_plans(fg, cpu, fresh_plans):
    x = fg.Tensor.new([1.0], [1], cpu)
    x.add(x).to_vec()
    assert fg.plan_stats()["entries"] >= 1
    fg.plan_cache(False)
    assert fg.plan_stats()["entries"] == 0


@pytest.mark.gpu
def test_graph_replays_match_direct_launches_hip(fg, hip, fresh_plans, graphs):
    # With graphs on, from its second replay a plan runs as one HIP graph.
    # Every step (with the loss read back, i.e. a synchronisation, between
    # replays) must match scheduling afresh with direct launches, bit for bit.
    before = fg.stats()["graph_replays"]
    l_on, p_on = train(fg, hip, 8, True)
    replays = fg.stats()["graph_replays"] - before
    l_off, p_off = train(fg, hip, 8, False)
    fg.plan_cache(True)
    assert replays >= 5
    assert l_on == l_off
    for a, b in zip(p_on, p_off):
        assert np.array_equal(a, b)


@pytest.mark.gpu
def test_graph_replay_with_changing_input_buffers_hip(fg, hip, fresh_plans, graphs):
    # The same two-kernel plan (transpose copy + GEMM with a relu epilogue)
    # over three different input buffers in turn: each replay updates the
    # graph's arguments and is checked against float64.
    r = seeded(3)
    xs_np = [r.standard_normal((64, 96)).astype(np.float32) for _ in range(3)]
    w_np = r.standard_normal((96, 80)).astype(np.float32)
    xs = [fg.Tensor.new(a, [64, 96], hip) for a in xs_np]
    w = fg.Tensor.new(w_np, [96, 80], hip)
    before = fg.stats()["graph_replays"]
    for i in range(9):
        x = xs_np[i % 3].astype(np.float64)
        got = xs[i % 3].matmul(w).relu().numpy().reshape(64, 80)
        want = np.maximum(x @ w_np.astype(np.float64), 0.0)
        scale = np.abs(x) @ np.abs(w_np).astype(np.float64)
        assert np.all(np.abs(got - want) <= 1e-4 * scale + 1e-6), i
    assert fg.stats()["graph_replays"] - before >= 6


@pytest.mark.gpu
def test_steady_state_graph_replays_keep_their_arguments_hip(fg, hip, fresh_plans, graphs):
    # A replayed plan asks the allocator for the blocks its outputs had last
    # time; once the previous step's tensors are gone it gets them back, so the
    # recorded graph launches with no argument updates.
    from ferrograd_amd.mlp import mlp_setup

    step, _ = mlp_setup(fg, hip, batch=64, dims=(784, 64, 10))
    for _ in range(4):
        step()
    s0 = fg.stats()
    for _ in range(6):
        step()
    s1 = fg.stats()
    assert s1["graph_replays"] - s0["graph_replays"] >= 6
    assert s1["graph_updated_launches"] - s0["graph_updated_launches"] == 0


@pytest.mark.gpu
def test_held_intermediate_selects_its_own_plan_hip(fg, hip, fresh_plans):
    # relu(x + y): fused into one kernel while nothing holds x + y; with a
    # tensor at x + y it is materialised (the reference's partition) and that
    # tensor is realised. The two partitions are two plans; each replays.
    x = fg.Tensor.new(np.arange(16, dtype=np.float32) - 8, [16], hip)
    y = fg.Tensor.new(np.full(16, 0.5, np.float32), [16], hip)
    want = np.maximum(np.arange(16, dtype=np.float32) - 7.5, 0)
    # Results are taken outside `assert`: pytest's assertion rewriting keeps
    # every subexpression alive, which would make x + y a held tensor.
    e0 = fg.plan_stats()["entries"]
    free = x.add(y).relu().numpy().reshape(16)
    assert np.array_equal(free, want)
    h = x.add(y)
    held = h.relu().numpy().reshape(16)
    assert np.array_equal(held, want) and h.is_realized()
    assert fg.plan_stats()["entries"] - e0 == 2
    hits = fg.plan_stats()["hits"]
    h2 = x.add(y)
    held2 = h2.relu().numpy().reshape(16)
    assert np.array_equal(held2, want) and h2.is_realized()
    del h, h2
    free2 = x.add(y).relu().numpy().reshape(16)
    assert np.array_equal(free2, want)
    assert fg.plan_stats()["hits"] - hits == 2 and fg.plan_stats()["entries"] - e0 == 2
