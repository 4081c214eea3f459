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


@pytest.mark.parametrize("seed", SEEDS)
def test_random_program_renders_for_hip(fg, cpu, seed):
    # Every kernel of the program through the HIP lowering and renderer, on
    # the CPU: a program the renderer cannot emit fails here without a GPU.
    nodes = randprog.random_program(fg, cpu, seed)
    fg.debug_plan([n.t for n in nodes], fuse=True, render_hip=True)


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


@pytest.mark.gpu
def test_a_sum_over_a_unit_axis_on_hip(fg, hip):
    # All of the reduction's ranges have extent 1: the lowering drops them and
    # the small-kernel body folds one term per output.
    import numpy as np

    xa = np.random.default_rng(5).uniform(-1, 1, (32, 1)).astype(np.float32)
    y = fg.Tensor.new(xa, [32, 1], hip).sum([1])
    z = y.narrow(0, 26, 4)
    fg.Tensor.realize_many([y, z])
    assert np.array_equal(y.numpy().reshape(32, 1), xa)
    assert np.array_equal(z.numpy().reshape(4, 1), xa[26:30])


@pytest.mark.gpu
def test_a_row_reduction_summed_again_over_its_axis_on_hip(fg, hip):
    # sum(log_softmax(x, 1)) feeding a matmul: the kernel of the sum inlines
    # the row sum of exp into a reduction over the same axis. Rangeify gives
    # both the one range of that axis, the inner loop shadowing the outer; the
    # lowering renames it, and the outer reduction's unrolled lanes are
    # emitted one at a time around the inner one.
    import numpy as np

    from conftest import rel_err_bound

    r = np.random.default_rng(6)
    xa = r.uniform(-1, 1, (16, 8)).astype(np.float32)
    wa = r.uniform(-1, 1, (1, 8)).astype(np.float32)
    x = fg.Tensor.new(xa, [16, 8], hip)
    w = fg.Tensor.new(wa, [1, 8], hip)
    ls = x.log_softmax(1)
    m = ls.sum([0, 1]).matmul(w)
    fg.Tensor.realize_many([ls, m])
    x64 = xa.astype(np.float64)
    z = x64 - x64.max(axis=1, keepdims=True)
    want = z - np.log(np.exp(z).sum(axis=1, keepdims=True))
    assert rel_err_bound(ls.numpy().reshape(16, 8), want, np.full((16, 8), 4.0), 1e-4) <= 1.0
    mag = 4.0 * 128 * np.abs(wa.astype(np.float64))
    assert rel_err_bound(m.numpy().reshape(1, 8), want.sum() * wa.astype(np.float64), mag, 1e-4) <= 1.0


LARGE_SEEDS = list(range(60))


@pytest.mark.parametrize("seed", LARGE_SEEDS)
def test_large_random_program_on_the_oracle(fg, cpu, seed):
    nodes = randprog.random_program(fg, cpu, seed, large=True)
    fg.debug_plan([n.t for n in nodes], fuse=True, render_hip=True)
    assert randprog.check(nodes, fg) <= 1.0


def serial_max_nest_program(fg, dev):
    """The program that stalled a GPU run: max over axes [1,2,3] of
    f32[6,8,10,12] (a one-workgroup kernel that folds 960 terms per output
    serially: a for 8 x for 10 x for 3 nest of float4 compare-selects), relu,
    two permutes, a product with a broadcast sum, and a max over every axis,
    realised as three roots (five block kernels). Left to unroll the whole
    nest, hiprtc at -O3 never finished compiling its first kernel."""
    import numpy as np

    rng = np.random.default_rng(1085)
    x = randprog.leaf(fg, dev, rng, (6, 8, 10, 12))
    z = randprog.leaf(fg, dev, rng, (1, 1, 1, 6))
    N = randprog.Node
    mx = N(x.t.max([1, 2, 3]), x.v.max(axis=(1, 2, 3), keepdims=True), x.m.max(axis=(1, 2, 3), keepdims=True))
    rl = N(mx.t.relu(), np.where(0 < mx.v, mx.v, 0.0), mx.m)
    p1 = N(rl.t.permute([1, 2, 0, 3]), rl.v.transpose(1, 2, 0, 3), rl.m.transpose(1, 2, 0, 3))
    p2 = N(mx.t.permute([2, 1, 3, 0]), mx.v.transpose(2, 1, 3, 0), mx.m.transpose(2, 1, 3, 0))
    zs = z.t.sum([1, 2, 3])
    zv, zm = z.v.sum(axis=(1, 2, 3), keepdims=True), z.m.sum(axis=(1, 2, 3), keepdims=True)
    pr = N(p2.t.mul(zs.expand([1, 1, 1, 6])), p2.v * zv, p2.m * zm)
    am = N(rl.t.max([0, 1, 2, 3]), rl.v.max(keepdims=True), rl.m.max(keepdims=True))
    return [p1, pr, am]


def test_serial_max_nest_compiles_in_seconds(fg, cpu):
    # Every kernel of the program, compiled for gfx950 in child processes
    # against a fresh cache: each serial fold's loops carry unroll bounds, so
    # the whole plan compiles within the minute (about a second per kernel).
    from hipcompile import compile_sources

    nodes = serial_max_nest_program(fg, cpu)
    items = fg.debug_plan([n.t for n in nodes], fuse=True, render_hip=True)["items"]
    assert [it["class"] for it in items] == ["block"] * 5
    assert "for (int ridx" in items[0]["source"] and "#pragma unroll 1" in items[0]["source"]
    compile_sources({it["source"]: it["name"] for it in items}, limit_s=60)
    assert randprog.check(nodes, fg) <= 1.0


@pytest.mark.gpu
def test_serial_max_nest_on_hip(fg, hip):
    print("serial max nest program on hip", flush=True)
    nodes = serial_max_nest_program(fg, hip)
    assert randprog.check(nodes, fg) <= 1.0


def test_every_random_program_compiles_for_gfx950(fg, cpu):
    # Every kernel of every random program the HIP tests run (small, large,
    # and the gradient programs' forward graphs), rendered and compiled
    # compile-only on the CPU, 8 at a time, within a time limit: a kernel
    # hiprtc cannot compile, or cannot compile in finite time, fails here
    # without a GPU.
    from hipcompile import compile_sources

    sources = {}
    programs = [(s, False) for s in SEEDS] + [(s, True) for s in LARGE_SEEDS + list(range(1000, 1140))]
    programs += [(s, False) for s in range(60)] + [(s, True) for s in range(2000, 2040)]
    programs += [(s, "odd") for s in range(3000, 3040)]
    for seed, large in programs:
        if large == "odd":
            nodes = randprog.random_program(fg, cpu, seed, odd=True)
        else:
            nodes = randprog.random_program(fg, cpu, seed, large=large)
        for it in fg.debug_plan([n.t for n in nodes], fuse=True, render_hip=True)["items"]:
            sources[it["source"]] = it["name"]
    timings = compile_sources(sources, limit_s=300)
    assert len(timings) == len(sources) and timings[0][1] < 30, timings[:3]


@pytest.mark.gpu
@pytest.mark.parametrize("seed", LARGE_SEEDS + list(range(1000, 1140)))
def test_large_random_program_on_hip(fg, hip, seed):
    # Shapes above the small-kernel limits: row and column reductions,
    # elementwise kernels and MFMA GEMMs, as well as block kernels.
    nodes = randprog.random_program(fg, hip, seed, large=True)
    assert randprog.check(nodes, fg) <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("seed,large", [(s, False) for s in SEEDS] + [(s, True) for s in LARGE_SEEDS])
def test_random_program_replayed_on_hip(fg, hip, seed, large):
    # The same program four times, each against float64: scheduled and run
    # kernel by kernel, then replayed from the plan cache (runs of block
    # kernels batched with their stage outputs handed on through LDS,
    # adjacent independent small GEMMs paired or run beside a batch, all
    # built on this replay), then with graphs on recorded as one HIP graph
    # and replayed through it.
    from conftest import graphs_on

    print(f"random program {seed} (large={large}) four times", flush=True)
    before = fg.plan_stats()["hits"]
    for rep in range(4):
        with graphs_on(fg, 2 if rep >= 2 else 0):
            nodes = randprog.random_program(fg, hip, seed, large=large)
            assert randprog.check(nodes, fg) <= 1.0, rep
    assert fg.plan_stats()["hits"] - before >= 3


def _program_gradients(fg, dev, seed, large):
    """d(sum of the last node)/d(each leaf), as float64 arrays."""
    import numpy as np

    leaves = []
    if large == "odd":
        nodes = randprog.random_program(fg, dev, seed, odd=True, leaves=leaves)
    else:
        nodes = randprog.random_program(fg, dev, seed, large=large, leaves=leaves)
    last = nodes[-1].t
    loss = last.sum(list(range(len(last.shape))))
    grads = loss.gradient([n.t for n in leaves])
    fg.Tensor.realize_many(grads)
    return [g.numpy().astype(np.float64).reshape(n.v.shape) for g, n in zip(grads, leaves)]


@pytest.mark.gpu
@pytest.mark.parametrize("seed,large", [(s, False) for s in range(60)] + [(s, True) for s in range(2000, 2040)] +
                         [(s, "odd") for s in range(3000, 3020)])
def test_random_program_gradients_on_hip_match_the_oracle(fg, cpu, hip, seed, large):
    # The backward graphs (expand-sums, relu and max masks, matmul
    # transposes, log_softmax's) of the random programs: HIP against the
    # oracle device, leaf by leaf, each element within 1e-4 of its own leaf's
    # largest gradient element, plus 1e-6 of the largest over all leaves (so
    # a leaf whose gradient is all but zero is still held to that). Both
    # share the front end; this checks the HIP kernels, fusions and batches
    # that run the backward.
    import numpy as np

    print(f"gradients of random program {seed} (large={large})", flush=True)
    want = _program_gradients(fg, cpu, seed, large)
    got = _program_gradients(fg, hip, seed, large)
    top = max([float(np.abs(w).max()) for w in want] + [1e-30])
    for i, (g, w) in enumerate(zip(got, want)):
        leaf = float(np.abs(w).max())
        bound = 1e-4 * leaf + 1e-6 * top
        assert np.all(np.abs(g - w) <= bound), (seed, i, float(np.max(np.abs(g - w))), leaf, top)


ODD_SEEDS = list(range(3000, 3040))


@pytest.mark.parametrize("seed", ODD_SEEDS)
def test_odd_shaped_random_program_on_the_oracle(fg, cpu, seed):
    nodes = randprog.random_program(fg, cpu, seed, odd=True)
    fg.debug_plan([n.t for n in nodes], fuse=True, render_hip=True)
    assert randprog.check(nodes, fg) <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("seed", ODD_SEEDS)
def test_odd_shaped_random_program_on_hip(fg, hip, seed):
    # Unit axes and ragged extents: every class's edge handling (clamped
    # loads, partial tiles, partial lanes), twice (scheduled, then replayed).
    print(f"odd-shaped random program {seed}", flush=True)
    for _ in range(2):
        nodes = randprog.random_program(fg, hip, seed, odd=True)
        assert randprog.check(nodes, fg) <= 1.0
