"""In-place updates that read their destination at another index, such as
w.assign(w + wᵀ) (Tensor::assign, tensor.rs:421-440; parameterize_store,
schedule.rs:156-170).

The reference compiles such a kernel to nested C loops and calls it once on
one thread (cpu.rs:373-377), so later outputs read values earlier outputs of
the same call have already overwritten. The HIP device runs these kernels in
the `sequential` class: one thread, the reference's loop order, the
innermost output loop in the reference's groups of 4 upcast lanes (each
group's reductions and lane-invariant values evaluated before its first
store). Integer-exact parity: the results are compared bit for bit.

The order itself is pinned on the CPU: the oracle's results equal explicit
Python loops written from that description, for a transpose (where lanes
never read each other), a row sum (each group of 4 reads the row before any
of its stores) and a broadcast column (lanes 1-3 read lane 0's element as it
was before the group)."""
from __future__ import annotations

import numpy as np
import pytest

F = np.float32


def transpose_add_loops(a):
    """w[i][j] = w[i][j] + w[j][i], i then j, each store seen by later reads."""
    e = a.copy()
    n = e.shape[0]
    for i in range(n):
        for j in range(n):
            e[i, j] = F(e[i, j] + e[j, i])
    return e


def grouped(n):
    return n > 4 and n % 4 == 0


def row_sum_loops(a):
    """w[i][:] = sum(w[i][:]) per output; the fold is acc + (((v0+v1)+v2)+v3)
    over groups of 4 terms when the row splits (unroll.rs), else left to
    right. With upcast groups, a group's 4 sums are taken before its stores."""
    e = a.copy()
    n = e.shape[1]

    def rsum(row):
        acc = F(0)
        if grouped(n):
            for k in range(0, n, 4):
                acc = F(acc + F(F(F(row[k] + row[k + 1]) + row[k + 2]) + row[k + 3]))
        else:
            for k in range(n):
                acc = F(acc + row[k])
        return acc

    for i in range(e.shape[0]):
        if grouped(n):
            for g in range(0, n, 4):
                s = rsum(e[i])
                e[i, g:g + 4] = s
        else:
            for j in range(n):
                e[i, j] = rsum(e[i])
    return e


def first_column_loops(a):
    """w[i][j] = w[i][j] + w[i][0]; within a group of 4 lanes, w[i][0] is
    read once before the group's first store."""
    e = a.copy()
    n = e.shape[1]
    for i in range(e.shape[0]):
        if grouped(n):
            for g in range(0, n, 4):
                c = e[i, 0]
                for u in range(4):
                    e[i, g + u] = F(e[i, g + u] + c)
        else:
            for j in range(n):
                e[i, j] = F(e[i, j] + e[i, 0])
    return e


def _transpose_add(fg, w, n, dev, x):
    return w.add(w.permute([1, 0]))


def _row_sum(fg, w, n, dev, x):
    return w.sum([1]).expand([n, n])


def _first_column(fg, w, n, dev, x):
    return w.add(w.narrow(1, 0, 1).expand([n, n]))


def _first_row_product(fg, w, n, dev, x):
    return w.mul(w.narrow(0, 0, 1).expand([n, n]))


def _matmul(fg, w, n, dev, x):
    return w.matmul(fg.Tensor.new(x, [n, n], dev))


def _relu_half(fg, w, n, dev, x):
    # relu reads its input twice, so the reference materialises w + wᵀ first
    # (from the old w) and the in-place kernel reads it at its own index: not
    # a sequential kernel, and the fusions must not make it one.
    return w.add(w.permute([1, 0])).relu().mul(fg.Tensor.scalar(0.5, dev))


def _shifted_rows(fg, w, n, dev, x):
    # Row i reads rows i and (0-th) through a narrow of the same buffer.
    return w.narrow(0, 0, 1).expand([n, n]).sub(w).mul(w.permute([1, 0]))


PROGRAMS = {
    "transpose_add": (_transpose_add, transpose_add_loops),
    "row_sum": (_row_sum, row_sum_loops),
    "first_column": (_first_column, first_column_loops),
    "first_row_product": (_first_row_product, None),
    "matmul": (_matmul, None),
    "relu_half": (_relu_half, None),
    "shifted_rows": (_shifted_rows, None),
}
SIZES = [2, 6, 8, 12]


def run(fg, dev, name, n, seed=0):
    r = np.random.default_rng(seed + n)
    a = r.uniform(-1, 1, (n, n)).astype(F)
    x = r.uniform(-1, 1, (n, n)).astype(F)
    w = fg.Tensor.new(a, [n, n], dev)
    w.assign(PROGRAMS[name][0](fg, w, n, dev, x))
    w.realize()
    return a, w.numpy().reshape(n, n)


@pytest.mark.parametrize("name", sorted(PROGRAMS))
def test_in_place_kernel_is_sequential_and_compiles(fg, cpu, name):
    from hipcompile import compile_sources

    n = 8
    w = fg.Tensor.new(np.zeros((n, n), F), [n, n], cpu)
    w.assign(PROGRAMS[name][0](fg, w, n, cpu, np.ones((n, n), F)))
    items = fg.debug_plan([w], fuse=True, render_hip=True)["items"]
    seq = [it for it in items if it["class"] == "sequential"]
    if name == "relu_half":
        assert not seq, [it["class"] for it in items]
    else:
        assert len(seq) == 1 and seq[0]["grid"] == [1, 1, 1], [it["class"] for it in items]
        assert seq[0]["name"].endswith("_seq")
    compile_sources({it["source"]: it["name"] for it in items}, limit_s=120)


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("name", [k for k, v in PROGRAMS.items() if v[1]])
def test_oracle_order_matches_the_loops(fg, cpu, name, n):
    a, got = run(fg, cpu, name, n)
    assert np.array_equal(got, PROGRAMS[name][1](a))


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("name", sorted(PROGRAMS))
def test_hip_schedule_fusions_keep_the_in_place_bits(fg, cpu, name, n):
    # The oracle device with the HIP device's schedule-time fusions on
    # computes the same bits as with the reference partition.
    import oracle

    a0, plain = run(fg, cpu, name, n)
    oracle.set_fuse(True)
    try:
        a1, fused = run(fg, cpu, name, n)
    finally:
        oracle.set_fuse(False)
    assert np.array_equal(a0, a1) and np.array_equal(plain, fused)


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("name", sorted(PROGRAMS))
def test_in_place_update_on_hip_matches_the_oracle(fg, cpu, hip, name, n):
    print(f"in-place {name} n={n}", flush=True)
    _, want = run(fg, cpu, name, n)
    _, got = run(fg, hip, name, n)
    assert np.array_equal(got, want), float(np.max(np.abs(got.astype(np.float64) - want)))


@pytest.mark.gpu
def test_in_place_update_replayed_on_hip(fg, cpu, hip):
    # The same in-place program three times: recorded, then replayed twice
    # from the plan cache; each call continues from the previous one's result.
    print("in-place transpose_add replayed", flush=True)
    n = 12
    a = np.random.default_rng(9).uniform(-1, 1, (n, n)).astype(F)
    outs = {}
    for dev in ("cpu", "hip"):
        w = fg.Tensor.new(a, [n, n], dev)
        res = []
        for _ in range(3):
            w.assign(w.add(w.permute([1, 0])))
            w.realize()
            res.append(w.numpy().reshape(n, n).copy())
        outs[dev] = res
    e = a
    for k in range(3):
        e = transpose_add_loops(e)
        assert np.array_equal(outs["cpu"][k], e) and np.array_equal(outs["hip"][k], e), k


def random_in_place(fg, dev, seed):
    """w.assign(e(w)) for a random elementwise expression e over views of w
    itself (its transpose, a broadcast row or column of it, a narrowed
    window) and other leaves, realised twice in a row. Elementwise ops round
    the same way on both devices, so whatever partition and order the
    schedule gives, the sequential kernels must reproduce the oracle's bits.
    Returns the two results."""
    r = np.random.default_rng(seed)
    n = int(r.choice([3, 4, 5, 8, 12]))
    m = n if r.random() < 0.6 else int(r.choice([4, 6, 8]))
    a = r.uniform(-1, 1, (n, m)).astype(F)
    w = fg.Tensor.new(a, [n, m], dev)
    others = [fg.Tensor.new(r.uniform(-1, 1, (n, m)).astype(F), [n, m], dev) for _ in range(2)]
    outs = []
    for _ in range(2):
        def view():
            k = int(r.integers(5 if n == m else 4))
            if k == 0:
                return w
            if k == 1:
                i = int(r.integers(n))
                return w.narrow(0, i, 1).expand([n, m])
            if k == 2:
                j = int(r.integers(m))
                return w.narrow(1, j, 1).expand([n, m])
            if k == 3:
                return others[int(r.integers(2))]
            return w.permute([1, 0])
        e = view()
        for _ in range(int(r.integers(1, 4))):
            op = int(r.integers(5))
            if op == 0:
                e = e.add(view())
            elif op == 1:
                e = e.mul(view())
            elif op == 2:
                e = e.relu()
            elif op == 3:
                e = e.mul(fg.Tensor.scalar(float(r.choice([0.5, -1.5, 0.25])), dev))
            else:
                e = e.sub(view())
        w.assign(e)
        w.realize()
        outs.append(w.numpy().reshape(n, m).copy())
    return outs


@pytest.mark.parametrize("seed", range(40))
def test_random_in_place_programs_keep_their_bits_under_the_fusions(fg, cpu, seed):
    import oracle

    plain = random_in_place(fg, cpu, seed)
    oracle.set_fuse(True)
    try:
        fused = random_in_place(fg, cpu, seed)
    finally:
        oracle.set_fuse(False)
    for p, q in zip(plain, fused):
        assert np.array_equal(p, q)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(40))
def test_random_in_place_programs_on_hip(fg, cpu, hip, seed):
    print(f"random in-place program {seed}", flush=True)
    want = random_in_place(fg, cpu, seed)
    got = random_in_place(fg, hip, seed)
    for g, w in zip(got, want):
        assert np.array_equal(g, w), float(np.max(np.abs(g.astype(np.float64) - w)))
