"""Pins the oracle (the restated reference CPU backend) before it is trusted:
against the reference's own known answers and against what the mathematics
fixes (float64 brute force, closed forms, per-op IEEE rounding), chosen so a
dropped term, swapped operand or wrong index fails. CPU only."""
import math

import numpy as np
import pytest

from conftest import rel_err_bound, seeded


# ── the reference's tensor known answers (src/tensor.rs:1133-1313) ─────────
def test_known_answers(fg, cpu):
    T = fg.Tensor
    assert T.new([1.0, 2.0, 3.0], [3], cpu).add(T.new([4.0, 5.0, 6.0], [3], cpu)).to_vec() == [5.0, 7.0, 9.0]
    assert T.new([2.0, 3.0, 4.0], [3], cpu).mul(T.new([5.0, 6.0, 7.0], [3], cpu)).to_vec() == [10.0, 18.0, 28.0]
    assert T.new([1.0, -2.0, 3.0, -4.0], [4], cpu).relu().to_vec() == [1.0, 0.0, 3.0, 0.0]
    ls = T.new([0.0, 1.0], [1, 2], cpu).log_softmax(1).to_vec()
    assert abs(ls[0] + 1.3132616) < 1e-5 and abs(ls[1] + 0.31326166) < 1e-5
    ce = T.new([2.0, 0, 0, 2.0], [2, 2], cpu).cross_entropy(T.new([1.0, 0, 0, 1.0], [2, 2], cpu)).to_vec()[0]
    assert abs(ce - 0.12692805) < 1e-5
    x = T.new([1.0, 2, 3, 4, 5, 6], [2, 3], cpu)
    assert x.sum([0]).to_vec() == [5.0, 7.0, 9.0]
    assert x.narrow(0, 1, 1).to_vec() == [4.0, 5.0, 6.0]
    assert x.permute([1, 0]).contiguous().to_vec() == [1.0, 4.0, 2.0, 5.0, 3.0, 6.0]


def test_gradient_known_answers(fg, cpu):  # tensor.rs:1219-1276
    T = fg.Tensor
    x = T.new([1.0, 2, 3, 4], [2, 2], cpu).narrow(0, 1, 1)
    w = T.new([10.0, 20.0], [2, 1], cpu).with_requires_grad(True)
    assert x.matmul(w).sum([0, 1]).gradient([w])[0].to_vec() == [3.0, 4.0]
    a = T.new([3.0], [1], cpu).with_requires_grad(True)
    b = T.new([5.0], [1], cpu).with_requires_grad(True)
    a.mul(b).sum([0]).backward()
    assert a.grad().to_vec() == [5.0] and b.grad().to_vec() == [3.0]


def test_sgd_closed_form(fg, cpu):  # optim.rs:81-94: p=3, t=2, lr=0.1 -> 3 - 0.1*2*(3-2) = 2.8
    p = fg.Tensor.new([3.0], [1], cpu).with_requires_grad(True)
    t = fg.Tensor.new([2.0], [1], cpu)
    loss = p.sub(t).mul(p.sub(t)).sum([0])
    opt = fg.Sgd([p], 0.1)
    opt.zero_grad()
    loss.backward()
    opt.step()
    assert abs(p.to_vec()[0] - 2.8) < 1e-6


def test_demo_closed_form(fg, cpu):  # examples/demo.rs:17-30
    T = fg.Tensor
    x = T.new([1.0, 2.0, 3.0, 4.0], [2, 2], cpu)
    w = T.new([0.1, 0.2, 0.3, 0.4], [2, 2], cpu).with_requires_grad(True)
    b = T.new([0.5, 0.6], [1, 2], cpu).with_requires_grad(True)
    loss = x.matmul(w).add(b).sum([0, 1])
    loss.backward()
    assert abs(loss.to_vec()[0] - 7.6) < 1e-5
    np.testing.assert_allclose(w.grad().to_vec(), [4, 4, 6, 6], rtol=1e-6)
    np.testing.assert_allclose(b.grad().to_vec(), [2, 2], rtol=1e-6)
    fg.Sgd([w], 0.1).step()
    np.testing.assert_allclose(w.to_vec(), [-0.3, -0.2, -0.3, -0.2], atol=1e-6)


def test_loss_realised_before_backward_detaches_graph(fg, cpu):
    # tensor.rs:222-252 rewrites the realised loss to its buffer, so a
    # backward() after to_vec() finds no parameters (as the reference does).
    x = fg.Tensor.new([1.0, 2.0], [1, 2], cpu)
    w = fg.Tensor.new([1.0, 1.0], [2, 1], cpu).with_requires_grad(True)
    loss = x.matmul(w).sum([0, 1])
    loss.to_vec()
    loss.backward()
    assert w.grad() is None


# ── what the mathematics fixes ─────────────────────────────────────────────
def test_c2_per_op_rounding(fg, cpu):
    # (a*b + c).relu() with each op rounded once in f32 equals numpy's f32
    # arithmetic bit for bit (a fused multiply-add or reordering would not).
    r = seeded(2)
    a, b, c = (r.uniform(-1, 1, 4097).astype(np.float32) for _ in range(3))
    T = fg.Tensor
    got = T.new(a, [4097], cpu).mul(T.new(b, [4097], cpu)).add(T.new(c, [4097], cpu)).relu().numpy()
    want = np.maximum(np.float32(0), (a * b) + c)
    want = np.where(np.float32(0) < (a * b) + c, (a * b) + c, np.float32(0)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("shape", [(64, 64), (5, 12), (33, 7)])
def test_c1_against_float64(fg, cpu, shape):
    x = seeded(1).standard_normal(shape).astype(np.float32)
    T = fg.Tensor
    got = T.new(x, list(shape), cpu).mul(T.scalar(0.5, cpu)).add(T.scalar(1.0, cpu)).relu().sum([1]).numpy()[:, 0]
    y = np.maximum((x * np.float32(0.5)) + np.float32(1.0), 0).astype(np.float64)
    assert rel_err_bound(got, y.sum(1), np.abs(y).sum(1), 1e-5) <= 1.0


def test_c1_sum_order_is_reference_unroll_fold(fg, cpu):
    # 8-wide rows: REDUCE(2) x UNROLL(4) and acc + (((v0+v1)+v2)+v3).
    v = np.array([[1e8, 1.0, -1e8, 1.0, 3.0, 5.0, 7.0, 0.5]], np.float32)
    got = fg.Tensor.new(v, [1, 8], cpu).sum([1]).numpy()[0, 0]
    f = np.float32
    g0 = ((f(1e8) + f(1.0)) + f(-1e8)) + f(1.0)
    g1 = ((f(3.0) + f(5.0)) + f(7.0)) + f(0.5)
    assert got == (f(0.0) + g0) + g1


@pytest.mark.parametrize("mnk", [(8, 6, 4), (16, 16, 784 // 16), (3, 5, 7)])
def test_c3_against_float64(fg, cpu, mnk):
    m, n, k = mnk
    r = seeded(5)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = r.uniform(-1, 1, (n, k)).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32)
    T = fg.Tensor
    got = T.new(x, [m, k], cpu).matmul(T.new(w, [n, k], cpu).permute([1, 0])).add(T.new(b, [n], cpu)).numpy()
    want = x.astype(np.float64) @ w.T.astype(np.float64) + b
    scale = np.abs(x).astype(np.float64) @ np.abs(w).T + np.abs(b)
    assert rel_err_bound(got, want, scale, 1e-5) <= 1.0
    # A transposed operand would fail: x@w (not w^T) differs grossly.
    if m == n == k:
        assert not np.allclose(got, x @ w + b, rtol=1e-3)


def test_column_reduction_with_upcast_and_unroll(fg, cpu):
    # [8,8].sum(0): the output axis is upcast and the reduce axis unrolled.
    # The oracle folds along the reduced axis (the mathematical column sum).
    v = np.arange(64, dtype=np.float32).reshape(8, 8)
    got = fg.Tensor.new(v, [8, 8], cpu).sum([0]).numpy()[0]
    assert got.tolist() == v.sum(0).tolist()


def test_log_softmax_cross_entropy_float64(fg, cpu):
    r = seeded(11)
    z = r.standard_normal((16, 10)).astype(np.float32) * 3
    t = np.eye(10, dtype=np.float32)[r.integers(0, 10, 16)]
    T = fg.Tensor
    got = T.new(z, [16, 10], cpu).cross_entropy(T.new(t, [16, 10], cpu)).to_vec()[0]
    z64 = z.astype(np.float64)
    lse = np.log(np.exp(z64 - z64.max(1, keepdims=True)).sum(1)) + z64.max(1)
    want = float(np.mean(lse - (z64 * t).sum(1)))
    assert abs(got - want) <= 1e-5 * max(1.0, abs(want))


_MASK64 = (1 << 64) - 1


def _lcg_draw(n: int, seed: int = 42) -> float:
    """The n-th (1-based) uniform of the init stream (nn.rs:17-27), computed
    by jump-ahead instead of iteration: the step s -> a*s + 1 is an affine map
    on Z/2^64, and its n-th power is found by repeated squaring."""
    a, c = 6364136223846793005, 1
    pa, pc = 1, 0          # accumulated map s -> pa*s + pc
    while n:
        if n & 1:
            pa, pc = (a * pa) & _MASK64, (a * pc + c) & _MASK64
        a, c = (a * a) & _MASK64, (a * c + c) & _MASK64
        n >>= 1
    s = (pa * seed + pc) & _MASK64
    return float(np.float32(s >> 33)) / 2.0 ** 31


def _check_box_muller_pairs(vals, first_draw, std):
    """Invert Box-Muller on consecutive output pairs: x0^2 + x1^2 must equal
    -2 std^2 ln(u1) and atan2(x1, x0) must equal 2 pi u2, with (u1, u2) the
    draws `first_draw`, `first_draw + 1`, ... of the LCG stream."""
    vals = np.asarray(vals, np.float64)
    tiny = float(np.finfo(np.float32).tiny)
    for k in range(0, len(vals), 2):
        u1 = max(_lcg_draw(first_draw + k), tiny)
        u2 = _lcg_draw(first_draw + k + 1)
        r2 = -2.0 * std * std * math.log(u1)
        if k + 1 < len(vals):
            x0, x1 = vals[k], vals[k + 1]
            assert abs(x0 * x0 + x1 * x1 - r2) <= 2e-5 * r2, (k, x0, x1, r2)
            theta = math.atan2(x1, x0) % (2 * math.pi)
            d = abs(theta - 2 * math.pi * u2)
            assert min(d, 2 * math.pi - d) <= 2e-5 * 2 * math.pi + 1e-6 / math.sqrt(r2), (k, theta, u2)
        else:  # odd count: the last value is the cosine half of a pair
            assert abs(vals[k] - math.sqrt(r2) * math.cos(2 * math.pi * u2)) <= 2e-5 * math.sqrt(r2) + 1e-7


def test_kaiming_init_inverts_to_the_lcg_stream(fg, cpu):
    # nn.rs:16-47: draws u = (s>>33)/2^31 from s <- s*6364136223846793005 + 1
    # (seed 42, one stream shared by every layer in construction order), pairs
    # (u1, u2) -> sqrt(-2 ln u1) std (cos, sin)(2 pi u2), std = sqrt(2/fan_in).
    fg.reset_init_seed(42)
    l1 = fg.Linear(3, 2, cpu)   # 6 values: draws 1..6
    l2 = fg.Linear(5, 3, cpu)   # 15 values: 8 pairs, draws 7..22, last sine dropped
    l3 = fg.Linear(2, 2, cpu)   # draws 23..26
    _check_box_muller_pairs(l1.weight.numpy().reshape(-1), 1, math.sqrt(2 / 3))
    _check_box_muller_pairs(l2.weight.numpy().reshape(-1), 7, math.sqrt(2 / 5))
    _check_box_muller_pairs(l3.weight.numpy().reshape(-1), 23, math.sqrt(2 / 2))
    assert l1.bias.to_vec() == [0.0, 0.0] and l2.bias.to_vec() == [0.0] * 3


def test_kaiming_init_distribution(fg, cpu):
    # Over a C4-sized layer the values are N(0, 2/fan_in): checks the scale
    # uses fan_in (not fan_out) and the transform is Gaussian.
    from scipy import stats

    fg.reset_init_seed(42)
    w = fg.Linear(784, 128, cpu).weight.numpy().astype(np.float64).reshape(-1)
    std = math.sqrt(2 / 784)
    assert abs(w.mean()) < 5 * std / math.sqrt(w.size)
    assert abs(w.std() / std - 1) < 0.01
    assert stats.kstest(w / std, "norm").pvalue > 1e-3


def test_renderer_text_matches_reference_shape(cpu, fg):  # clang.rs:449-460, 574-665
    import oracle

    x = fg.Tensor.new([1.0, 2, 3], [3], cpu)
    src = oracle.plan_c([x.add(fg.Tensor.new([4.0, 5, 6], [3], cpu))])[0]
    assert "#include <math.h>" in src and "void kernel_0(" in src
    assert "float* restrict data0" in src
    assert "for (int idx0 = 0; idx0 < 3; idx0++)" in src
    m = fg.Tensor.new(np.ones((2, 8), np.float32), [2, 8], cpu)
    src = oracle.plan_c([m.max([1])])[0]
    assert "(-INFINITY)" in src and "ridx1" in src
    assert src.index("(-INFINITY)") < src.index("for (int ridx1")


def test_upcast_and_unroll_splits(cpu, fg):  # upcast.rs:346-369, unroll.rs:153-253
    import oracle

    a = fg.Tensor.new(np.ones(8, np.float32), [8], cpu)
    src = oracle.plan_c([a.add(a.neg())])[0]
    assert "idx0 < 2" in src  # GLOBAL 2 x UPCAST 4
    six = fg.Tensor.new(np.ones((1, 6), np.float32), [1, 6], cpu)
    assert "ridx1 < 6" in oracle.plan_c([six.sum([1])])[0]  # 6 is not split
    s64 = fg.Tensor.new(np.ones((1, 64), np.float32), [1, 64], cpu)
    assert "ridx1 < 16" in oracle.plan_c([s64.sum([1])])[0]  # 64 -> 16 x 4


def test_opt_env_disables_passes(cpu, fg, monkeypatch):  # optimize/mod.rs:85-112
    import oracle

    monkeypatch.setenv("OPT", "0")
    a = fg.Tensor.new(np.ones(8, np.float32), [8], cpu)
    assert "idx0 < 8" in oracle.plan_c([a.add(a.neg())])[0]
    monkeypatch.setenv("OPT", "symbolic,unroll")
    s64 = fg.Tensor.new(np.ones((8, 64), np.float32), [8, 64], cpu)
    src = oracle.plan_c([s64.sum([1])])[0]
    assert "idx0 < 8" in src and "ridx1 < 16" in src


def test_tensor_new_shape_mismatch(fg, cpu):  # tensor.rs:260-276
    with pytest.raises(fg.FerrogradError, match="doesn't match shape"):
        fg.Tensor.new(np.ones(3, np.float32), [2, 2], cpu)


def test_copy_from_host_size_error(fg, cpu):  # device.rs:457-466, cpu.rs:294-300
    t = fg.Tensor.new(np.ones(2, np.float32), [2], cpu)
    with pytest.raises(fg.FerrogradError, match="copy_from_host: expected 8 bytes, got 4"):
        t.write(np.ones(1, np.float32))
    t.write(np.array([3.0, 4.0], np.float32))
    assert t.to_vec() == [3.0, 4.0]
