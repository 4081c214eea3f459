"""HIP path vs the oracle CPU device on identical programs and inputs.

Bars (north star): bit-exact for integer/index kernels, elementwise fp32
within 1e-5 relative (checked bit-exact here: both sides round each op once),
reductions and matmuls within 1e-4 * sum|terms| per element.
"""
import numpy as np
import pytest

from conftest import check_recorded_steps, recorded_steps, rel_err_bound, seeded

pytestmark = pytest.mark.gpu


def both(fn, cpu):
    """Run fn(device) on the oracle CPU device and on HIP."""
    return fn(cpu), fn("hip")


# ── the reference's tensor tests (src/tensor.rs:1133-1313) on HIP ──────────
def test_roundtrip(fg, hip):
    t = fg.Tensor.new([1.0, 2.0, 3.0], [3], hip)
    assert t.shape == (3,) and t.is_realized()
    assert t.to_vec() == [1.0, 2.0, 3.0]


def test_add_mul_relu(fg, hip):
    a = fg.Tensor.new([1.0, 2.0, 3.0], [3], hip)
    b = fg.Tensor.new([4.0, 5.0, 6.0], [3], hip)
    assert a.add(b).to_vec() == [5.0, 7.0, 9.0]
    c = fg.Tensor.new([2.0, 3.0, 4.0], [3], hip)
    d = fg.Tensor.new([5.0, 6.0, 7.0], [3], hip)
    assert c.mul(d).to_vec() == [10.0, 18.0, 28.0]
    x = fg.Tensor.new([1.0, -2.0, 3.0, -4.0], [4], hip)
    assert x.relu().to_vec() == [1.0, 0.0, 3.0, 0.0]


def test_log_softmax_known_values(fg, hip):
    r = fg.Tensor.new([0.0, 1.0], [1, 2], hip).log_softmax(1).realize().to_vec()
    assert abs(r[0] - (-1.3132616)) < 1e-5 and abs(r[1] - (-0.31326166)) < 1e-5


def test_cross_entropy_known_value(fg, hip):
    logits = fg.Tensor.new([2.0, 0.0, 0.0, 2.0], [2, 2], hip)
    targets = fg.Tensor.new([1.0, 0.0, 0.0, 1.0], [2, 2], hip)
    assert abs(logits.cross_entropy(targets).realize().to_vec()[0] - 0.12692805) < 1e-5


def test_sum_narrow_contiguous(fg, hip):
    x = fg.Tensor.new([1.0, 2, 3, 4, 5, 6], [2, 3], hip)
    assert x.sum([0]).to_vec() == [5.0, 7.0, 9.0]
    n = x.narrow(0, 1, 1)
    assert n.shape == (1, 3) and n.to_vec() == [4.0, 5.0, 6.0]
    c = x.permute([1, 0]).contiguous()
    assert c.shape == (3, 2) and c.to_vec() == [1.0, 4.0, 2.0, 5.0, 3.0, 6.0]


def test_gradients(fg, hip):
    x = fg.Tensor.new([1.0, 2, 3, 4], [2, 2], hip).narrow(0, 1, 1)
    w = fg.Tensor.new([10.0, 20.0], [2, 1], hip).with_requires_grad(True)
    g = x.matmul(w).sum([0, 1]).gradient([w])
    assert g[0].to_vec() == [3.0, 4.0] and not g[0].requires_grad()
    x2 = fg.Tensor.new([1.0, 2, 3, 4, 5, 6], [2, 3], hip).with_requires_grad(True)
    g2 = x2.permute([1, 0]).contiguous().sum([0, 1]).gradient([x2])
    assert g2[0].to_vec() == [1.0] * 6


def test_realize_idempotent_and_aliasing(fg, hip):
    a = fg.Tensor.new([1.0, 2.0], [2], hip)
    b = a.add(fg.Tensor.new([3.0, 4.0], [2], hip))
    assert b.realize().realize().to_vec() == [4.0, 6.0]
    left = fg.Tensor.zeros([2], hip)
    alias = left.alias()
    left.replace(fg.Tensor.new([5.0, 7.0], [2], hip))
    assert alias.to_vec() == [5.0, 7.0]


def test_assign_in_place(fg, hip):
    t = fg.Tensor.new([1.0, 2.0], [2], hip)
    alias = t.alias()
    t.assign(fg.Tensor.new([8.0, 9.0], [2], hip))
    fg.Tensor.realize_many([t])
    assert t.to_vec() == [8.0, 9.0] and alias.to_vec() == [8.0, 9.0]


def test_backward_stores_gradients(fg, hip):
    x = fg.Tensor.new([3.0], [1], hip).with_requires_grad(True)
    y = fg.Tensor.new([5.0], [1], hip).with_requires_grad(True)
    x.mul(y).sum([0]).backward()
    assert x.grad().to_vec() == [5.0] and y.grad().to_vec() == [3.0]


def test_int_and_bool_roundtrip(fg, hip):
    t = fg.Tensor.new(np.array([1, 2, 3], np.int32), [3], hip).realize()
    assert t.dtype == fg.I32 and t.numpy().tolist() == [1, 2, 3]
    b = fg.Tensor.new([True, False, True], [3], hip).realize()
    assert b.dtype == fg.BOOL and b.raw_bytes() == bytes([1, 0, 1])


def test_demo_closed_form(fg, hip):  # examples/demo.rs:17-30
    x = fg.Tensor.new([1.0, 2.0, 3.0, 4.0], [2, 2], hip)
    w = fg.Tensor.new([0.1, 0.2, 0.3, 0.4], [2, 2], hip).with_requires_grad(True)
    b = fg.Tensor.new([0.5, 0.6], [1, 2], hip).with_requires_grad(True)
    loss = x.matmul(w).add(b).sum([0, 1])
    # Realising the loss first would rewrite its graph to a buffer and leave
    # backward() no path to w (tensor.rs:222-252, 971-980), as in the
    # reference; the gradient pass runs before the loss is read.
    loss.backward()
    assert abs(loss.to_vec()[0] - 7.6) < 1e-5
    np.testing.assert_allclose(w.grad().to_vec(), [4.0, 4.0, 6.0, 6.0], rtol=1e-6)
    np.testing.assert_allclose(b.grad().to_vec(), [2.0, 2.0], rtol=1e-6)
    fg.Sgd([w], 0.1).step()
    np.testing.assert_allclose(w.to_vec(), [-0.3, -0.2, -0.3, -0.2], atol=1e-6)


# ── benchmark configs at parity-test sizes ─────────────────────────────────
def c1(fg, dev, x):
    t = fg.Tensor.new(x, list(x.shape), dev)
    return t.mul(fg.Tensor.scalar(0.5, dev)).add(fg.Tensor.scalar(1.0, dev)).relu().sum([1]).numpy()


def c2(fg, dev, a, b, c):
    ta, tb, tc = (fg.Tensor.new(v, list(v.shape), dev) for v in (a, b, c))
    return ta.mul(tb).add(tc).relu().numpy()


def c3(fg, dev, x, w, b):
    tx = fg.Tensor.new(x, list(x.shape), dev)
    tw = fg.Tensor.new(w, list(w.shape), dev)
    tb = fg.Tensor.new(b, list(b.shape), dev)
    return tx.matmul(tw.permute([1, 0])).add(tb).numpy()


@pytest.mark.parametrize("n", [4, 4096, 1 << 20, 1000, 6])
def test_c2_elementwise_bit_exact(fg, cpu, n):
    r = seeded(2)
    a, b, c = (r.uniform(-1, 1, n).astype(np.float32) for _ in range(3))
    want, got = both(lambda d: c2(fg, d, a, b, c), cpu)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("shape", [(64, 64), (256, 512), (3, 5), (4096, 4096)])
def test_c1_row_reduce(fg, cpu, shape):
    x = seeded(1).standard_normal(shape).astype(np.float32)
    want, got = both(lambda d: c1(fg, d, x), cpu)
    scale = np.maximum(x * 0.5 + 1.0, 0).sum(1)
    assert got.shape == want.shape == (shape[0], 1)
    got, want = got[:, 0], want[:, 0]
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0


# Shapes cover each GEMM tile path: 64/128-wide tiles, 256x128 and 128x256
# (BK 8) and 256x256 (BK 16, 8 waves), with ragged M/N edges and K not a
# multiple of the k-tile; split K (partials summed by a second pass) on a
# short grid, on narrow 32-wide tiles for N or M of 10, and with a ragged
# last column group. The narrow rows layout with its operand in registers:
# k not a multiple of 1024, an odd or ragged count of rows per workgroup,
# fewer rows than workgroups.
@pytest.mark.parametrize("mnk", [(64, 64, 64), (256, 128, 784), (128, 10, 128), (512, 512, 512), (100, 70, 30),
                                 (4100, 4000, 100), (4096, 2100, 72), (2100, 4096, 40), (4096, 10, 2048),
                                 (10, 4096, 2048), (1000, 70, 3000), (12, 602, 4000), (1500, 10, 2000),
                                 (1537, 16, 1500), (300, 10, 4096)])
def test_c3_linear_forward(fg, cpu, mnk):
    m, n, k = mnk
    r = seeded(5)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = r.uniform(-1 / 64, 1 / 64, (n, k)).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32)
    want, got = both(lambda d: c3(fg, d, x, w, b), cpu)
    scale = np.abs(x).astype(np.float64) @ np.abs(w).T.astype(np.float64) + np.abs(b)
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0
    exact = x.astype(np.float64) @ w.T.astype(np.float64) + b
    assert rel_err_bound(got, exact, scale, 1e-4) <= 1.0


@pytest.mark.parametrize("batch,hidden,steps", [(8, (16,), 2), (256, (128,), 2), (64, (96, 64), 1)])
def test_mlp_train_step(fg, cpu, batch, hidden, steps):
    # Every step on each device product by product against float64 on that
    # device's own values (forward products, loss, and each parameter's
    # effective gradient (p0 - p1)/lr, all within 1e-4 of their scales); the
    # two devices' losses within 1e-4 of each other.
    r = seeded(7)
    x = r.uniform(0, 1, (batch, 784)).astype(np.float32)
    labels = np.floor(r.uniform(0, 1, batch) * 10).astype(np.int64)
    t = np.eye(10, dtype=np.float32)[labels]
    dims = (784,) + tuple(hidden) + (10,)
    lc, lh = (check_recorded_steps(recorded_steps(fg, d, x, t, dims, steps=steps)) for d in (cpu, "hip"))
    np.testing.assert_allclose(lh, lc, rtol=1e-4)


def test_mlp_steps_on_narrowed_batches(fg, cpu):
    # Kernel-scalar row starts inside the MFMA operands of the forward and dW
    # products; the start changes every step while the plan replays.
    r = seeded(11)
    x = r.uniform(0, 1, (1024, 784)).astype(np.float32)
    labels = np.floor(r.uniform(0, 1, 1024) * 10).astype(np.int64)
    t = np.eye(10, dtype=np.float32)[labels]
    starts = [0, 256, 512, 768, 256]
    lc, lh = (check_recorded_steps(recorded_steps(fg, d, x, t, (784, 128, 10), starts=starts, batch=256))
              for d in (cpu, "hip"))
    np.testing.assert_allclose(lh, lc, rtol=1e-4)


@pytest.mark.parametrize("shape", [(8192, 512), (1000, 12), (4096, 4096), (3, 257), (256, 128)])
@pytest.mark.parametrize("op", ["sum", "max"])
def test_column_reductions(fg, cpu, shape, op):
    x = seeded(3).standard_normal(shape).astype(np.float32)

    def run(dev):
        t = fg.Tensor.new(x, list(shape), dev)
        return (t.sum([0]) if op == "sum" else t.max([0])).numpy()[0]

    want, got = both(run, cpu)
    if op == "max":
        assert np.array_equal(got, want)
    else:
        assert rel_err_bound(got, want, np.abs(x).sum(0), 1e-4) <= 1.0


def test_bias_gradient_sgd_update_in_place(fg, cpu):
    # b <- b - lr * sum_m g[m, :]: the column reduction with an in-place epilogue (K12).
    g = seeded(4).standard_normal((8192, 4096)).astype(np.float32)
    b0 = seeded(5).standard_normal(4096).astype(np.float32)

    def run(dev):
        b = fg.Tensor.new(b0, [4096], dev)
        gt = fg.Tensor.new(g, [8192, 4096], dev)
        b.assign(b.detach().sub(gt.sum([0]).reshape([4096]).mul(fg.Tensor.scalar(0.01, dev))))
        fg.Tensor.realize_many([b])
        return b.numpy()

    want, got = both(run, cpu)
    scale = np.abs(b0) + 0.01 * np.abs(g).sum(0)
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0


def test_lazy_zero_buffers(fg, hip):
    z = fg.Tensor.zeros([1000], hip)
    assert z.to_vec() == [0.0] * 1000
    z2 = fg.Tensor.zeros([4, 4], hip)
    assert z2.add(fg.Tensor.ones([4, 4], hip)).to_vec() == [1.0] * 16
    z3 = fg.Tensor.zeros([3], hip)
    z3.assign(fg.Tensor.new([1.0, 2.0, 3.0], [3], hip))
    fg.Tensor.realize_many([z3])
    assert z3.to_vec() == [1.0, 2.0, 3.0]
    i0 = fg.Tensor.zeros([5], hip, dtype=fg.I32)
    assert i0.numpy().tolist() == [0] * 5


def test_identity_copy_read_after_an_in_place_store(fg, cpu):
    # y = x @ (Wᵀ)ᵀ and W += 1 realised together with the store first: y must
    # use W from before the store. On HIP the identity copy of W is skipped
    # for readers that run before the store and taken for the root that runs
    # after it.
    r = seeded(11)
    xs = r.standard_normal((64, 96)).astype(np.float32)
    ws = r.standard_normal((80, 96)).astype(np.float32)

    def run(dev):
        x = fg.Tensor.new(xs, [64, 96], dev)
        w = fg.Tensor.new(ws, [80, 96], dev)
        y = x.matmul(w.permute([1, 0]))
        w.assign(w.add(fg.Tensor.scalar(1.0, dev)))
        fg.Tensor.realize_many([w, y])
        return y.numpy().reshape(64, 80), w.numpy().reshape(80, 96)

    (y_cpu, w_cpu), (y_hip, w_hip) = both(run, cpu)
    assert np.array_equal(w_hip, ws + np.float32(1.0)) and np.array_equal(w_cpu, w_hip)
    scale = np.abs(xs).astype(np.float64) @ np.abs(ws).T.astype(np.float64)
    exact_old_w = xs.astype(np.float64) @ ws.T.astype(np.float64)
    assert rel_err_bound(y_hip, exact_old_w, scale, 1e-4) <= 1.0
    assert rel_err_bound(y_hip, y_cpu, scale, 1e-4) <= 1.0


@pytest.mark.parametrize("case", ["ties", "large", "random"])
def test_cross_entropy_gradient_small_class_axis(fg, cpu, case):
    # The class-axis max and sums of log_softmax and its gradient are folded
    # again by each consumer on HIP (reductions over at most 16 elements). Tied
    # maxima split the max gradient by their count (gradient.rs Reduce(Max)),
    # large logits stress the max subtraction.
    r = seeded(13)
    b, c = 300, 10
    if case == "ties":
        z = np.round(r.standard_normal((b, c)) * 2.0).astype(np.float32)  # integers: many tied maxima
        z[:, 3] = z.max(axis=1)
    elif case == "large":
        z = (r.standard_normal((b, c)) * 60.0).astype(np.float32)
    else:
        z = r.standard_normal((b, c)).astype(np.float32)
    t = np.eye(c, dtype=np.float32)[r.integers(0, c, b)]

    def run(dev):
        logits = fg.Tensor.new(z, [b, c], dev).with_requires_grad(True)
        loss = logits.cross_entropy(fg.Tensor.new(t, [b, c], dev))
        g = loss.gradient([logits])[0]
        return loss.to_vec()[0], g.numpy().reshape(b, c)

    (l_cpu, g_cpu), (l_hip, g_hip) = both(run, cpu)
    assert abs(l_hip - l_cpu) <= 1e-5 * max(1.0, abs(l_cpu))
    # each gradient element is a handful of terms of magnitude <= 1/b
    assert np.max(np.abs(g_hip - g_cpu)) <= 1e-5 / b * 10
    zz = z.astype(np.float64) - z.max(axis=1, keepdims=True)
    p = np.exp(zz) / np.exp(zz).sum(axis=1, keepdims=True)
    assert np.max(np.abs(g_hip - (p - t) / b)) <= 1e-5 / b * 10


def test_requested_identity_contiguous_is_a_snapshot(fg, cpu):
    # c = w.T.T.contiguous() realised through y becomes its own buffer
    # (tensor.rs:625-630, 781-828); updating w in place afterwards leaves c
    # holding the old values, on both devices.
    ws = seeded(17).standard_normal((6, 8)).astype(np.float32)

    def run(dev):
        w = fg.Tensor.new(ws, [6, 8], dev)
        c = w.permute([1, 0]).permute([1, 0]).contiguous()
        c.add(fg.Tensor.scalar(1.0, dev)).realize()
        w.assign(w.add(fg.Tensor.scalar(1.0, dev)))
        w.realize()
        return c.numpy().reshape(6, 8), c.is_realized(), w.numpy().reshape(6, 8)

    (c_cpu, r_cpu, w_cpu), (c_hip, r_hip, w_hip) = both(run, cpu)
    assert r_cpu and r_hip
    assert np.array_equal(c_cpu, ws) and np.array_equal(c_hip, ws)
    assert np.array_equal(w_hip, ws + np.float32(1.0)) and np.array_equal(w_cpu, w_hip)


# ── narrow products: one output side of at most 16 (the class axis) ────────
# They run as VALU kernels that stream the wide operand once: "rows" when it
# is contiguous along k (the forward x·Wᵀ), "cols" when it is contiguous along
# the wide output (the weight gradient dZᵀ·H, split over k into partials).
@pytest.mark.parametrize("m,n,k", [(8192, 10, 4096), (1000, 16, 1000), (300, 3, 260), (10, 4096, 2048),
                                   (4097, 7, 1024), (513, 1, 64)])
def test_narrow_forward_rows(fg, cpu, m, n, k):
    r = seeded(23)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = r.uniform(-1 / 32, 1 / 32, (n, k)).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32)
    want, got = both(lambda d: c3(fg, d, x, w, b), cpu)
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    scale = np.abs(x64) @ np.abs(w64).T + np.abs(b)
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0
    assert rel_err_bound(got, x64 @ w64.T + b, scale, 1e-4) <= 1.0


@pytest.mark.parametrize("m,k", [(4096, 2048), (1537, 1500)])
def test_narrow_rows_with_a_fused_two_input_operand(fg, cpu, m, k):
    # relu(a*b)·Wᵀ: the elementwise producer is recomputed inside the narrow
    # kernel, so its register ring holds the raw loads of both inputs.
    r = seeded(31)
    a = r.standard_normal((m, k)).astype(np.float32)
    b = r.standard_normal((m, k)).astype(np.float32)
    w = r.uniform(-1 / 32, 1 / 32, (10, k)).astype(np.float32)

    def run(dev):
        ta, tb = fg.Tensor.new(a, [m, k], dev), fg.Tensor.new(b, [m, k], dev)
        tw = fg.Tensor.new(w, [10, k], dev)
        return ta.mul(tb).relu().matmul(tw.permute([1, 0])).numpy().reshape(m, 10)

    want, got = both(run, cpu)
    h64 = np.maximum(a * b, np.float32(0)).astype(np.float64)
    scale = np.abs(h64) @ np.abs(w.astype(np.float64)).T
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0
    assert rel_err_bound(got, h64 @ w.astype(np.float64).T, scale, 1e-4) <= 1.0


@pytest.mark.parametrize("bsz,nn,w", [(8192, 10, 4096), (256, 10, 1000), (4096, 16, 258), (1000, 1, 4099),
                                      (64, 10, 512)])
def test_narrow_weight_gradient_cols_with_sgd(fg, cpu, bsz, nn, w):
    r = seeded(29)
    g = (r.standard_normal((bsz, nn)) / bsz).astype(np.float32)
    h = np.maximum(r.standard_normal((bsz, w)), 0).astype(np.float32)
    w0 = r.standard_normal((nn, w)).astype(np.float32)

    def run(dev):
        th, tg = fg.Tensor.new(h, [bsz, w], dev), fg.Tensor.new(g, [bsz, nn], dev)
        wt = fg.Tensor.new(w0, [nn, w], dev).with_requires_grad(True)
        (dw,) = th.matmul(wt.permute([1, 0])).mul(tg).sum([0, 1]).gradient([wt])
        wt.assign(wt.detach().sub(dw.mul(fg.Tensor.scalar(0.01, dev))))
        fg.Tensor.realize_many([wt])
        return wt.numpy().reshape(nn, w)

    w_cpu, w_hip = both(run, cpu)
    import f64ref

    g64, h64 = g.astype(np.float64), h.astype(np.float64)
    assert f64ref.sgd_effective_gradient_err(w0, w_hip, g64.T @ h64, np.abs(g64).T @ np.abs(h64)) <= 1.0
    assert f64ref.sgd_effective_gradient_err(w0, w_cpu, g64.T @ h64, np.abs(g64).T @ np.abs(h64)) <= 1.0
