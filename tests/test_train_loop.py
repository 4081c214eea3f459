"""The examples/mnist.rs:84-101 loop body run from native code
(fg_mlp_train_steps) against the same loop driven op by op from Python: the
same Tensor/Linear/Sgd calls, so the same kernels, losses and parameters, bit
for bit."""
import numpy as np
import pytest


def run(fg, dev, dims, batch, steps, native):
    from ferrograd_amd.mlp import Mlp, synthetic_batch, train_step, train_steps_native

    fg.reset_init_seed(42)
    model = Mlp(dims, dev)
    opt = fg.Sgd(model.parameters(), 0.01)
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 7, 8)
    x = fg.Tensor.new(xs, list(xs.shape), dev)
    t = fg.Tensor.new(ts, list(ts.shape), dev)
    if native:
        losses = train_steps_native(model, opt, x, t, steps)
    else:
        losses = [train_step(model, opt, x, t).to_vec()[0] for _ in range(steps)]
    return losses, [p.numpy() for p in model.parameters()]


@pytest.mark.parametrize("dims", [(16, 8, 4), (12, 16, 8, 5)])
def test_native_loop_matches_python_loop_cpu(fg, cpu, dims):
    l_py, p_py = run(fg, cpu, dims, 8, 3, native=False)
    l_nat, p_nat = run(fg, cpu, dims, 8, 3, native=True)
    assert l_nat == l_py and l_nat[-1] < l_nat[0]
    for a, b in zip(p_nat, p_py):
        assert np.array_equal(a, b)


def test_native_loop_errors_cross_the_abi(fg, cpu):
    from ferrograd_amd.mlp import Mlp

    model = Mlp((4, 3), cpu)
    opt = fg.Sgd(model.parameters(), 0.01)
    x = fg.Tensor.new(np.ones((2, 4), np.float32), [2, 4], cpu)
    t = fg.Tensor.new(np.ones((2, 5), np.float32), [2, 5], cpu)  # 5 classes, the layer gives 3
    with pytest.raises(fg.FerrogradError, match="cross_entropy"):
        fg.train_steps_native(model.layers, opt, x, t, 1)
    assert fg.train_steps_native(model.layers, opt, x, x, 0) == []
    with pytest.raises(fg.FerrogradError, match="negative step count"):
        fg.train_steps_native(model.layers, opt, x, x, -1)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,dims", [(256, (784, 128, 10)), (64, (96, 64, 32, 10))])
def test_native_loop_matches_python_loop_hip(fg, cpu, batch, dims):
    l_py, p_py = run(fg, "hip", dims, batch, 3, native=False)
    l_nat, p_nat = run(fg, "hip", dims, batch, 3, native=True)
    assert l_nat == l_py
    for a, b in zip(p_nat, p_py):
        assert np.array_equal(a, b)
    # The loop's steps are the recorded steps' kernels: each step of the
    # Python-driven loop, product by product against float64 on the device's
    # own values, and the oracle's losses within 1e-4.
    from conftest import check_recorded_steps, recorded_steps
    from ferrograd_amd.mlp import synthetic_batch

    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 7, 8)
    l_rec = check_recorded_steps(recorded_steps(fg, "hip", xs, ts, dims, steps=3))
    assert np.allclose(l_rec, l_nat, rtol=1e-6)
    l_cpu, _ = run(fg, cpu, dims, batch, 3, native=True)
    assert np.allclose(l_nat, l_cpu, rtol=1e-4, atol=1e-6)
