"""The examples/mnist.rs:84-101 loop body run from native code
(fg_mlp_train_steps) against the same loop driven op by op from Python: the
same Tensor/Linear/Sgd calls, so the same kernels, losses and parameters, bit
for bit."""
import numpy as np
import pytest


def run(fg, dev, dims, batch, steps, native, chunks=None):
    """Params, losses and the last step's gradients after `steps` steps; the
    native loop is called once, or once per entry of `chunks`."""
    from ferrograd_amd.mlp import Mlp, synthetic_batch, train_step, train_steps_native

    fg.reset_init_seed(42)
    model = Mlp(dims, dev)
    opt = fg.Sgd(model.parameters(), 0.01)
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 7, 8)
    x = fg.Tensor.new(xs, list(xs.shape), dev)
    t = fg.Tensor.new(ts, list(ts.shape), dev)
    if native:
        losses = [l for n in (chunks or [steps]) for l in train_steps_native(model, opt, x, t, n)]
    else:
        losses = [train_step(model, opt, x, t).to_vec()[0] for _ in range(steps)]
    params = model.parameters()
    return losses, [p.numpy() for p in params] + [p.grad().numpy() for p in params]


@pytest.mark.parametrize("dims", [(16, 8, 4), (12, 16, 8, 5)])
def test_native_loop_matches_python_loop_cpu(fg, cpu, dims):
    # 9 steps: once two consecutive steps replayed the same plans (from the
    # third step on) the native loop launches the following steps from the
    # capture; the last one runs in full. Losses,
    # parameters and the last step's gradients equal the Python loop's bit for
    # bit, also when the loop is entered several times.
    before = fg.stats()
    l_py, p_py = run(fg, cpu, dims, 8, 9, native=False)
    l_nat, p_nat = run(fg, cpu, dims, 8, 9, native=True)
    after = fg.stats()
    assert after["steps_replayed"] - before["steps_replayed"] >= 4
    assert l_nat == l_py and l_nat[-1] < l_nat[0]
    for a, b in zip(p_nat, p_py):
        assert np.array_equal(a, b)
    # Calls shorter and longer than the loop's steps in flight (8 by default).
    for chunks in ([4, 1, 4], [2, 3, 4], [6, 3], [9]):
        l_ch, p_ch = run(fg, cpu, dims, 8, 9, native=True, chunks=chunks)
        assert l_ch == l_py and all(np.array_equal(a, b) for a, b in zip(p_ch, p_py)), chunks


def test_step_capture_off_matches(fg, cpu):
    # FG_STEP_CAPTURE=0 in a fresh process: every step runs in full, same bits.
    import json
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys, json; sys.path.insert(0, %r); sys.path.insert(0, %r); import ferrograd_amd as fg, oracle; "
            "oracle.load(); from test_train_loop import run; l, p = run(fg, 'cpu', (16, 8, 4), 8, 7, True); "
            "print(json.dumps([l, [a.tolist() for a in p], fg.stats()['steps_replayed']]))") % (root, os.path.join(root, "tests"))
    out = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, FG_STEP_CAPTURE="0"), capture_output=True,
                         text=True, check=True).stdout
    l_off, p_off, replayed = json.loads(out.strip().splitlines()[-1])
    l_on, p_on = run(fg, cpu, (16, 8, 4), 8, 7, native=True)
    assert replayed == 0 and l_off == l_on
    assert all(np.array_equal(np.array(a, np.float32).reshape(b.shape), b) for a, b in zip(p_off, p_on))


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


@pytest.mark.parametrize("depth,ok", [("1", True), ("3", True), ("0", False), ("9", False), ("x", False)])
def test_steps_in_flight_setting(fg, cpu, depth, ok):
    # FG_STEPS_IN_FLIGHT (read once per process) sets how many steps the
    # native loop queues ahead; any depth gives the same bits, and a value
    # outside 1..8 fails with a message naming the setting.
    import json
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys, json; sys.path.insert(0, %r); sys.path.insert(0, %r); import ferrograd_amd as fg, oracle; "
            "oracle.load(); from test_train_loop import run; l, p = run(fg, 'cpu', (16, 8, 4), 8, 7, True); "
            "print(json.dumps(l))") % (root, os.path.join(root, "tests"))
    r = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, FG_STEPS_IN_FLIGHT=depth),
                       capture_output=True, text=True)
    if ok:
        assert r.returncode == 0, r.stderr[-2000:]
        l_py, _ = run(fg, cpu, (16, 8, 4), 8, 7, native=False)
        assert json.loads(r.stdout.strip().splitlines()[-1]) == l_py
    else:
        assert r.returncode != 0 and "FG_STEPS_IN_FLIGHT must be 1 to 8" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("graph_min", [0, 2])
@pytest.mark.parametrize("batch,dims", [(256, (784, 128, 10)), (64, (96, 64, 32, 10))])
def test_native_loop_matches_python_loop_hip(fg, cpu, batch, dims, graph_min):
    # With replayed plans launched kernel by kernel (graph_min 0, the
    # default) or as HIP graphs (2): the steps built in full differ, the
    # captured steps go through the direct queue either way.
    from conftest import graphs_on

    print(f"native loop B={batch} dims={dims} graph_min={graph_min}", flush=True)
    l_py, p_py = run(fg, "hip", dims, batch, 9, native=False)
    before = fg.stats()
    with graphs_on(fg, graph_min):
        l_nat, p_nat = run(fg, "hip", dims, batch, 9, native=True)
    assert fg.stats()["steps_replayed"] - before["steps_replayed"] >= 4
    assert (fg.stats()["graph_replays"] > before["graph_replays"]) == (graph_min > 0)
    assert l_nat == l_py
    for a, b in zip(p_nat, p_py):
        assert np.array_equal(a, b)
    with graphs_on(fg, graph_min):
        l_ch, p_ch = run(fg, "hip", dims, batch, 9, native=True, chunks=[2, 7])
    assert l_ch == l_py and all(np.array_equal(a, b) for a, b in zip(p_ch, p_py))
    # The loop's steps are the recorded steps' kernels: each step of the
    # Python-driven loop, product by product against float64 on the device's
    # own values, and the oracle's losses within 1e-4.
    from conftest import check_recorded_steps, recorded_steps
    from ferrograd_amd.mlp import synthetic_batch

    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 7, 8)
    l_rec = check_recorded_steps(recorded_steps(fg, "hip", xs, ts, dims, steps=9))
    assert np.allclose(l_rec, l_nat, rtol=1e-6)
    l_cpu, _ = run(fg, cpu, dims, batch, 9, native=True)
    assert np.allclose(l_nat, l_cpu, rtol=1e-4, atol=1e-6)


def run_batches(fg, dev, dims, batch, nbatches, steps, native, chunks=None, first=0):
    """examples/mnist.rs:84-98 over a resident dataset of `nbatches` batches:
    step i narrows batch (first + i) mod nbatches. Losses, then parameters and
    the last step's gradients."""
    from ferrograd_amd.mlp import Mlp, synthetic_batch, train_batches_native, train_step

    fg.reset_init_seed(42)
    model = Mlp(dims, dev)
    opt = fg.Sgd(model.parameters(), 0.01)
    # one row more than the whole batches: the remainder is never trained on
    xs, ts = synthetic_batch(batch * nbatches + 1, dims[0], dims[-1], 7, 8)
    x = fg.Tensor.new(xs, list(xs.shape), dev)
    t = fg.Tensor.new(ts, list(ts.shape), dev)
    if native:
        losses, done = [], first
        for n in chunks or [steps]:
            losses += train_batches_native(model, opt, x, t, batch, n, first_batch=done)
            done += n
    else:
        losses = []
        for i in range(steps):
            s = ((first + i) % nbatches) * batch
            losses.append(train_step(model, opt, x.narrow(0, s, batch), t.narrow(0, s, batch)).to_vec()[0])
    params = model.parameters()
    return losses, [p.numpy() for p in params] + [p.grad().numpy() for p in params]


@pytest.mark.parametrize("dims", [(16, 8, 4), (12, 16, 8, 5)])
def test_native_batched_loop_matches_python_loop_cpu(fg, cpu, dims):
    # 14 steps over 6 batches (every start taken, then wrapping): from the
    # third step on, the steps replay the capture with their own batch start.
    # Bit for bit against the narrow()ed loop driven from Python, also when
    # entered in chunks that continue from the previous call's batch.
    before = fg.stats()
    l_py, p_py = run_batches(fg, cpu, dims, 8, 6, 14, native=False)
    l_nat, p_nat = run_batches(fg, cpu, dims, 8, 6, 14, native=True)
    assert fg.stats()["steps_replayed"] - before["steps_replayed"] >= 10
    assert l_nat == l_py and len(set(l_py)) == 14
    assert all(np.array_equal(a, b) for a, b in zip(p_nat, p_py))
    l_ch, p_ch = run_batches(fg, cpu, dims, 8, 6, 14, native=True, chunks=[5, 1, 8])
    assert l_ch == l_py and all(np.array_equal(a, b) for a, b in zip(p_ch, p_py))
    l_f, _ = run_batches(fg, cpu, dims, 8, 6, 5, native=False, first=4)
    l_fn, _ = run_batches(fg, cpu, dims, 8, 6, 5, native=True, first=4)
    assert l_f == l_fn


def test_native_batched_loop_errors(fg, cpu):
    from ferrograd_amd.mlp import Mlp

    model = Mlp((4, 3), cpu)
    opt = fg.Sgd(model.parameters(), 0.01)
    x = fg.Tensor.new(np.ones((10, 4), np.float32), [10, 4], cpu)
    t = fg.Tensor.new(np.ones((9, 3), np.float32), [9, 3], cpu)
    with pytest.raises(fg.FerrogradError, match="same number of rows"):
        fg.train_batches_native(model.layers, opt, x, t, 2, 1)
    t = fg.Tensor.new(np.ones((10, 3), np.float32), [10, 3], cpu)
    with pytest.raises(fg.FerrogradError, match="batch size larger than the dataset"):
        fg.train_batches_native(model.layers, opt, x, t, 11, 1)
    with pytest.raises(fg.FerrogradError, match="batch size must be positive"):
        fg.train_batches_native(model.layers, opt, x, t, 0, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("graph_min", [0, 2])
@pytest.mark.parametrize("batch,dims", [(256, (784, 128, 10)), (64, (96, 64, 32, 10))])
def test_native_batched_loop_matches_python_loop_hip(fg, cpu, batch, dims, graph_min):
    # The mnist.rs loop with a new batch every step: captured steps take the
    # batch start as a kernel argument; replayed plans launch kernel by kernel
    # (graph_min 0, the default) or as HIP graphs (2).
    from conftest import graphs_on

    print(f"batched native loop B={batch} dims={dims} graph_min={graph_min}", flush=True)
    l_py, p_py = run_batches(fg, "hip", dims, batch, 7, 16, native=False)
    before = fg.stats()
    with graphs_on(fg, graph_min):
        l_nat, p_nat = run_batches(fg, "hip", dims, batch, 7, 16, native=True)
    # steps 4 to 14: steps 0-3 record (zero biases, then the steady plan twice), 15 runs in full
    assert fg.stats()["steps_replayed"] - before["steps_replayed"] >= 11
    assert (fg.stats()["graph_replays"] > before["graph_replays"]) == (graph_min > 0)
    assert l_nat == l_py
    assert all(np.array_equal(a, b) for a, b in zip(p_nat, p_py))
    with graphs_on(fg, graph_min):
        l_ch, p_ch = run_batches(fg, "hip", dims, batch, 7, 16, native=True, chunks=[3, 13])
    assert l_ch == l_py and all(np.array_equal(a, b) for a, b in zip(p_ch, p_py))
    l_cpu, _ = run_batches(fg, cpu, dims, batch, 7, 16, native=True)
    assert np.allclose(l_nat, l_cpu, rtol=1e-4, atol=1e-6)
