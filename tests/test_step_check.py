"""The product-by-product train-step check (tests/f64ref.py check_mlp_step)
that the GPU tests and bench.py apply, exercised on the CPU oracle: the
pre-activations a step computes are read back from held tensors, the check
passes on the oracle's step, sampled and in full, and fails when one
backward product is planted wrong."""
from __future__ import annotations

import numpy as np
import pytest

import f64ref


def recorded_step(fg, dev, xs, ts, dims, lr=0.01):
    """One train step holding the pre-activations; returns what
    check_mlp_step takes."""
    from ferrograd_amd.mlp import Mlp

    fg.reset_init_seed(42)
    model = Mlp(dims, dev)
    params = model.parameters()
    p0 = [p.numpy().copy() for p in params]
    opt = fg.Sgd(params, lr)
    x, t = fg.Tensor.new(xs, list(xs.shape), dev), fg.Tensor.new(ts, list(ts.shape), dev)
    zs, h = [], x
    for i, layer in enumerate(model.layers):
        h = layer(h)
        zs.append(h)
        if i + 1 < len(model.layers):
            h = h.relu()
    loss = h.cross_entropy(t)
    opt.zero_grad()
    loss.backward()
    opt.step()
    lv = loss.to_vec()[0]
    assert all(z.is_realized() for z in zs), "the step materialises every pre-activation"
    B = xs.shape[0]
    return p0, [p.numpy() for p in params], lv, [z.numpy().reshape(B, -1) for z in zs[:-1]], \
        zs[-1].numpy().reshape(B, -1)


@pytest.mark.parametrize("sampled", [False, True])
def test_check_passes_on_the_oracle_step(fg, cpu, sampled):
    from ferrograd_amd.mlp import synthetic_batch

    dims = (64, 48, 40, 10)
    xs, ts = synthetic_batch(96, dims[0], dims[-1], 5, 6)
    p0, p1, loss, hidden, logits = recorded_step(fg, cpu, xs, ts, dims)
    rows = [np.array([0, 7, 47]), np.array([3, 39])] if sampled else None
    rep = f64ref.check_mlp_step(xs, ts, p0, p1, loss, hidden, logits, rows=rows,
                                batch_rows=np.arange(0, 96, 5) if sampled else None)
    assert rep["ok"], rep


@pytest.mark.parametrize("param", [0, 1, 2, 4, 5])
def test_check_fails_on_a_planted_backward_mistake(fg, cpu, param):
    # One term of the batch sum lost from one gradient element (the largest
    # term of all): an update the step check must reject, and only for that
    # parameter.
    from ferrograd_amd.mlp import synthetic_batch

    dims = (64, 48, 40, 10)
    xs, ts = synthetic_batch(96, dims[0], dims[-1], 5, 6)
    p0, p1, loss, hidden, logits = recorded_step(fg, cpu, xs, ts, dims)
    ws = [np.asarray(p, np.float64) for p in p0[0::2]]
    ins = [xs.astype(np.float64)] + [np.maximum(np.asarray(z, np.float64), 0) for z in hidden]
    zc = logits - logits.max(1, keepdims=True)
    dz = (np.exp(zc) / np.exp(zc).sum(1, keepdims=True) - ts) / xs.shape[0]
    layer = param // 2
    for i in range(len(ws) - 1, layer, -1):
        dz = (dz @ ws[i]) * (hidden[i - 1] > 0)
    terms = dz[:, :, None] * ins[layer][:, None, :] if param % 2 == 0 else dz[:, :, None]
    b, j, k = np.unravel_index(int(np.argmax(np.abs(terms))), terms.shape)
    bad = [p.copy() for p in p1]
    lost = terms[b, j, k]
    idx = (j, k) if param % 2 == 0 else (j,)
    bad[param][idx] = np.float32(bad[param][idx] + np.float32(0.01) * np.float32(lost))
    rep = f64ref.check_mlp_step(xs, ts, p0, bad, loss, hidden, logits)
    assert not rep["ok"] and rep["grad_err_over_bound"][param] > 1.0
    assert max(r for i, r in enumerate(rep["grad_err_over_bound"]) if i != param) <= 1.0
