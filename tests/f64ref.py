"""Float64 references for the MLP train step and the SGD-update check.

Used by the parity tests and by bench.py's C4/C5 checks. Nothing here runs
the path under test or the CPU oracle: it is numpy float64 arithmetic.

The train step (examples/mnist.rs:84-97): Linear layers with ReLU between
them, mean softmax cross-entropy (tensor.rs:715-752), backward by the
textbook rules ((softmax - t)/B propagated through the layers; gradient.rs
gives the same products: Mul and Expand rules, gradient.rs:100-105, 165-176),
then SGD `p <- p - lr * g` (optim.rs:60-71).

Each gradient comes with a condition scale: the sum over its terms of the
absolute values of every input that reaches it, to first order. For a weight
gradient dW_l = dZ_lᵀ·H_l that is S(dZ_l)ᵀ·|H_l|, where S(dZ_l) carries the
absolute values through the layers above (S(dZ_top) = |dZ_top|,
S(dZ_{l-1}) = (S(dZ_l)·|W_l|) masked). A reduction or product computed in f32
in any order stays within 1e-4 of that scale per element (the north star's
bar for reductions and matmuls), and so does a chain of them.

The SGD check tests the effective gradient (p0 - p1)/lr, not p1: a bound on
p1 is dominated by |p0| and would let gradient errors of percents through.
"""
from __future__ import annotations

import numpy as np

LR = 0.01


def relu_masks(zs):
    return [np.asarray(z, np.float64) > 0 for z in zs]


def mlp_step_f64(x, t, params, lr=LR, masks=None, logits=None, hidden=None):
    """One train step in float64.

    params: [W0, b0, W1, b1, ...] (W_l of shape [out, in]).
    masks: relu masks of the hidden pre-activations (default: from float64).
    hidden, logits: the device's own hidden pre-activations and logits; when
    given, the backward pass is evaluated on them (relu(z) as the layer inputs,
    softmax of the logits), which isolates each backward product's error from
    the forward pass's.

    Returns (loss, new params, grads, scales)."""
    ws = [np.asarray(p, np.float64) for p in params[0::2]]
    bs = [np.asarray(p, np.float64) for p in params[1::2]]
    x, t = np.asarray(x, np.float64), np.asarray(t, np.float64)
    B = x.shape[0]
    h, hs = x, np.abs(x)
    ins, in_scales, gates = [], [], []
    for i, (w, b) in enumerate(zip(ws, bs)):
        ins.append(h)
        in_scales.append(hs)
        if i + 1 < len(ws):
            z = np.asarray(hidden[i], np.float64) if hidden is not None else h @ w.T + b
            # The device's own pre-activations are exact inputs to the layers
            # above; float64's carry the forward products' error scale.
            zs = np.abs(z) if hidden is not None else hs @ np.abs(w).T + np.abs(b)
            gate = (z > 0) if masks is None else np.asarray(masks[i], bool)
            gates.append(gate)
            h, hs = np.where(gate, z, 0.0), np.where(gate, zs, 0.0)
        else:
            h = np.asarray(logits, np.float64) if logits is not None else h @ w.T + b
    zc = h - h.max(1, keepdims=True)
    logp = zc - np.log(np.exp(zc).sum(1, keepdims=True))
    loss = float(-np.mean((t * logp).sum(1)))
    dz = (np.exp(logp) - t) / B
    dzs = np.abs(dz)
    grads, scales = [None] * len(params), [None] * len(params)
    for i in reversed(range(len(ws))):
        grads[2 * i] = dz.T @ ins[i]
        scales[2 * i] = dzs.T @ in_scales[i]
        grads[2 * i + 1] = dz.sum(0)
        scales[2 * i + 1] = dzs.sum(0)
        if i > 0:
            dz = (dz @ ws[i]) * gates[i - 1]
            dzs = (dzs @ np.abs(ws[i])) * gates[i - 1]
    lr32 = float(np.float32(lr))
    new = [np.asarray(p, np.float64) - lr32 * g for p, g in zip(params, grads)]
    return loss, new, grads, scales


def mlp_step_f64_sampled(x, t, params, hidden, logits, rows):
    """The gradients of mlp_step_f64 on the device's own forward values
    (`hidden` pre-activations, `logits`), for every row of the last layer's
    weight and bias and for rows `rows[l]` of each lower layer l. For C5's
    shapes at B=8192, where the full float64 products would take minutes:
    dZ of each layer above the first is formed in full (from the [B, classes]
    top gradient that is one thin product per layer), dZ of the first layer
    only for its sampled columns. Scales take the device's layer inputs as
    exact, so they bound each backward product's own error.

    Returns (loss, {param index: (rows, grad rows, scale rows)})."""
    ws = [np.asarray(p, np.float64) for p in params[0::2]]
    L = len(ws)
    x, t = np.asarray(x, np.float64), np.asarray(t, np.float64)
    B = x.shape[0]
    zh = [np.asarray(z, np.float64) for z in hidden]
    gates = [z > 0 for z in zh]
    ins = [x] + [np.where(g, z, 0.0) for g, z in zip(gates, zh)]
    h = np.asarray(logits, np.float64)
    zc = h - h.max(1, keepdims=True)
    logp = zc - np.log(np.exp(zc).sum(1, keepdims=True))
    loss = float(-np.mean((t * logp).sum(1)))
    dz_up = (np.exp(logp) - t) / B  # dZ of layer i+1, every column
    dzs_up = np.abs(dz_up)
    out = {}
    for i in reversed(range(L)):
        if i == L - 1:
            sel, dz, dzs = np.arange(ws[i].shape[0]), dz_up, dzs_up
        else:
            # dZ_i = (dZ_{i+1} · W_{i+1}) ⊙ mask_i, for the sampled columns.
            sel = np.asarray(rows[i])
            w_sel = ws[i + 1][:, sel]
            dz = (dz_up @ w_sel) * gates[i][:, sel]
            dzs = (dzs_up @ np.abs(w_sel)) * gates[i][:, sel]
        out[2 * i] = (sel, dz.T @ ins[i], dzs.T @ np.abs(ins[i]))
        out[2 * i + 1] = (sel, dz.sum(0), dzs.sum(0))
        if 0 < i < L - 1:
            # Layer i-1 needs every column of dZ_i (dz_up holds the top
            # layer's already).
            dz_up = (dz_up @ ws[i + 1]) * gates[i]
            dzs_up = (dzs_up @ np.abs(ws[i + 1])) * gates[i]
    return loss, out


def sgd_effective_gradient_err(p0, p1, grad, scale, lr=LR, tol=1e-4):
    """Worst |(p0 - p1)/lr - grad| / bound over the elements (<= 1 passes).

    p1 = fl(p0 - fl(lr * g)) for the device's f32 gradient g, so
    (p0 - p1)/lr = g (1 + e) + d/lr with |e| <= 2^-24 and |d| <= ulp(p1)/2.
    The bound is tol * scale (the reduction's own error) + 2^-23 |grad| (the
    f32 roundings of g and lr*g) + ulp(p1)/lr (the rounding of the update)."""
    p0 = np.asarray(p0, np.float32).astype(np.float64).reshape(np.shape(grad))
    p1 = np.asarray(p1, np.float32).reshape(np.shape(grad))
    lr32 = float(np.float32(lr))
    geff = (p0 - p1.astype(np.float64)) / lr32
    g = np.asarray(grad, np.float64)
    bound = tol * np.asarray(scale, np.float64) + 2.0 ** -23 * np.abs(g) + np.spacing(np.abs(p1)).astype(
        np.float64) / lr32
    return float(np.max(np.abs(geff - g) / np.maximum(bound, 1e-300)))


def check_sgd_step(p0s, p1s, grads, scales, lr=LR, tol=1e-4, names=None):
    """Asserts every parameter's effective gradient is within bound."""
    for i, (p0, p1, g, s) in enumerate(zip(p0s, p1s, grads, scales)):
        worst = sgd_effective_gradient_err(p0, p1, g, s, lr, tol)
        assert worst <= 1.0, f"param {names[i] if names else i}: effective gradient off by {worst:.3g} x bound"


def check_mlp_step(x, t, p0, p1, loss, hidden, logits, lr=LR, rows=None, batch_rows=None, tol=1e-4):
    """One MLP train step checked product by product on the device's own
    values. `hidden` / `logits` are the pre-activations the step itself
    computed (read from the held tensors after the step). Checks:

    - each forward product z_l = h_l·W_lᵀ + b_l (h_l the device's relu of the
      layer below) on batch rows `batch_rows` (all when None), within
      tol · (|h_l|·|W_l|ᵀ + |b_l|);
    - the loss against float64 cross-entropy of the device's logits, within
      tol relative;
    - every parameter's effective gradient (p0 - p1)/lr against float64
      backward products on the device's forward values
      (mlp_step_f64_sampled with `rows`, else the full mlp_step_f64).

    Returns a report dict; report["ok"] is the verdict."""
    x = np.asarray(x, np.float64)
    B = x.shape[0]
    br = np.arange(B) if batch_rows is None else np.asarray(batch_rows)
    ins = [x] + [np.maximum(np.asarray(z, np.float64), 0.0) * (np.asarray(z) > 0) for z in hidden]
    outs = list(hidden) + [logits]
    fwd = []
    for l in range(len(ins)):
        w, b = np.asarray(p0[2 * l], np.float64), np.asarray(p0[2 * l + 1], np.float64)
        hl = ins[l][br]
        want = hl @ w.T + b
        scale = np.abs(hl) @ np.abs(w).T + np.abs(b)
        got = np.asarray(outs[l], np.float64)[br]
        fwd.append(float(np.max(np.abs(got - want) / np.maximum(tol * scale, 1e-300))))
    if rows is None:
        want_loss, _, grads, scales = mlp_step_f64(x, t, p0, lr, logits=logits, hidden=hidden)
        sel = {i: None for i in range(len(p0))}
    else:
        want_loss, out = mlp_step_f64_sampled(x, t, p0, hidden, logits, rows)
        sel = {i: out[i][0] for i in out}
        grads = [out[i][1] for i in range(len(p0))]
        scales = [out[i][2] for i in range(len(p0))]
    params = []
    for i in range(len(p0)):
        a, b = np.asarray(p0[i], np.float32), np.asarray(p1[i], np.float32)
        if sel[i] is not None:
            a, b = a[sel[i]], b[sel[i]]
        params.append(sgd_effective_gradient_err(a, b, grads[i], scales[i], lr, tol))
    loss_rel = abs(float(loss) - want_loss) / max(abs(want_loss), 1e-30)
    return {"forward_err_over_bound": fwd, "loss_rel_err": loss_rel, "grad_err_over_bound": params,
            "ok": bool(max(fwd) <= 1.0 and loss_rel <= tol and max(params) <= 1.0)}
