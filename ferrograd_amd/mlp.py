"""The training callers of the path: the MLP and train step of
examples/mnist.rs:30-97, generalised to any layer widths, plus the seeded
synthetic batches the benchmark configs use (no dataset download)."""
from __future__ import annotations

from typing import Callable, Sequence

import numpy as np

from . import Linear, Sgd, Tensor


def one_hot(labels: np.ndarray, num_classes: int) -> np.ndarray:
    """mnist.rs:18-25."""
    out = np.zeros((len(labels), num_classes), dtype=np.float32)
    out[np.arange(len(labels)), labels] = 1.0
    return out


class Mlp:
    """Linear -> ReLU -> ... -> Linear (mnist.rs:30-54 is dims = (784, 128, 10))."""

    def __init__(self, dims: Sequence[int], device="hip"):
        self.layers = [Linear(dims[i], dims[i + 1], device) for i in range(len(dims) - 1)]

    def forward(self, x: Tensor) -> Tensor:
        h = x
        for i, layer in enumerate(self.layers):
            h = layer(h)
            if i + 1 < len(self.layers):
                h = h.relu()
        return h

    def parameters(self) -> list:
        return [p for layer in self.layers for p in layer.parameters()]


def train_step(model: Mlp, opt: Sgd, x: Tensor, targets: Tensor) -> Tensor:
    """One step as mnist.rs:90-97: forward, cross-entropy, zero_grad, backward, SGD."""
    logits = model.forward(x)
    loss = logits.cross_entropy(targets)
    opt.zero_grad()
    loss.backward()
    opt.step()
    return loss


def synthetic_batch(batch: int, in_features: int, classes: int, seed_x: int, seed_y: int):
    """x ~ U(0,1) [batch, in]; labels floor(u*classes) one-hot."""
    x = np.random.default_rng(seed_x).uniform(0, 1, (batch, in_features)).astype(np.float32)
    labels = np.floor(np.random.default_rng(seed_y).uniform(0, 1, batch) * classes).astype(np.int64)
    labels = np.minimum(labels, classes - 1)
    return x, one_hot(labels, classes)


def mlp_setup(fg, device, batch: int, dims: Sequence[int], lr: float = 0.01, seed: int = 42,
              seeds=(7, 8)) -> tuple[Callable[[], float], Mlp]:
    """Model (reference LCG init, seed 42), optimizer and a resident batch;
    returns a closure running one train step and reading the loss."""
    fg.reset_init_seed(seed)
    model = Mlp(dims, device)
    opt = Sgd(model.parameters(), lr)
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], *seeds)
    x = Tensor.new(xs, list(xs.shape), device)
    t = Tensor.new(ts, list(ts.shape), device)

    def step() -> float:
        loss = train_step(model, opt, x, t)
        return loss.to_vec()[0]

    return step, model
