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

    def __init__(self, dims: Sequence[int], device=None):
        self.layers = [Linear(dims[i], dims[i + 1], device) for i in range(len(dims) - 1)]

    def forward(self, x: Tensor) -> Tensor:
        return self.forward_preactivations(x)[-1]

    def forward_preactivations(self, x: Tensor) -> list:
        """Every layer's output before its ReLU, the logits last. Holding
        them across a train step keeps the reference's partition for them
        (each is materialised anyway, as a multi-consumer node), and after the
        step's realize they point at the buffers the step computed
        (tensor.rs:222-252)."""
        zs, h = [], x
        for i, layer in enumerate(self.layers):
            h = layer(h)
            zs.append(h)
            if i + 1 < len(self.layers):
                h = h.relu()
        return zs

    def parameters(self) -> list:
        return [p for layer in self.layers for p in layer.parameters()]


def train_step(model: Mlp, opt: Sgd, x: Tensor, targets: Tensor, preactivations: list | None = None) -> Tensor:
    """One step as mnist.rs:90-97: forward, cross-entropy, zero_grad, backward,
    SGD. With a list for `preactivations`, the layers' outputs before ReLU
    (logits last) are appended to it, realised by the step itself."""
    zs = model.forward_preactivations(x)
    if preactivations is not None:
        preactivations.extend(zs)
    loss = zs[-1].cross_entropy(targets)
    opt.zero_grad()
    loss.backward()
    opt.step()
    return loss


def train_steps_native(model: Mlp, opt: Sgd, x: Tensor, targets: Tensor, steps: int) -> list:
    """`steps` train steps as train_step, looped in native code
    (fg_mlp_train_steps), with each step's loss read back as
    examples/mnist.rs:98 does; returns the losses."""
    from . import train_steps_native as native

    return native(model.layers, opt, x, targets, steps)


def train_batches_native(model: Mlp, opt: Sgd, images: Tensor, targets: Tensor, batch_size: int, steps: int,
                         first_batch: int = 0) -> list:
    """`steps` train steps over narrow()ed batches of the resident `images`
    and `targets` (examples/mnist.rs:84-98), batch index first_batch + i
    wrapping over the whole batches, looped in native code
    (fg_mlp_train_batches); returns the losses."""
    from . import train_batches_native as native

    return native(model.layers, opt, images, targets, batch_size, steps, first_batch)


def synthetic_batch(batch: int, in_features: int, classes: int, seed_x: int, seed_y: int):
    """x ~ U(0,1) [batch, in]; labels floor(u*classes) one-hot."""
    x = np.random.default_rng(seed_x).uniform(0, 1, (batch, in_features)).astype(np.float32)
    labels = np.floor(np.random.default_rng(seed_y).uniform(0, 1, batch) * classes).astype(np.int64)
    labels = np.minimum(labels, classes - 1)
    return x, one_hot(labels, classes)


def mlp_setup(fg, device, batch: int, dims: Sequence[int], lr: float = 0.01, seed: int = 42,
              seeds=(7, 8), with_state: bool = False):
    """Model (reference LCG init, seed 42), optimizer and a resident batch;
    returns a closure running one train step and reading the loss, and the
    model (or, with_state, the model, optimizer, inputs and targets)."""
    fg.reset_init_seed(seed)
    model = Mlp(dims, device)
    opt = Sgd(model.parameters(), lr)
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], *seeds)
    x = Tensor.new(xs, list(xs.shape), device)
    t = Tensor.new(ts, list(ts.shape), device)

    def step() -> float:
        loss = train_step(model, opt, x, t)
        return loss.to_vec()[0]

    return step, ((model, opt, x, t) if with_state else model)


def predictions(logits: np.ndarray) -> np.ndarray:
    """Index of the largest logit per row; among equal maxima the last one, as
    Iterator::max_by in examples/mnist.rs:108-114 returns."""
    flipped = logits[:, ::-1]
    return logits.shape[1] - 1 - np.argmax(flipped, axis=1)


def train_mnist(dataset, device=None, epochs: int = 5, batch_size: int = 256, lr: float = 0.01,
                max_batches: int | None = None, log=print, native: bool = False) -> dict:
    """examples/mnist.rs:59-126 on `device`: Linear(784,128) -> ReLU ->
    Linear(128,10), cross-entropy, SGD; batches are narrow()ed views of the
    resident training set. Returns per-batch losses and per-epoch average loss
    and test accuracy (percent). With `native`, each epoch's batch loop runs
    in native code (fg_mlp_train_batches: the same steps, captured and
    replayed with each batch's start as an argument)."""
    train_targets = Tensor.new(one_hot(dataset.train_labels, dataset.num_classes),
                               [dataset.train_len(), dataset.num_classes], device)
    model = Mlp((784, 128, 10), device)
    opt = Sgd(model.parameters(), lr)
    num_batches = dataset.train_len() // batch_size
    if max_batches is None:
        import os

        max_batches = int(os.environ.get("MAX_BATCHES", num_batches))
    runs = min(max_batches, num_batches)
    history = {"batch_loss": [], "epoch_loss": [], "accuracy": []}
    for epoch in range(epochs):
        epoch_loss = np.float32(0.0)
        if native:
            for b, v in enumerate(train_batches_native(model, opt, dataset.train_images, train_targets, batch_size,
                                                       runs)):
                epoch_loss = np.float32(epoch_loss + np.float32(v))
                history["batch_loss"].append(v)
                if log:
                    log(f"  epoch {epoch} batch {b:>4}/{num_batches}  loss={v:.4f}")
        for b in range(0 if native else runs):
            start = b * batch_size
            x = dataset.train_images.narrow(0, start, batch_size)
            t = train_targets.narrow(0, start, batch_size)
            loss = model.forward(x).cross_entropy(t)
            opt.zero_grad()
            loss.backward()
            opt.step()
            v = loss.to_vec()[0]
            epoch_loss = np.float32(epoch_loss + np.float32(v))
            history["batch_loss"].append(v)
            if log:
                log(f"  epoch {epoch} batch {b:>4}/{num_batches}  loss={v:.4f}")
        avg = float(epoch_loss / np.float32(runs))
        logits = model.forward(dataset.test_images).numpy().reshape(dataset.test_len(), dataset.num_classes)
        acc = float(np.float32(np.sum(predictions(logits) == dataset.test_labels)) / np.float32(dataset.test_len())
                    * np.float32(100.0))
        history["epoch_loss"].append(avg)
        history["accuracy"].append(acc)
        if log:
            log(f"Epoch {epoch}: avg_loss={avg:.4f}, test_accuracy={acc:.1f}%")
    return history


if __name__ == "__main__":
    import argparse

    from .dataset import MNISTDataset

    ap = argparse.ArgumentParser(description="Train the examples/mnist.rs MLP on local IDX files")
    ap.add_argument("--data", default="data/mnist")
    ap.add_argument("--device", default="hip")
    ap.add_argument("--epochs", type=int, default=5)
    a = ap.parse_args()
    train_mnist(MNISTDataset.load(a.data, a.device), a.device, epochs=a.epochs)
