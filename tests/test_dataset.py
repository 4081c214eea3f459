"""Offline IDX loader (src/dataset.rs:116-161) and the examples/mnist.rs loop,
on synthetic IDX files written by the test (no MNIST download here)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import seeded


def make_mnist(tmp_path, n_train=512, n_test=64, seed=0):
    """Separable synthetic digits: class c lights up rows 2c..2c+2."""
    from ferrograd_amd.dataset import FILES, write_idx_images, write_idx_labels

    r = seeded(seed)

    def split(n):
        labels = r.integers(0, 10, n).astype(np.uint8)
        px = r.integers(0, 40, (n, 28, 28)).astype(np.uint8)
        for i, c in enumerate(labels):
            px[i, 2 * c:2 * c + 3, :] = 200 + r.integers(0, 55, (3, 28))
        return px, labels

    (tr_x, tr_y), (te_x, te_y) = split(n_train), split(n_test)
    d = str(tmp_path)
    write_idx_images(os.path.join(d, FILES[0]), tr_x)
    write_idx_labels(os.path.join(d, FILES[1]), tr_y)
    write_idx_images(os.path.join(d, FILES[2]), te_x)
    write_idx_labels(os.path.join(d, FILES[3]), te_y)
    return d, tr_x, tr_y, te_x, te_y


def test_idx_images_scale_pixels_by_255(fg, cpu, tmp_path):
    from ferrograd_amd.dataset import MNISTDataset

    d, tr_x, tr_y, te_x, te_y = make_mnist(tmp_path, n_train=20, n_test=7)
    ds = MNISTDataset.load(d, cpu)
    assert ds.train_len() == 20 and ds.test_len() == 7 and ds.num_classes == 10
    img = ds.train_images.numpy()
    assert img.shape == (20, 784)
    want = tr_x.reshape(20, 784).astype(np.float32) / np.float32(255.0)  # f32 division, dataset.rs:138
    assert np.array_equal(img.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(ds.train_labels, tr_y) and np.array_equal(ds.test_labels, te_y)
    assert img.max() <= 1.0 and img.min() >= 0.0


def test_idx_format_errors_carry_reference_messages(fg, cpu, tmp_path):
    from ferrograd_amd.dataset import idx_images, idx_labels, write_idx_images

    bad = tmp_path / "bad"
    bad.write_bytes(np.array([2049, 1, 28, 28], ">u4").tobytes())
    with pytest.raises(fg.FerrogradError, match="expected IDX image magic 2051, got 2049"):
        idx_images(str(bad), cpu)
    write_idx_images(str(tmp_path / "small"), np.zeros((2, 14, 14), np.uint8))
    with pytest.raises(fg.FerrogradError, match="expected IDX label magic 2049, got 2051"):
        idx_labels(str(tmp_path / "small"))
    with pytest.raises(fg.FerrogradError, match="expected 28x28 images, got 14x14"):
        idx_images(str(tmp_path / "small"), cpu)
    trunc = tmp_path / "trunc"
    trunc.write_bytes(np.array([2051, 3, 28, 28], ">u4").tobytes() + bytes(100))
    with pytest.raises(fg.FerrogradError, match="io: "):
        idx_images(str(trunc), cpu)
    with pytest.raises(fg.FerrogradError, match="io: "):
        idx_labels(str(tmp_path / "missing"))


def test_predictions_take_last_of_equal_maxima():
    from ferrograd_amd.mlp import predictions

    logits = np.array([[1, 3, 3, 0], [5, 1, 1, 5], [0, 0, 0, 0]], np.float32)
    assert predictions(logits).tolist() == [2, 3, 3]


def test_mnist_loop_learns_on_cpu(fg, cpu, tmp_path):
    from ferrograd_amd.dataset import MNISTDataset
    from ferrograd_amd.mlp import train_mnist

    d, *_ = make_mnist(tmp_path)
    fg.reset_init_seed(42)
    h = train_mnist(MNISTDataset.load(d, cpu), cpu, epochs=3, batch_size=64, lr=0.05, log=None)
    assert len(h["batch_loss"]) == 3 * 8
    assert h["epoch_loss"][-1] < h["epoch_loss"][0]
    assert h["accuracy"][-1] >= 90.0


@pytest.mark.gpu
def test_mnist_loop_matches_cpu_on_hip(fg, cpu, hip, tmp_path):
    from ferrograd_amd.dataset import MNISTDataset
    from ferrograd_amd.mlp import train_mnist

    d, *_ = make_mnist(tmp_path)
    runs = {}
    for dev in (cpu, hip):
        fg.reset_init_seed(42)
        runs[dev] = train_mnist(MNISTDataset.load(d, dev), dev, epochs=2, batch_size=64, lr=0.05, log=None)
    np.testing.assert_allclose(runs[hip]["batch_loss"], runs[cpu]["batch_loss"], rtol=1e-4)
    assert runs[hip]["accuracy"] == runs[cpu]["accuracy"]


def test_mnist_native_loop_matches_the_python_loop_on_cpu(fg, cpu, tmp_path):
    # train_mnist(native=True) runs each epoch's batches through
    # fg_mlp_train_batches (captured steps that take each batch's start as an
    # argument): the same losses and accuracies bit for bit.
    from ferrograd_amd.dataset import MNISTDataset
    from ferrograd_amd.mlp import train_mnist

    d, *_ = make_mnist(tmp_path)
    runs = {}
    for native in (False, True):
        fg.reset_init_seed(42)
        runs[native] = train_mnist(MNISTDataset.load(d, cpu), cpu, epochs=2, batch_size=64, lr=0.05, log=None,
                                   native=native)
    assert runs[True] == runs[False]


@pytest.mark.gpu
def test_mnist_native_loop_matches_the_python_loop_on_hip(fg, hip, tmp_path):
    from ferrograd_amd.dataset import MNISTDataset
    from ferrograd_amd.mlp import train_mnist

    print("mnist loop, native and Python-driven, on hip", flush=True)
    d, *_ = make_mnist(tmp_path)
    runs = {}
    for native in (False, True):
        fg.reset_init_seed(42)
        runs[native] = train_mnist(MNISTDataset.load(d, hip), hip, epochs=2, batch_size=64, lr=0.05, log=None,
                                   native=native)
    assert runs[True] == runs[False]
