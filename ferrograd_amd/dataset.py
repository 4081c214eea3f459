"""MNIST from local IDX files (src/dataset.rs:25-161), parsed by the native
library. The reference downloads and gunzips missing files (dataset.rs:170-196);
this build has no network path, so the four files must already be unpacked in
the directory given to `MNISTDataset.load`."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import Tensor, _check, _dev, lib

FILES = ("train-images-idx3-ubyte", "train-labels-idx1-ubyte", "t10k-images-idx3-ubyte", "t10k-labels-idx1-ubyte")


def idx_images(path: str, device="hip") -> Tensor:
    """parse_images (dataset.rs:116-142): f32 [count, 784], pixels / 255."""
    out = ctypes.c_void_p()
    _check(lib().fg_idx_images(os.fsencode(path), _dev(device), ctypes.byref(out)))
    return Tensor(out.value)


def idx_labels(path: str) -> np.ndarray:
    """parse_labels (dataset.rs:144-157): one byte per label."""
    n = ctypes.c_size_t()
    _check(lib().fg_idx_labels(os.fsencode(path), None, 0, ctypes.byref(n)))
    out = np.empty(n.value, np.uint8)
    _check(lib().fg_idx_labels(os.fsencode(path), out.ctypes.data, out.size, ctypes.byref(n)))
    return out


class MNISTDataset:
    """dataset.rs:25-79: train/test images (tensors on `device`) and labels."""

    def __init__(self, train_images: Tensor, train_labels: np.ndarray, test_images: Tensor, test_labels: np.ndarray,
                 num_classes: int = 10):
        self.train_images = train_images
        self.train_labels = train_labels
        self.test_images = test_images
        self.test_labels = test_labels
        self.num_classes = num_classes

    @staticmethod
    def load(directory: str = os.path.join("data", "mnist"), device="hip") -> "MNISTDataset":
        p = [os.path.join(directory, f) for f in FILES]
        return MNISTDataset(idx_images(p[0], device), idx_labels(p[1]), idx_images(p[2], device), idx_labels(p[3]))

    def train_len(self) -> int:
        return len(self.train_labels)

    def test_len(self) -> int:
        return len(self.test_labels)


def write_idx_images(path: str, pixels: np.ndarray) -> None:
    """Writes u8 images [count, 28, 28] in IDX format (magic 2051)."""
    pixels = np.ascontiguousarray(pixels, dtype=np.uint8)
    hdr = np.array([2051, pixels.shape[0], pixels.shape[1], pixels.shape[2]], dtype=">u4")
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(pixels.tobytes())


def write_idx_labels(path: str, labels: np.ndarray) -> None:
    """Writes u8 labels in IDX format (magic 2049)."""
    labels = np.ascontiguousarray(labels, dtype=np.uint8)
    with open(path, "wb") as f:
        f.write(np.array([2049, labels.size], dtype=">u4").tobytes())
        f.write(labels.tobytes())
