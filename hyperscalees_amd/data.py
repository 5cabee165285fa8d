"""Data path of the SNN ES driver: IDX/MNIST files and the batch sampler.

Thin wrappers over libhses.so's host-only entry points:
  * read_idx_images / read_idx_labels / load_mnist_from_dir
    (burn_impl/hyperscalees-envs/src/snn_mnist.rs:39-135): IDX buffers, plain
    or gzip, images as pixels / 255 (float32), labels raw (uint8);
  * shuffled_indices (burn_impl/hyperscalees/src/bin/accumulate_train.rs:157-174)
    and the per-epoch draw of the driver (accumulate_train.rs:724-730).
"""
import ctypes
import os

import numpy as np

from . import _lib

KEY_MUL = 0x9E3779B97F4A7C15

# snn_mnist.rs:24-31
IDX_IMAGES = (("train", "train-images-idx3-ubyte.gz"), ("test", "t10k-images-idx3-ubyte.gz"))
IDX_LABELS = (("train", "train-labels-idx1-ubyte.gz"), ("test", "t10k-labels-idx1-ubyte.gz"))


def _buf(data):
    data = bytes(data)
    return ctypes.c_char_p(data), len(data), data


def read_idx_images(data):
    """IDX images bytes (plain or gzip) -> float32 array (n, rows * cols) in [0, 1]."""
    p, n_bytes, keep = _buf(data)
    n, per = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("hses_read_idx_images", ctypes.cast(p, ctypes.c_void_p), n_bytes, None, 0,
              ctypes.byref(n), ctypes.byref(per))
    out = np.empty((n.value, per.value), np.float32)
    _lib.call("hses_read_idx_images", ctypes.cast(p, ctypes.c_void_p), n_bytes,
              out.ctypes.data, out.size, ctypes.byref(n), ctypes.byref(per))
    del keep
    return out


def read_idx_labels(data):
    """IDX labels bytes (plain or gzip) -> uint8 array (n,)."""
    p, n_bytes, keep = _buf(data)
    n = ctypes.c_int64()
    _lib.call("hses_read_idx_labels", ctypes.cast(p, ctypes.c_void_p), n_bytes, None, 0,
              ctypes.byref(n))
    out = np.empty(n.value, np.uint8)
    _lib.call("hses_read_idx_labels", ctypes.cast(p, ctypes.c_void_p), n_bytes, out.ctypes.data,
              out.size, ctypes.byref(n))
    del keep
    return out


def load_mnist_from_dir(path):
    """The four standard MNIST IDX files of `path`:
    ((train_images, train_labels), (test_images, test_labels))."""
    def read(name):
        with open(os.path.join(path, name), "rb") as f:
            return f.read()
    train = (read_idx_images(read(IDX_IMAGES[0][1])), read_idx_labels(read(IDX_LABELS[0][1])))
    test = (read_idx_images(read(IDX_IMAGES[1][1])), read_idx_labels(read(IDX_LABELS[1][1])))
    return train, test


def shuffled_indices(n, count, seed):
    """The first `count` indices of the driver's deterministic partial shuffle of [0, n)."""
    out = np.empty(count, np.int64)
    _lib.call("hses_shuffled_indices", n, count, seed & (2**64 - 1), out.ctypes.data)
    return out


def epoch_indices(n_train, batch, seed, epoch):
    """The driver's sample of one epoch: shuffled_indices(n_train, batch,
    seed ^ (epoch + 1) * KEY_MUL) (accumulate_train.rs:724-730)."""
    return shuffled_indices(n_train, batch, (seed ^ ((epoch + 1) * KEY_MUL)) & (2**64 - 1))
