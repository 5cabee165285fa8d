"""Host-side data path: IDX parsing (snn_mnist.rs:39-112) against the reference's
own test vectors (snn_mnist.rs:242-311), and the driver's batch sampler
shuffled_indices (accumulate_train.rs:157-174).  No GPU needed."""
import gzip
import struct

import numpy as np
import pytest

from hyperscalees_amd import data
from hyperscalees_amd._lib import HsesError

KEY = 0x9E3779B97F4A7C15
PIXELS = bytes([0, 64, 128, 255, 1, 2, 3, 4])


def idx_images_bytes(n, rows, cols, payload):
    return struct.pack(">IIII", 0x803, n, rows, cols) + bytes(payload)


def idx_labels_bytes(n, payload):
    return struct.pack(">II", 0x801, n) + bytes(payload)


def test_reads_plain_idx_images():
    # snn_mnist.rs:243-263
    v = data.read_idx_images(idx_images_bytes(2, 2, 2, PIXELS))
    assert v.shape == (2, 4)
    expected = np.array([0, 64, 128, 255, 1, 2, 3, 4], np.float32) / np.float32(255.0)
    np.testing.assert_array_equal(v.ravel(), expected)


def test_reads_plain_idx_labels():
    np.testing.assert_array_equal(data.read_idx_labels(idx_labels_bytes(2, [1, 7])), [1, 7])


def test_reads_gzipped_idx():
    # snn_mnist.rs:283-311
    raw = idx_images_bytes(2, 2, 2, PIXELS)
    gz = gzip.compress(raw)
    assert gz[:2] == b"\x1f\x8b"
    np.testing.assert_array_equal(data.read_idx_images(gz), data.read_idx_images(raw))
    np.testing.assert_array_equal(data.read_idx_labels(gzip.compress(idx_labels_bytes(2, [1, 7]))),
                                  [1, 7])


def test_rejects_bad_magic_and_short_buffers():
    # snn_mnist.rs:272-280, plus the size checks of read_idx_images/labels
    bad = bytearray(idx_images_bytes(1, 1, 1, [42]))
    bad[0] = 0x99
    with pytest.raises(HsesError):
        data.read_idx_images(bytes(bad))
    lbad = bytearray(idx_labels_bytes(1, [5]))
    lbad[3] = 0x55
    with pytest.raises(HsesError):
        data.read_idx_labels(bytes(lbad))
    for blob in (b"", idx_images_bytes(2, 2, 2, PIXELS)[:20], idx_labels_bytes(3, [1, 2])):
        with pytest.raises(HsesError):
            (data.read_idx_labels if blob[:4] == b"\x00\x00\x08\x01" else data.read_idx_images)(blob)
    with pytest.raises(HsesError):  # 2^31 images of one pixel: beyond 2^30 elements
        data.read_idx_images(idx_images_bytes(2**31, 1, 1, b""))
    with pytest.raises(HsesError):  # truncated gzip stream
        data.read_idx_images(gzip.compress(idx_images_bytes(2, 2, 2, PIXELS))[:-9])


def test_load_mnist_from_dir(tmp_path):
    rng = np.random.default_rng(0)
    imgs = {s: rng.integers(0, 256, (n, 28 * 28), dtype=np.uint8) for s, n in (("train", 5), ("test", 3))}
    lbls = {s: rng.integers(0, 10, len(imgs[s]), dtype=np.uint8) for s in imgs}
    for (split, name), (_, lname) in zip(data.IDX_IMAGES, data.IDX_LABELS):
        (tmp_path / name).write_bytes(gzip.compress(idx_images_bytes(len(imgs[split]), 28, 28,
                                                                     imgs[split].tobytes())))
        (tmp_path / lname).write_bytes(gzip.compress(idx_labels_bytes(len(lbls[split]),
                                                                      lbls[split].tobytes())))
    (tri, trl), (tei, tel) = data.load_mnist_from_dir(str(tmp_path))
    np.testing.assert_array_equal(tri, imgs["train"].astype(np.float32) / np.float32(255.0))
    np.testing.assert_array_equal(tel, lbls["test"])
    assert tri.shape == (5, 784) and tei.shape == (3, 784) and trl.shape == (5,)


def test_shuffled_indices_structure():
    for n, seed in ((1, 0), (10, 3), (1000, 12345)):
        full = data.shuffled_indices(n, n, seed)
        assert sorted(full.tolist()) == list(range(n))             # a permutation
        for c in (0, 1, n // 2):
            np.testing.assert_array_equal(data.shuffled_indices(n, c, seed), full[:c])  # prefixes
    assert not np.array_equal(data.shuffled_indices(50, 50, 1), data.shuffled_indices(50, 50, 2))
    with pytest.raises(HsesError):
        data.shuffled_indices(5, 6, 0)


def test_shuffled_indices_first_draw_parity():
    # n = 2: the first index is draw % 2, the parity of the first xorshift64
    # state (the odd multiplier keeps it), which is 1 ^ bit 7 of the start
    # state (seed ^ KEY) | 1: x ^= x << 13 keeps bits 0..12, x ^= x >> 7 adds
    # bit 7 into bit 0, x ^= x << 17 keeps bit 0.
    for s0 in (0x1, 0x81, 0x12345601, 0xFFFFFF7F):
        seed = s0 ^ KEY
        expect = 1 ^ ((s0 >> 7) & 1)
        assert data.shuffled_indices(2, 1, seed)[0] == expect


def py_shuffled_indices(n, count, seed):
    """accumulate_train.rs:157-174 in Python integers: xorshift64 (13, 7, 17)
    from (seed ^ 0x9E3779B97F4A7C15) | 1, each draw times 0x2545F4914F6CDD1D
    (wrapping u64), partial Fisher-Yates swap of i with i + draw % (n - i)."""
    m64 = 2**64 - 1
    state = ((seed ^ 0x9E3779B97F4A7C15) | 1) & m64
    idx = list(range(n))
    for i in range(count):
        state ^= (state << 13) & m64
        state ^= state >> 7
        state ^= (state << 17) & m64
        draw = (state * 0x2545F4914F6CDD1D) & m64
        j = i + draw % (n - i)
        idx[i], idx[j] = idx[j], idx[i]
    return idx[:count]


@pytest.mark.parametrize("n,count,seed", [(60000, 100, 0), (60000, 100, 42 ^ KEY),
                                          (1000, 1000, 12345), (7, 7, 2**64 - 1),
                                          (2**20, 100, 0xDEADBEEF), (3, 2, 5)])
def test_shuffled_indices_match_python_restatement(n, count, seed):
    np.testing.assert_array_equal(data.shuffled_indices(n, count, seed),
                                  py_shuffled_indices(n, count, seed))


def test_shuffled_indices_first_index_uniform():
    n = 7
    counts = np.bincount([data.shuffled_indices(n, 1, s)[0] for s in range(7000)], minlength=n)
    chi2 = ((counts - 1000.0) ** 2 / 1000.0).sum()
    assert chi2 < 22.5  # 6 degrees of freedom, p = 0.001


def test_epoch_indices_follow_the_driver_seed():
    a = data.epoch_indices(60000, 256, 42, 0)
    np.testing.assert_array_equal(a, data.shuffled_indices(60000, 256, 42 ^ KEY))
    assert not np.array_equal(a, data.epoch_indices(60000, 256, 42, 1))
    assert len(set(a.tolist())) == 256
