"""GPU parity of the noiser stream: bit-exact against the oracle.

The exhaustive test evaluates the device Box-Muller halves on all 2^24 unit
indices and compares them with glibc (through the oracle): since every normal
is radius(k1) * cos(k2) with one f32 multiply, agreement on all k makes every
normal of every stream bit-exact."""
import numpy as np
import pytest
import torch

from tests import oracle_lib as O

pytestmark = pytest.mark.gpu


def test_bm_halves_exhaustive(hses_gpu):
    n = 1 << 24
    lg, rad, cs = hses_gpu.bm_eval(0, n)
    torch.cuda.synchronize()
    rl, rr, rc = (np.zeros(n, np.float32) for _ in range(3))
    O.load().or_bm_eval(0, n, rl, rr, rc)
    for name, dev, ref in (("logf", lg, rl), ("radius", rad, rr), ("cosf", cs, rc)):
        d = dev.cpu().numpy()
        bad = np.flatnonzero(d.view(np.uint32) != ref.view(np.uint32))
        assert bad.size == 0, f"{name}: {bad.size} mismatches, first k={bad[:8]}"


def test_bm_stats_match_glibc_exception_counts(hses_gpu):
    nlog, ncos = hses_gpu.bm_stats()
    assert nlog > 0 and ncos > 0


@pytest.mark.parametrize("a,b,r,tids,epoch,nreuse", [
    (128, 784, 4, list(range(8)), 0, 0),            # C1 fc1 shape
    (10, 128, 4, [0, 1, 254, 255], 0, 0),           # C1 readout
    (1024, 1024, 1, [0, 1, 2, 4095], 0, 0),         # C2 layer
    (128, 784, 128, [0, 1, 8191], 0, 0),            # C3 fc1 shape
    (128, 128, 128, [5, 6, 7], 3, 2),               # noise_reuse > 0, odd start
    (3, 5, 7, [0, 1, 2, 3, 2**20 + 1], 9, 4),
])
def test_lora_factors_bit_exact(hses_gpu, a, b, r, tids, epoch, nreuse):
    key = 0x9E3779B97F4A7C15 * 3 % 2**64
    bs = O.load().or_base_sigma(0.02, r)
    A, B = hses_gpu.lora_factors(bs, key, r, epoch, nreuse, tids, a, b)
    rA, rB = O.lora_factors(bs, key, r, epoch, tids, a, b, noise_reuse=nreuse)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(A.cpu().numpy().view(np.uint32), rA.view(np.uint32))
    np.testing.assert_array_equal(B.cpu().numpy().view(np.uint32), rB.view(np.uint32))


def test_lora_factors_contiguous_range_equals_tid_list(hses_gpu):
    A1, B1 = hses_gpu.lora_factors(0.1, 7, 8, 0, 0, (3, 6), 16, 24)
    A2, B2 = hses_gpu.lora_factors(0.1, 7, 8, 0, 0, list(range(3, 9)), 16, 24)
    assert torch.equal(A1, A2) and torch.equal(B1, B2)


def test_nonlora_noise_bit_exact(hses_gpu):
    L = O.load()
    out = hses_gpu.nonlora_noise(0.02, 11, 0, 0, [0, 1, 5], 3, 7)
    torch.cuda.synchronize()
    for i, t in enumerate([0, 1, 5]):
        ref = np.zeros((3, 7), np.float32)
        L.or_get_nonlora_update_params(0.02, 11, 0, t, 3, 7, 0, ref)
        np.testing.assert_array_equal(out[i].cpu().numpy().view(np.uint32), ref.view(np.uint32))
