"""The allocation-free ES update (hses_es_update_noalloc) against
hses_es_update through the C ABI: two calls in a row on the library's fixed
device scratch, the second with a smaller input, each within the fp32 bar
(rel 1e-5 of the gradient's scale; the split count, hence the summation
order, may differ).  Also the size limit and the accumulate form."""
import ctypes

import numpy as np
import pytest
import torch

from hyperscalees_amd import _lib
from hyperscalees_amd import kernels as K

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 3 % 2**64
SCRATCH = 32 << 20


def noalloc(fit, tid_lo, rank, sigma, a, b, scale, out, accumulate=0):
    _lib.call("hses_es_update_noalloc", K._p(fit), fit.numel(), tid_lo, KEY, rank, sigma, 0, 0,
              a, b, scale, accumulate, K._p(out), K._stream())
    return out


def close(got, ref, rel=1e-5):
    g, r = got.cpu().numpy().astype(np.float64), ref.cpu().numpy().astype(np.float64)
    assert np.abs(g - r).max() <= rel * np.abs(r).max(), (np.abs(g - r).max(), np.abs(r).max())


@pytest.mark.parametrize("first,second", [
    ((8192, 128, 128, 784, 0), (1000, 128, 10, 128, 1)),   # C3 fc1, then the readout
    ((4096, 1, 1024, 1024, 0), (300, 1, 96, 512, 3)),     # C2 layer (r < 32 path), then smaller
])
def test_noalloc_matches_workspace_entry_point(hses_gpu, first, second):
    rng = np.random.default_rng(1)
    for n, rank, a, b, tid_lo in (first, second):
        fit = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
        scale = np.float32(-np.sqrt(n) / n)
        ref = hses_gpu.es_update(fit, tid_lo, KEY, rank, 0.02, 0, 0, a, b, scale)
        got = torch.full((a, b), np.nan, dtype=torch.float32, device="cuda")
        noalloc(fit, tid_lo, rank, 0.02, a, b, scale, got)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        close(got, ref)


def test_noalloc_accumulate_and_limit(hses_gpu):
    rng = np.random.default_rng(2)
    a, b, rank, n = 128, 128, 128, 512
    f1 = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    f2 = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    ref = hses_gpu.es_update(f1, 0, KEY, rank, 0.02, 0, 0, a, b, np.float32(1.0))
    hses_gpu.es_update(f2, n, KEY, rank, 0.02, 0, 0, a, b, np.float32(1.0), out=ref,
                       accumulate=True)
    got = torch.zeros((a, b), dtype=torch.float32, device="cuda")
    noalloc(f1, 0, rank, 0.02, a, b, np.float32(1.0), got)
    noalloc(f2, n, rank, 0.02, a, b, np.float32(1.0), got, accumulate=1)
    torch.cuda.synchronize()
    close(got, ref)
    # one fp32 partial of a * b elements plus the scale words must fit the scratch
    big = SCRATCH // 4
    lib = _lib.load()
    rc = lib.hses_es_update_noalloc(K._p(f1), n, 0, KEY, rank, 0.02, 0, 0, big // 4096, 4096,
                                    1.0, 0, K._p(got), K._stream())
    assert rc == _lib.HSES_ERR_INVALID_ARG and b"scratch" in _lib.last_error().encode()
