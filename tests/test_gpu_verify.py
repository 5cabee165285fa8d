"""The reference driver's four-path equivalence check (accumulate_train.rs:381-559)
on the GPU path: the chunked forward (B) and the chunked accumulation (D) equal
one batch (A) within 1e-3 of any parameter, the chunk-local z-score (C) does
not (its delta exceeds 1e-3)."""
import pytest

from hyperscalees_amd import snn, verify
from hyperscalees_amd._lib import MATH_BF16, MATH_F32, SGD

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("math,rank,T,chunks", [(MATH_F32, 4, 8, 4), (MATH_BF16, 32, 16, 2)])
def test_four_paths(hses_gpu, math, rank, T, chunks):
    cfg = dict(dims=(784, 128, 128, 128, 10), T=T, rows=16, n=64, rank=rank, sigma=0.02,
               tau_m=10.0, v_th=1.0, math=math, solver=SGD, lr=0.05, poisson_seed=(1, 2, 3, 4))
    pool, labels = snn.synthetic_pool(2000, 784, 10, 0)
    idx = snn.sample_index(0, cfg["n"], cfg["rows"], 2000)
    W = snn.init_weights(cfg["dims"], 0, gain=snn.ACTIVE_GAIN)
    r = verify.verify_paths(cfg, chunks, pool, labels, idx, W)
    print(r)
    assert r["d_ab"] < verify.THRESHOLD, r
    assert r["d_ad"] < verify.THRESHOLD, r
    assert r["d_ac"] > verify.THRESHOLD, r
    # B repeats A's forward and update exactly; D differs only in summation order
    assert r["d_ab"] == 0.0, r
