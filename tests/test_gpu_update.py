"""GPU parity of the ES update (eggroll.rs:353-404, 579-702, 778-915).

The reference value is the oracle's double-accumulated -sqrt(N)/N * sum_i f_i
A_i B_i^T with bit-exact factors; the fp32 bar is rel 1e-5 of the gradient's
scale (max |g|)."""
import math

import numpy as np
import pytest
import torch

from tests import oracle_lib as O

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 2 % 2**64


def oracle_grad(sigma, r, fit, a, b, tid_lo=0, epoch=0, nreuse=0):
    L = O.load()
    bs = L.or_base_sigma(sigma, r)
    g = np.zeros((a, b), np.float64)
    tids = np.arange(tid_lo, tid_lo + fit.size, dtype=np.int32)
    L.or_lora_einsum_f64(bs, KEY, r, nreuse, epoch, np.ascontiguousarray(fit, np.float32), tids,
                         fit.size, a, b, g)
    return g


def gpu_grad(hses_gpu, sigma, r, fit, a, b, scale, tid_lo=0, epoch=0, nreuse=0, out=None,
             accumulate=False):
    ft = torch.from_numpy(np.ascontiguousarray(fit, np.float32)).cuda()
    g = hses_gpu.es_update(ft, tid_lo, KEY, r, sigma, epoch, nreuse, a, b, scale, out=out,
                           accumulate=accumulate)
    torch.cuda.synchronize()
    return g


def assert_close(g, ref, rel=1e-5):
    scale = np.abs(ref).max()
    err = np.abs(g - ref).max()
    assert err <= rel * scale, f"max err {err:.3e} > {rel:.1e} * {scale:.3e}"


@pytest.mark.parametrize("a,b,r,n,tid_lo", [
    (128, 784, 4, 256, 0),      # C1 fc1
    (10, 128, 4, 256, 0),       # C1 readout
    (1024, 1024, 1, 4096, 0),   # C2
    (128, 784, 128, 64, 0),     # C3 fc1 shape, 32 pairs
    (128, 128, 128, 40, 0),
    (70, 33, 5, 31, 3),         # odd start and count: half pairs at both ends
    (16, 40, 37, 12, 1),        # rank not a multiple of 4 with a tail chunk
])
def test_es_update_matches_oracle(hses_gpu, a, b, r, n, tid_lo):
    fit = np.random.default_rng(a + b + r).standard_normal(n).astype(np.float32)
    scale = -math.sqrt(n) / n
    ref = oracle_grad(0.02, r, fit, a, b, tid_lo) * scale
    g = gpu_grad(hses_gpu, 0.02, r, fit, a, b, np.float32(scale), tid_lo).cpu().numpy()
    assert_close(g, ref)


def test_es_update_against_reference_f32_order(hses_gpu):
    # _do_update in the reference's own f32 member order (eggroll.rs:353-404).
    a, b, r, n = 12, 20, 3, 16
    fit = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    ref = np.zeros((a, b), np.float32)
    O.load().or_do_update_lora(0.5, KEY, r, 0, fit, np.zeros(n, np.int32),
                               np.arange(n, dtype=np.int32), n, a, b, ref)
    g = gpu_grad(hses_gpu, 0.5, r, fit, a, b, np.float32(-math.sqrt(n) / n)).cpu().numpy()
    assert_close(g, ref.astype(np.float64), 1e-5)


def test_es_update_chunked_accumulation_equals_full(hses_gpu):
    # accumulated_update: per-chunk contributions summed == one full update.
    a, b, r, n, K = 32, 48, 8, 64, 4
    fit = np.random.default_rng(2).standard_normal(n).astype(np.float32)
    scale = np.float32(-1.0 / math.sqrt(n))
    full = gpu_grad(hses_gpu, 0.1, r, fit, a, b, scale).cpu().numpy()
    out = torch.zeros((a, b), dtype=torch.float32, device="cuda")
    ch = n // K
    for k in range(K):
        gpu_grad(hses_gpu, 0.1, r, fit[k * ch:(k + 1) * ch], a, b, scale, tid_lo=k * ch, out=out,
                 accumulate=True)
    assert_close(out.cpu().numpy(), full.astype(np.float64), 1e-5)


def test_es_update_deterministic(hses_gpu):
    fit = np.random.default_rng(3).standard_normal(512).astype(np.float32)
    g1 = gpu_grad(hses_gpu, 0.02, 16, fit, 128, 128, 1.0)
    g2 = gpu_grad(hses_gpu, 0.02, 16, fit, 128, 128, 1.0)
    assert torch.equal(g1, g2)


def test_es_update_noise_reuse(hses_gpu):
    fit = np.random.default_rng(4).standard_normal(20).astype(np.float32)
    ref = oracle_grad(0.3, 4, fit, 9, 13, epoch=7, nreuse=3)
    g = gpu_grad(hses_gpu, 0.3, 4, fit, 9, 13, 1.0, epoch=7, nreuse=3).cpu().numpy()
    assert_close(g, ref)


# Split-count sweep of the rank-128 contraction (the C3 layers' k_es_rows), as
# the reference sweeps its fused einsum's K-chunk count against an f64 CPU
# value (einsum_pair_fused_oxide.rs:758-795).  At the fc1 shape the split count
# is min(512, pairs / 8): the member counts below give 1, 2, 3, 16, 128 and 511
# splits (48 and 8190 members: pair ranges of unequal length); fc2 and the
# readout at the benched population.  Both forms: the normals drawn in-kernel
# and the factor record of a forward's draw.
SWEEP = [(128, 784, 16), (128, 784, 32), (128, 784, 48), (128, 784, 256), (128, 784, 2048),
         (128, 784, 8190), (128, 128, 8192), (10, 128, 8192)]


@pytest.mark.parametrize("a,b,n", SWEEP)
def test_es_update_split_sweep_rank128(hses_gpu, a, b, n):
    r, sigma = 128, 0.02
    fit = np.random.default_rng(n + a).standard_normal(n).astype(np.float32)
    ref = O.lora_grad_f64(sigma, KEY, r, 0, fit, a, b, nthreads=16).astype(np.float64)
    scale = np.float32(-math.sqrt(n) / n)
    g = gpu_grad(hses_gpu, sigma, r, fit, a, b, scale).cpu().numpy()
    assert_close(g, ref)
    rec = hses_gpu.factor_record(a, b, r, 0, n)
    hses_gpu.pair_factors(KEY, r, sigma, 0, 0, 0, n, a, b, rec, None)
    ft = torch.from_numpy(fit).cuda()
    gr = hses_gpu.es_update_rec(ft, 0, rec, r, sigma, a, b, scale).cpu().numpy()
    torch.cuda.synchronize()
    assert_close(gr, ref)
    # the two forms run the same contraction on the same factors
    assert np.array_equal(g, gr)


# The reference's own sweep of its fused ES contraction against an f64 CPU
# value (einsum_pair_fused_oxide.rs:758-795): (pairs, rank, a, b), the
# contraction length K = pairs x rank bisected over 1..64 chunks of 32, large K
# against small outputs and the reverse, the a thresholds of its small-M path,
# one K slice over many N blocks and the reverse, the fc3 (a = 10) and fc1
# (b = 784) shapes, and the noise-bench shape.  (Its pitched variants have no
# counterpart: the gradient here is a dense (a, b) array.)  Ranks that are a
# multiple of 16 in [32, 128] also run the record form.
REF_SWEEP = [(8, 3, 2, 3), (2, 16, 8, 8), (2, 32, 8, 8), (4, 32, 8, 8), (8, 64, 8, 8),
             (16, 64, 8, 8), (32, 64, 8, 8), (50, 64, 8, 128), (50, 64, 64, 8), (2, 64, 12, 8),
             (2, 64, 16, 8), (2, 64, 24, 8), (2, 64, 32, 8), (50, 64, 64, 128),
             (100, 64, 64, 48), (100, 64, 64, 128), (64, 64, 10, 128), (200, 64, 128, 784),
             (1000, 16, 32, 48), (2, 64, 32, 48)]


@pytest.mark.parametrize("pairs,r,a,b", REF_SWEEP)
def test_es_update_reference_sweep(hses_gpu, pairs, r, a, b):
    n, sigma = 2 * pairs, 0.02
    fit = np.random.default_rng(pairs * 7 + r + a + b).standard_normal(n).astype(np.float32)
    ref = O.lora_grad_f64(sigma, KEY, r, 0, fit, a, b, nthreads=8).astype(np.float64)
    scale = np.float32(-math.sqrt(n) / n)
    g = gpu_grad(hses_gpu, sigma, r, fit, a, b, scale).cpu().numpy()
    assert_close(g, ref)
    if r % 16 == 0 and 32 <= r <= 128:
        rec = hses_gpu.factor_record(a, b, r, 0, n)
        hses_gpu.pair_factors(KEY, r, sigma, 0, 0, 0, n, a, b, rec, None)
        gr = hses_gpu.es_update_rec(torch.from_numpy(fit).cuda(), 0, rec, r, sigma, a, b,
                                    scale).cpu().numpy()
        assert np.array_equal(g, gr)
