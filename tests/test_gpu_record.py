"""The factor record: the *_rec forwards keep every antithetic pair's raw
normals, and hses_es_update_rec reads them instead of drawing them again.

Pinned against the generating paths, which the oracle pins elsewhere: the
record equals hses_lora_factors' factors (B as drawn, A = record * sign *
base_sigma), the forwards' outputs are unchanged, and the update from the
record equals hses_es_update bit for bit (same operands, tiles and order),
also inside whole SNN steps."""
import numpy as np
import pytest
import torch

from hyperscalees_amd import kernels as K
from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAMW, FMT_F32, MATH_BF16, MATH_F32X, SGD
from tests import oracle_lib as O
from tests.test_gpu_linear import pack_bits

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 5 % 2**64


def pairs_of(tid_lo, n):
    return (tid_lo + n - 1) // 2 - tid_lo // 2 + 1


def check_record(rec, a, b, r, sigma, tid_lo, n, epoch, nreuse):
    """rec against hses_lora_factors of the same members, exactly."""
    P = pairs_of(tid_lo, n)
    view = rec[: P * r * (a + b)].view(P, r, a + b)
    bs = np.float32(O.load().or_base_sigma(sigma, r))
    A, B = K.lora_factors(float(bs), KEY, r, epoch, nreuse, (tid_lo, n), a, b)
    for m in range(n):
        p = (tid_lo + m) // 2 - tid_lo // 2
        assert torch.equal(view[p, :, :b].t(), B[m]), f"B of member {m}"
        a_abs = view[p, :, b:].t() * torch.tensor(bs, device="cuda")
        ok_pos = torch.equal(A[m], a_abs)
        ok_neg = torch.equal(A[m], -a_abs)
        assert ok_pos or ok_neg, f"A of member {m}"
        if m > 0 and (tid_lo + m) % 2 == 1:  # the pair's partner has the opposite sign
            assert torch.equal(A[m], -A[m - 1])


@pytest.mark.parametrize("a,b,r,n,tid_lo,T,epoch,nreuse", [
    (128, 784, 128, 6, 0, 16, 0, 0),    # C3 fc1 shape, three pairs
    (128, 128, 64, 5, 3, 4, 2, 0),      # odd start and count: half pairs at both ends
    (96, 200, 48, 4, 1, 2, 1, 3),       # rank 48 (a short rank chunk), noise reuse
])
def test_lif_forward_record(hses_gpu, a, b, r, n, tid_lo, T, epoch, nreuse):
    rng = np.random.default_rng(a + b + r)
    rows, sigma = 8, 0.05
    x = pack_bits((rng.random((T, n * rows, b)) < 0.3).astype(np.float32))
    W = torch.from_numpy((3.0 * rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)).cuda()
    s0, q0 = K.perturbed_linear_lif(x, W, KEY, r, sigma, epoch, nreuse, tid_lo, n, rows, T, 10.0,
                                    1.0, want_spikes=True, want_rate=True)
    s0, q0 = s0.clone(), q0.clone()
    rec = K.factor_record(a, b, r, tid_lo, n)
    rec.fill_(float("nan"))
    s1, q1 = K.perturbed_linear_lif(x, W, KEY, r, sigma, epoch, nreuse, tid_lo, n, rows, T, 10.0,
                                    1.0, want_spikes=True, want_rate=True, rec=rec)
    torch.cuda.synchronize()
    assert torch.equal(s0, s1) and torch.equal(q0, q1)
    assert s0.any(), "no spikes: the case checks nothing"
    assert not torch.isnan(rec).any(), "record not fully written"
    check_record(rec, a, b, r, sigma, tid_lo, n, epoch, nreuse)
    # the update from the record equals the generating update
    fit = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    scale = np.float32(-1.0 / np.sqrt(n))
    g0 = K.es_update(fit, tid_lo, KEY, r, sigma, epoch, nreuse, a, b, scale)
    g1 = K.es_update_rec(fit, tid_lo, rec, r, sigma, a, b, scale)
    acc = g0.clone()
    K.es_update_rec(fit, tid_lo, rec, r, sigma, a, b, scale, out=acc, accumulate=True)
    g2 = K.es_update(fit, tid_lo, KEY, r, sigma, epoch, nreuse, a, b, scale, out=g0.clone(),
                     accumulate=True)
    torch.cuda.synchronize()
    assert torch.equal(g0, g1)
    assert torch.equal(acc, g2)


@pytest.mark.parametrize("a,b,r,n,tid_lo", [
    (10, 128, 128, 6, 0),     # C3 readout on rates
    (40, 96, 32, 7, 2),       # several pairs per generation group
])
def test_linear_forward_record(hses_gpu, a, b, r, n, tid_lo):
    rng = np.random.default_rng(a * b + n)
    rows, sigma = 16, 0.02
    x = torch.from_numpy(rng.random((n * rows, b)).astype(np.float32)).cuda()
    W = torch.from_numpy((rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)).cuda()
    y0 = K.perturbed_linear(x, W, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_F32,
                            math=MATH_BF16).clone()
    rec = K.factor_record(a, b, r, tid_lo, n)
    rec.fill_(float("nan"))
    y1 = K.perturbed_linear(x, W, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_F32,
                            math=MATH_BF16, rec=rec)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    assert not torch.isnan(rec).any()
    check_record(rec, a, b, r, sigma, tid_lo, n, 0, 0)
    fit = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    g0 = K.es_update(fit, tid_lo, KEY, r, sigma, 0, 0, a, b, np.float32(0.5))
    g1 = K.es_update_rec(fit, tid_lo, rec, r, sigma, a, b, np.float32(0.5))
    torch.cuda.synchronize()
    assert torch.equal(g0, g1)


C3_SMALL = dict(dims=(784, 128, 128, 128, 10), T=16, rows=64, n=8, rank=128, sigma=0.02,
                tau_m=10.0, v_th=1.0, math=MATH_BF16, solver=ADAMW, lr=0.01,
                poisson_seed=(5, 6, 7, 8))


def make(cfg, record, seed=0, pool_size=3000):
    pool, labels = snn.synthetic_pool(pool_size, cfg.dims[0], cfg.dims[-1], seed)
    idx = snn.sample_index(seed, cfg.n, cfg.rows, pool_size)
    W = snn.init_weights(cfg.dims, seed, gain=snn.ACTIVE_GAIN)
    # the factored forward (member weights would change the arithmetic)
    return snn.SnnEs(cfg, W, pool, labels, idx, fused=True, record=record, member_weights=False)


@pytest.mark.parametrize("extra", [dict(), dict(accumulate=2, solver=SGD, lr=0.05)])
def test_snn_steps_with_record_equal_generating(hses_gpu, extra):
    cfg = dict(C3_SMALL, **extra)
    es_g = make(snn.SnnConfig(**cfg), record=False)
    es_r = make(snn.SnnConfig(**cfg), record=True)
    assert es_r.rec is not None and es_g.rec is None
    for epoch in range(2):
        f_g = es_g.step(epoch).clone()
        f_r = es_r.step(epoch).clone()
        torch.cuda.synchronize()
        assert torch.equal(f_g, f_r)
        for l in range(es_g.L):
            assert torch.equal(es_g.grads[l], es_r.grads[l]), f"layer {l} gradient, epoch {epoch}"
            assert torch.equal(es_g.W[l], es_r.W[l])
    assert any(g.abs().max() > 0 for g in es_r.grads)


def test_update_without_matching_forward_draws_the_normals(hses_gpu):
    # a record holds one epoch's normals: an update for another epoch must not read it
    cfg = snn.SnnConfig(**dict(C3_SMALL, solver=SGD, lr=0.05))
    es_r = make(cfg, record=True)
    es_g = make(cfg, record=False)
    fit = es_r.forward(0).clone()
    es_g.forward(0)
    es_r.update(fit, epoch=1)
    es_g.update(fit, epoch=1)
    torch.cuda.synchronize()
    for l in range(es_r.L):
        assert torch.equal(es_r.grads[l], es_g.grads[l])


@pytest.mark.parametrize("math", [MATH_F32X, MATH_BF16])
def test_noise_cache_steps_equal_redrawn(hses_gpu, math):
    # noise_reuse = 0: the factors depend on the layer key and thread id only
    # (eggroll.rs:60-65), so keeping the records across epochs (the reference's
    # LoraNoiseCache, eggroll.rs:229-309, 627) gives the steps that redraw them
    cfg = dict(C3_SMALL, math=math)
    pool, labels = snn.synthetic_pool(3000, 784, 10, 0)
    idx = snn.sample_index(0, cfg["n"], cfg["rows"], 3000)
    W = snn.init_weights(snn.SnnConfig(**cfg).dims, 0, gain=snn.ACTIVE_GAIN)
    es_d = snn.SnnEs(snn.SnnConfig(**cfg), W, pool, labels, idx)
    es_c = snn.SnnEs(snn.SnnConfig(**cfg), W, pool, labels, idx, noise_cache=True)
    assert es_c.noise_cache and es_c.mw and not es_c.overlap
    for epoch in range(3):
        f_d = es_d.step(epoch).clone()
        f_c = es_c.step(epoch).clone()
        torch.cuda.synchronize()
        assert torch.equal(f_d, f_c), f"epoch {epoch}"
        for l in range(es_d.L):
            assert torch.equal(es_d.grads[l], es_c.grads[l]), f"layer {l} gradient, epoch {epoch}"
            assert torch.equal(es_d.W[l], es_c.W[l])


def test_noise_cache_rejects_epoch_dependent_noise(hses_gpu):
    cfg = snn.SnnConfig(**dict(C3_SMALL, noise_reuse=2))
    pool, labels = snn.synthetic_pool(100, 784, 10, 0)
    idx = snn.sample_index(0, cfg.n, cfg.rows, 100)
    W = snn.init_weights(cfg.dims, 0)
    with pytest.raises(ValueError, match="noise_reuse = 0"):
        snn.SnnEs(cfg, W, pool, labels, idx, noise_cache=True)
