"""GPU parity of the dense (PARAM-class) ES path and the TrustRegion solver.

* hses_noisy_standard: get_noisy_standard_impl (eggroll.rs:480-503), each
  member's param + sign*sigma*noise, bit-exact against the oracle's
  get_nonlora_update_params (pinned by the do_update sign test).
* hses_full_update: _simple_full_update + _do_update (eggroll.rs:331-350,
  384-404) against a float64 sum of the oracle's per-member f32 terms (rel
  1e-5) and the oracle's own f32 sequential do_update (rel 1e-4).
* hses_clip_global_norm + hses_solver_step_scaled: clip_grads_global_norm and
  Solver::TrustRegion (noiser.rs:215-244) against the pinned oracle clip
  factor and solver step.
"""
import math

import numpy as np
import pytest
import torch

from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAM, ADAMW, MATH_F32, SGD
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 5 % 2**64


def oracle_noise(sigma, key, epoch, tid, a, b, nreuse=0):
    out = np.zeros(a * b, np.float32)
    O.load().or_get_nonlora_update_params(sigma, key, epoch, tid, a, b, nreuse, out)
    return out.reshape(a, b)


@pytest.mark.parametrize("a,b,tids,epoch,nreuse", [
    (1, 1, (0, 6), 0, 0),              # out_gain / v_th leaves, (1, 1)
    (1, 512, (3, 5), 0, 0),            # a d_model vector, odd first member
    (3, 1000, [7, 2, 9, 0], 4, 2),     # explicit thread ids, noise_reuse epochs
    (2, 257, (0, 3), 0, 0),            # row length with no divisor <= 256 but 1
])
def test_noisy_standard_bit_exact(hses_gpu, a, b, tids, epoch, nreuse):
    rng = np.random.default_rng(a * b)
    param = rng.standard_normal((a, b)).astype(np.float32)
    sigma = 0.05
    out = hses_gpu.noisy_standard(torch.from_numpy(param).cuda(), KEY, sigma, epoch, nreuse, tids)
    torch.cuda.synchronize()
    ids = list(range(tids[0], tids[0] + tids[1])) if isinstance(tids, tuple) else tids
    got = out.cpu().numpy()
    for i, t in enumerate(ids):
        ref = param + oracle_noise(sigma, KEY, epoch, t, a, b, nreuse)
        np.testing.assert_array_equal(got[i], ref, err_msg=f"member {t}")


def dense_grad_f64(fit, tid_lo, sigma, key, a, b, epoch=0, nreuse=0):
    """sum_m (noise_m * f_m) with each term in f32 (as the reference forms it), summed in float64."""
    acc = np.zeros((a, b), np.float64)
    for m, f in enumerate(fit):
        up = oracle_noise(sigma, key, epoch, tid_lo + m, a, b, nreuse)
        acc += (up * np.float32(f)).astype(np.float64)
    return acc


@pytest.mark.parametrize("n,tid_lo,a,b", [(2048, 0, 1, 512), (9, 1, 1, 1), (300, 5, 4, 700),
                                          (64, 0, 40, 1000)])
def test_full_update(hses_gpu, n, tid_lo, a, b):
    rng = np.random.default_rng(n + a)
    fit = rng.standard_normal(n).astype(np.float32)
    sigma = 0.02
    scale = np.float32(-math.sqrt(n) / n)
    g = hses_gpu.full_update(torch.from_numpy(fit).cuda(), tid_lo, KEY, sigma, 0, 0, a, b, scale)
    torch.cuda.synchronize()
    got = g.cpu().numpy()
    ref = dense_grad_f64(fit, tid_lo, sigma, KEY, a, b) * float(scale)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # the oracle's own do_update (f32 sequential sum, then * (1/N) * sqrt(N), negated)
    ref32 = np.zeros((a, b), np.float32)
    tids = np.arange(tid_lo, tid_lo + n, dtype=np.int32)
    O.load().or_do_update_full(sigma, KEY, 0, 0, fit, np.zeros(n, np.int32), tids, n, a, b, ref32)
    assert np.abs(got - ref32).max() <= 1e-4 * np.abs(ref32).max()


def test_full_update_accumulates_chunks(hses_gpu):
    # K chunks with accumulate == one call over all members (thread ids continue)
    rng = np.random.default_rng(3)
    fit = torch.from_numpy(rng.standard_normal(96).astype(np.float32)).cuda()
    one = hses_gpu.full_update(fit, 0, KEY, 0.1, 0, 0, 3, 200, np.float32(1.0))
    acc = torch.empty_like(one)
    for k in range(3):
        hses_gpu.full_update(fit[32 * k:32 * (k + 1)].contiguous(), 32 * k, KEY, 0.1, 0, 0, 3, 200,
                             np.float32(1.0), out=acc, accumulate=k > 0)
    torch.cuda.synchronize()
    g1, gk = one.cpu().numpy(), acc.cpu().numpy()
    assert np.abs(g1 - gk).max() <= 1e-6 * np.abs(g1).max()


@pytest.mark.parametrize("max_norm,expect_clip", [(0.5, True), (1e6, False)])
def test_clip_global_norm_and_scaled_step(hses_gpu, max_norm, expect_clip):
    rng = np.random.default_rng(11)
    shapes = [(128, 784), (128, 128), (10, 128), (1, 1)]
    grads = [(rng.standard_normal(s) * 0.01).astype(np.float32) for s in shapes]
    g_dev = [torch.from_numpy(g).cuda() for g in grads]
    scale = hses_gpu.clip_global_norm(g_dev, max_norm)
    torch.cuda.synchronize()
    ref = O.clip_scale(grads, max_norm)
    got = float(scale.cpu().numpy()[0])
    if expect_clip:
        assert ref < 1.0 and abs(got - ref) <= 1e-6 * ref
    else:
        assert got == 1.0 and ref == 1.0
    # the inner solver on the clipped gradient (TrustRegion = clip then inner)
    for kind in (SGD, ADAM, ADAMW):
        p = rng.standard_normal((128, 128)).astype(np.float32)
        pd = torch.from_numpy(p).cuda()
        m = torch.zeros_like(pd)
        v = torch.zeros_like(pd)
        wd = 1e-4 if kind == ADAMW else 0.0
        hses_gpu.solver_step(kind, 0.01, pd, g_dev[1], m, v, step_t=1, wd=wd, gscale=scale)
        torch.cuda.synchronize()
        gc = (grads[1] * np.float32(got)).astype(np.float32)
        out = np.zeros_like(p)
        O.load().or_solver_step(kind, 0.01, 0.9, 0.999, 1e-8, wd, 1, p.ravel(), gc.ravel(),
                                np.zeros(p.size, np.float32), np.zeros(p.size, np.float32),
                                p.size, out.reshape(-1))
        np.testing.assert_allclose(pd.cpu().numpy(), out, rtol=1e-6, atol=1e-8)


def test_snn_step_with_trust_region(hses_gpu):
    # SnnEs with max_norm: every layer's gradient of the step is clipped by the
    # one global factor before SGD (Solver::TrustRegion wrapping Sgd)
    from tests.test_gpu_snn import C1, make
    cfg = snn.SnnConfig(**dict(C1, n=32, solver=SGD, lr=0.05, max_norm=0.01))
    es, *_ = make(cfg)
    W0 = [w.cpu().numpy().copy() for w in es.W]
    es.step(0)
    torch.cuda.synchronize()
    grads = [g.cpu().numpy() for g in es.grads]
    sc = O.clip_scale(grads, cfg.max_norm)
    assert sc < 1.0, "the test needs the clip to apply"
    for l in range(es.L):
        p_ref = W0[l] - (grads[l] * np.float32(sc)) * np.float32(cfg.lr)
        tol = 2 * np.spacing(np.abs(p_ref)) + 1e-6 * np.abs(grads[l]).max() * cfg.lr
        assert np.all(np.abs(es.W[l].cpu().numpy() - p_ref) <= tol), f"layer {l}"
