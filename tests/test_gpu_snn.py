"""GPU parity of the SNN-MLP ES step against the oracle.

Layer by layer (C1, fp32): each hidden layer's currents are recomputed by the
oracle from the GPU's own (bit-exact) input spikes, so a layer is judged on
its own error: currents within rel 1e-5, LIF spike mismatches <= 1e-4 of all
spikes.  End to end: member fitness against the oracle's composition, and the
updated weights after one ES step against the oracle's double-accumulated
gradient and solver on the same fitness."""
import math

import numpy as np
import pytest
import torch

from hyperscalees_amd import kernels as K
from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAMW, FMT_BITS, MATH_BF16, MATH_F32, SGD
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu


def unpack(words, width):
    w = words.cpu().numpy().view(np.uint64)
    bits = ((w[..., None] >> np.arange(64, dtype=np.uint64)) & np.uint64(1)).astype(np.float32)
    return bits.reshape(*w.shape[:-1], -1)[..., :width]


def make(cfg, pool_size=3000, seed=0, fused=False, member_weights=None):
    pool, labels = snn.synthetic_pool(pool_size, cfg.dims[0], cfg.dims[-1], seed)
    idx = snn.sample_index(seed, cfg.n, cfg.rows, pool_size)
    W = snn.init_weights(cfg.dims, seed, gain=snn.ACTIVE_GAIN)
    return (snn.SnnEs(cfg, W, pool, labels, idx, fused=fused, member_weights=member_weights),
            pool, labels, idx, W)


def oracle_layer(x_tm, W, cfg, l):
    """Currents (T, M, a) of layer l from time-major input x_tm (T, M, b)."""
    T, M, b = x_tm.shape
    a = W.shape[0]
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    A, B = O.lora_factors(bs, cfg.keys[l], cfg.rank, 0, np.arange(cfg.n), a, b)
    y = np.zeros((T, M, a), np.float32)
    for m in range(cfg.n):
        xs = x_tm[:, m * cfg.rows:(m + 1) * cfg.rows].reshape(-1, b)
        y[:, m * cfg.rows:(m + 1) * cfg.rows] = O.do_mm(xs, W, A[m], B[m]).reshape(T, cfg.rows, a)
    return y


def oracle_fitness(cfg, W, pool, labels, idx, nthreads=8):
    L = O.load()
    dims = np.array(cfg.dims, np.int32)
    c = O.SnnCfg()
    c.n_layers = len(cfg.dims) - 1
    c.dims = dims.ctypes.data_as(O.ctypes.POINTER(O.c_i32))
    c.T, c.rows, c.tau_m, c.v_th, c.sigma = cfg.T, cfg.rows, cfg.tau_m, cfg.v_th, cfg.sigma
    c.rank, c.noise_reuse, c.epoch = cfg.rank, cfg.noise_reuse, 0
    for i in range(4):
        c.poisson_seed[i] = cfg.poisson_seed[i]
    probs = np.ascontiguousarray(pool[idx], np.float32)
    lab = np.ascontiguousarray(labels[idx], np.int32)
    Ws = [np.ascontiguousarray(w) for w in W]
    Wp = (O.ctypes.c_void_p * len(Ws))(*[w.ctypes.data for w in Ws])
    keys = (O.c_u64 * len(cfg.keys))(*cfg.keys)
    fit = np.zeros(cfg.n, np.float32)
    L.or_snn_forward_members(O.ctypes.byref(c), Wp, keys, probs, lab, 0, cfg.n, nthreads, fit)
    return fit


C1 = dict(dims=(784, 128, 128, 128, 10), T=8, rows=64, n=256, rank=4, sigma=0.02, tau_m=10.0,
          v_th=1.0, math=MATH_F32, solver=SGD, lr=0.05, poisson_seed=(1, 2, 3, 4))


def test_c1_layerwise_parity(hses_gpu):
    cfg = snn.SnnConfig(**C1)
    es, pool, labels, idx, W = make(cfg)
    es.poisson()
    torch.cuda.synchronize()
    ref0 = O.poisson(pool[idx], cfg.T, cfg.poisson_seed)
    np.testing.assert_array_equal(unpack(es.spikes_tm(0), cfg.dims[0]), ref0)
    total = mism = 0
    for l in range(es.L - 1):
        es.hidden_layer(l, 0)
        torch.cuda.synchronize()
        x = unpack(es.spikes_tm(l), cfg.dims[l])
        a = cfg.dims[l + 1]
        cur_ref = oracle_layer(x, W[l], cfg, l)
        cur_gpu = es.cur.view(-1)[: cur_ref.size].view(cur_ref.shape).cpu().numpy()
        err = np.abs(cur_gpu - cur_ref).max()
        assert err <= 1e-5 * np.abs(cur_ref).max(), f"layer {l} currents err {err}"
        spk_ref, _ = O.lif(cur_ref, cfg.tau_m, cfg.v_th)
        spk_gpu = unpack(es.spikes_tm(l + 1), a)
        # LIF on the GPU's own currents is bit-exact; flips come only from
        # current rounding near the threshold
        spk_own, _ = O.lif(cur_gpu, cfg.tau_m, cfg.v_th)
        np.testing.assert_array_equal(spk_gpu, spk_own)
        mism += int((spk_gpu != spk_ref).sum())
        total += int(spk_ref.sum())  # the bar counts spikes that fired, not slots
        assert spk_gpu.mean() > 0.005, "layer is silent; the test would pin nothing"
    print(f"C1 spike mismatches {mism} of {total} reference spikes")
    assert mism <= 1e-4 * total, f"spike mismatches {mism} of {total} reference spikes"


def test_c1_fitness_and_update(hses_gpu):
    cfg = snn.SnnConfig(**C1)
    es, pool, labels, idx, W = make(cfg)
    fit = es.forward(0)
    torch.cuda.synchronize()
    fit_gpu = fit.cpu().numpy()
    fit_ref = oracle_fitness(cfg, W, pool, labels, idx)
    np.testing.assert_allclose(fit_gpu, fit_ref, rtol=1e-4, atol=1e-4)
    # update on the GPU's fitness, against the oracle on the same fitness
    W_before = [w.cpu().numpy().copy() for w in es.W]
    es.update(fit, 0)
    torch.cuda.synchronize()
    z, _, _ = O.convert_fitnesses(fit_gpu)
    for l in range(es.L):
        a, b = W_before[l].shape
        g = O.lora_grad_f64(cfg.sigma, cfg.keys[l], cfg.rank, 0, z, a, b)
        g_gpu = es.grads[l].cpu().numpy()
        err = np.abs(g_gpu - g).max()
        assert err <= 1e-5 * np.abs(g).max(), f"layer {l} gradient err {err}"
        # SGD step p - g*lr (noiser.rs:161-165): within 2 ulps of the f32
        # parameter plus the gradient tolerance carried through lr
        p_ref = W_before[l] - g * np.float32(cfg.lr)
        w_gpu = es.W[l].cpu().numpy()
        ulp = np.spacing(np.abs(p_ref).astype(np.float32))
        tol = 2 * ulp + 1e-5 * np.abs(g).max() * cfg.lr
        assert np.all(np.abs(w_gpu - p_ref) <= tol), f"layer {l} parameter step"


C3_SMALL = dict(dims=(784, 128, 128, 128, 10), T=16, rows=64, n=8, rank=128, sigma=0.02,
                tau_m=10.0, v_th=1.0, math=MATH_BF16, solver=ADAMW, lr=0.01,
                poisson_seed=(5, 6, 7, 8))


def test_c3_shape_bf16_step(hses_gpu):
    # bf16 path at the north-star shape (8 members): each layer within the
    # bf16 bar against the oracle's fp32 currents on the GPU's own inputs, and
    # the ES update within the fp32 bar on the GPU's fitness.
    # Spikes: against the LIF of float64 currents with the kernel's bf16
    # arithmetic, mismatches <= 1e-4 of the reference spikes; against the
    # fp32 oracle's currents <= 2e-2 (the bf16-path bar).
    from tests.test_gpu_c3_full import member_currents
    cfg = snn.SnnConfig(**C3_SMALL)
    es, pool, labels, idx, W = make(cfg)
    es.poisson()
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    R = cfg.rows
    for l in range(es.L - 1):
        es.hidden_layer(l, 0)
        torch.cuda.synchronize()
        x = unpack(es.spikes_tm(l), cfg.dims[l])
        cur_ref = oracle_layer(x, W[l], cfg, l)
        cur_gpu = es.cur.view(-1)[: cur_ref.size].view(cur_ref.shape).cpu().numpy()
        err = np.abs(cur_gpu - cur_ref).max()
        assert err <= 2e-2 * np.abs(cur_ref).max(), f"layer {l} bf16 currents err {err}"
        a = cfg.dims[l + 1]
        A, B = O.lora_factors(bs, cfg.keys[l], cfg.rank, 0, np.arange(cfg.n), a, cfg.dims[l])
        cur_bf = np.concatenate([member_currents(x[:, m * R:(m + 1) * R], W[l], A[m], B[m], True)
                                 for m in range(cfg.n)], axis=1)
        spk_gpu = unpack(es.spikes_tm(l + 1), a)
        spk_bf, _ = O.lif(cur_bf.astype(np.float32), cfg.tau_m, cfg.v_th)
        spk_32, _ = O.lif(cur_ref, cfg.tau_m, cfg.v_th)
        n_ref = int(spk_32.sum())
        m_bf, m_32 = int((spk_gpu != spk_bf).sum()), int((spk_gpu != spk_32).sum())
        print(f"layer {l}: {n_ref} spikes, mismatches bf16-arith {m_bf}, fp32 {m_32}")
        assert n_ref > 0 and m_bf <= 1e-4 * n_ref and m_32 <= 2e-2 * n_ref, f"layer {l} spikes"
    fit = es.readout(0)
    W_before = [w.cpu().numpy().copy() for w in es.W]
    es.update(fit, 0)
    torch.cuda.synchronize()
    z, _, _ = O.convert_fitnesses(fit.cpu().numpy())
    l = 1
    g = O.lora_grad_f64(cfg.sigma, cfg.keys[l], cfg.rank, 0, z, 128, 128)
    assert np.allclose(es.grads[l].cpu().numpy(), g, rtol=0, atol=1e-5 * np.abs(g).max())


def test_c3_fused_forward_equals_unfused(hses_gpu):
    # The fused forward+LIF path computes the same currents and the same LIF
    # update in-kernel, so spikes, rates and fitness are identical bit for bit.
    cfg = snn.SnnConfig(**C3_SMALL)
    es_u, *_ = make(cfg, fused=False)
    es_f, *_ = make(cfg, fused=True, member_weights=False)
    assert es_f.fused and not es_u.fused
    fit_u = es_u.forward(0)
    fit_f = es_f.forward(0)
    torch.cuda.synchronize()
    for l in range(1, es_u.L - 1):
        assert torch.equal(es_u.spikes_tm(l), es_f.spikes_tm(l)), f"layer {l} spikes"
    assert torch.equal(es_u.rate, es_f.rate)
    assert torch.equal(fit_u, fit_f)
    assert float(es_f.rate.mean()) > 0.005


@pytest.mark.parametrize("n,K,fused", [(16, 2, False), (9, 3, False), (16, 4, True)])
def test_k_chunk_step_equals_one_chunk(hses_gpu, n, K, fused):
    # accumulate_train.rs:770-944: K chunks with frozen parameters, raw-weighted
    # gradients and the affine z-score (combine_affine_grads) == the one-chunk
    # step on z-scored fitness, the identity of eggroll.rs:1502-1568.  Chunk
    # Poisson seeds continue the whole-population encode, so every member's
    # fitness is bit-identical; n=9, K=3 splits pairs across chunks and leaves
    # an unpaired last member (its ones term is the only non-zero one).
    base = dict(C3_SMALL if fused else C1, n=n, solver=SGD, lr=0.05)
    es1, *_ = make(snn.SnnConfig(**base), fused=fused)
    esk, *_ = make(snn.SnnConfig(**base, accumulate=K), fused=fused)
    W0 = [w.cpu().numpy().copy() for w in es1.W]
    f1 = es1.step(0).clone()
    fk = esk.step(0).clone()
    torch.cuda.synchronize()
    assert torch.equal(f1, fk)
    assert int(es1.correct) == int(esk.correct) and int(esk.correct) > 0
    for l in range(es1.L):
        g1, gk = es1.grads[l].cpu().numpy(), esk.grads[l].cpu().numpy()
        gmax = np.abs(g1).max()
        assert gmax > 0 and np.abs(gk - g1).max() <= 1e-5 * gmax, f"layer {l} gradient"
        w1, wk = es1.W[l].cpu().numpy(), esk.W[l].cpu().numpy()
        tol = 2 * np.spacing(np.abs(W0[l])) + 1e-5 * gmax * base["lr"]
        assert np.all(np.abs(wk - w1) <= tol), f"layer {l} parameter step"


def test_k_chunk_step_matches_oracle_two_phase(hses_gpu):
    # The K-chunk gradient against the oracle's two-phase accumulated_update
    # (eggroll.rs:579-702: global z-score, per-chunk einsum, -1/sqrt(batch)) on
    # the GPU's own raw fitness.
    cfg = snn.SnnConfig(**dict(C1, n=12, accumulate=3))
    es, *_ = make(cfg)
    raw = es.step(0).cpu().numpy()
    torch.cuda.synchronize()
    conv, _, _ = O.convert_fitnesses(raw)
    tids = np.arange(cfg.n, dtype=np.int32)
    for l in range(es.L):
        a, b = es.W[l].shape
        ref = np.zeros((a, b), np.float32)
        O.load().or_accumulated_lora_grad(cfg.sigma, cfg.keys[l], cfg.rank, 0, 0, conv, tids,
                                          cfg.accumulate, cfg.chunk, a, b, ref)
        g = es.grads[l].cpu().numpy()
        assert np.abs(g - ref).max() <= 1e-5 * np.abs(ref).max(), f"layer {l}"
