"""The headline configuration C3 at its full size (N = 8192 members, r = 128,
T = 16, 64 samples per member), run through the product path (bit-packed
Poisson, factors drawn ahead, member weights W_m = W + A_m B_m^T formed once
per member and the fused forward + LIF on them, bf16 math) and checked on
sampled members against the oracle.

Members are sampled at both ends of the population, on either side of pair
255 / 256 (where the persistent forward kernel's workgroups wrap around to
their second pair) and in the middle.  Each layer is judged on the GPU's own
input spikes, so a single spike flip does not cascade into later layers:

* input spikes: bit-exact against the oracle's Poisson encode;
* hidden layers: spikes against the LIF scan of float64 currents computed with
  the kernel's bf16 arithmetic (x times the bf16 rounding of W_m, formed to
  fp32 accuracy):
  mismatches <= 1e-4 of the reference spikes; against the fp32 oracle
  (or_do_mm) the mismatch rate is reported and held under 2e-2 of the
  reference spikes (the bf16-path bar);
* readout: member fitness from the GPU's own rates within rel 2e-2 of the fp32
  oracle, and the whole member forward (or_snn_forward_member) within rel 5e-2;
* ES update: every layer's gradient at N = 8192 (the hidden layers' from the
  factor record the forward's draws wrote, the readout's generated) against the
  oracle's double-accumulated gradient, rel 1e-5.
"""
import numpy as np
import pytest
import torch

from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAMW, MATH_BF16
from tests import oracle_lib as O
from tests.test_gpu_linear import bf16_round
from tests.test_gpu_snn import unpack

pytestmark = pytest.mark.gpu

C3 = dict(dims=(784, 128, 128, 128, 10), T=16, rows=64, n=8192, rank=128, sigma=0.02,
          tau_m=10.0, v_th=1.0, math=MATH_BF16, solver=ADAMW, lr=0.01, poisson_seed=(5, 6, 7, 8))
MEMBERS = (0, 1, 510, 511, 512, 513, 2047, 4094, 4095, 8190, 8191)
POOL = 60000


def member_currents(x, W, A, B, bf16, mw=False):
    """Currents (T, R, a) of one member from its input spikes x (T, R, b), float64.
    bf16: the factored kernel's arithmetic (bf16 W, A, B and a bf16 rounding of
    x B), or with mw the member-weight kernel's (bf16 of W + A B^T)."""
    T, R, b = x.shape
    xs = x.reshape(-1, b).astype(np.float64)
    if not bf16:
        return O.do_mm(x.reshape(-1, b), W, A, B).reshape(T, R, -1).astype(np.float64)
    if mw:
        wm = (W.astype(np.float64) + A.astype(np.float64) @ B.astype(np.float64).T).astype(np.float32)
        return (xs @ bf16_round(wm).astype(np.float64).T).reshape(T, R, -1)
    xb = (xs @ bf16_round(B).astype(np.float64)).astype(np.float32)
    y = xs @ bf16_round(W).astype(np.float64).T
    y += bf16_round(xb).astype(np.float64) @ bf16_round(A).astype(np.float64).T
    return y.reshape(T, R, -1)


def oracle_cfg(cfg):
    dims = np.array(cfg.dims, np.int32)
    c = O.SnnCfg()
    c.n_layers = len(cfg.dims) - 1
    c.dims = dims.ctypes.data_as(O.ctypes.POINTER(O.c_i32))
    c.T, c.rows, c.tau_m, c.v_th, c.sigma = cfg.T, cfg.rows, cfg.tau_m, cfg.v_th, cfg.sigma
    c.rank, c.noise_reuse, c.epoch = cfg.rank, cfg.noise_reuse, 0
    for i in range(4):
        c.poisson_seed[i] = cfg.poisson_seed[i]
    return c, dims


@pytest.fixture(scope="module")
def c3_run(hses_gpu):
    cfg = snn.SnnConfig(**C3)
    pool, labels = snn.synthetic_pool(POOL, cfg.dims[0], cfg.dims[-1], 0)
    idx = snn.sample_index(0, cfg.n, cfg.rows, POOL)
    W = snn.init_weights(cfg.dims, 0, gain=snn.ACTIVE_GAIN)
    es = snn.SnnEs(cfg, W, pool, labels, idx)
    assert es.fused, "the full-size C3 step runs the fused forward + LIF kernel"
    assert es.record and es.ahead, "the full-size C3 step draws factors ahead into the record"
    assert es.mw, "the full-size C3 step runs on member weights"
    assert es.ppool is not None, "the full-size C3 step encodes from the prepared pool"
    fit = es.forward(0)
    torch.cuda.synchronize()
    R = cfg.rows
    rows = np.concatenate([np.arange(m * R, (m + 1) * R) for m in MEMBERS])
    rows_t = torch.as_tensor(rows, device="cuda")
    spk = [unpack(es.spikes_tm(l).index_select(1, rows_t), cfg.dims[l]) for l in range(es.L - 1)]
    rate = es.rate.index_select(0, rows_t).cpu().numpy()
    fit_gpu = fit.cpu().numpy().copy()
    es.update(fit, 0)
    torch.cuda.synchronize()
    grads = [g.cpu().numpy() for g in es.grads]
    return dict(cfg=cfg, pool=pool, labels=labels, idx=idx, W=W, spk=spk, rate=rate,
                fit=fit_gpu, grads=grads, mw=es.mw)


def test_c3_full_input_spikes_bit_exact(c3_run):
    cfg, R = c3_run["cfg"], c3_run["cfg"].rows
    mix = 0
    for s in cfg.poisson_seed:
        mix ^= s
    for j, m in enumerate(MEMBERS):
        p = c3_run["pool"][c3_run["idx"][m * R:(m + 1) * R]]
        seed = (mix + 1000000007 * m * R * cfg.dims[0]) & 0xFFFFFFFF
        ref = O.poisson(p, cfg.T, (seed, 0, 0, 0))
        np.testing.assert_array_equal(c3_run["spk"][0][:, j * R:(j + 1) * R], ref,
                                      err_msg=f"member {m}")


def test_c3_full_hidden_layers_and_readout(c3_run):
    cfg, W, R = c3_run["cfg"], c3_run["W"], c3_run["cfg"].rows
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    L = len(cfg.dims) - 1
    stats = {}
    for l in range(L - 1):
        a, b = cfg.dims[l + 1], cfg.dims[l]
        A, B = O.lora_factors(bs, cfg.keys[l], cfg.rank, 0, np.array(MEMBERS), a, b)
        n_ref = mism_bf = mism_32 = 0
        for j, m in enumerate(MEMBERS):
            x = c3_run["spk"][l][:, j * R:(j + 1) * R]
            cur_bf = member_currents(x, W[l], A[j], B[j], True, mw=c3_run["mw"])
            cur_32 = member_currents(x, W[l], A[j], B[j], False)
            err = np.abs(cur_bf - cur_32).max()
            assert err <= 2e-2 * np.abs(cur_32).max(), f"layer {l} member {m}: currents"
            ref_bf, _ = O.lif(cur_bf.astype(np.float32), cfg.tau_m, cfg.v_th)
            ref_32, _ = O.lif(cur_32.astype(np.float32), cfg.tau_m, cfg.v_th)
            if l < L - 2:
                got = c3_run["spk"][l + 1][:, j * R:(j + 1) * R]
                mism_bf += int((got != ref_bf).sum())
                mism_32 += int((got != ref_32).sum())
            else:
                # the last hidden layer only leaves its spike rates; each flip
                # moves a rate by 1/T, so T * |rate difference| counts flips
                # that do not cancel within a (row, column) series
                got = c3_run["rate"][j * R:(j + 1) * R]
                mism_bf += int(np.rint(cfg.T * np.abs(got - ref_bf.mean(0))).sum())
                mism_32 += int(np.rint(cfg.T * np.abs(got - ref_32.mean(0))).sum())
            n_ref += int(ref_32.sum())
        stats[l] = (mism_bf, mism_32, n_ref)
        print(f"layer {l}: {n_ref} reference spikes, mismatches bf16-arith {mism_bf}, "
              f"fp32 {mism_32} ({mism_32 / max(n_ref, 1):.2e})")
        assert n_ref > 0.03 * cfg.T * R * len(MEMBERS) * a, f"layer {l} is nearly silent"
        assert mism_bf <= 1e-4 * n_ref, f"layer {l}: {mism_bf} of {n_ref} vs bf16 arithmetic"
        assert mism_32 <= 2e-2 * n_ref, f"layer {l}: {mism_32} of {n_ref} vs fp32"
    # readout on the GPU's own rates: logits in fp32 by the oracle, fitness per member
    a, b = cfg.dims[-1], cfg.dims[-2]
    A, B = O.lora_factors(bs, cfg.keys[-1], cfg.rank, 0, np.array(MEMBERS), a, b)
    for j, m in enumerate(MEMBERS):
        rate = np.ascontiguousarray(c3_run["rate"][j * R:(j + 1) * R])
        logits = O.do_mm(rate, W[-1], A[j], B[j])
        lab = c3_run["labels"][c3_run["idx"][m * R:(m + 1) * R]]
        ref = float(O.loglik(logits, lab).astype(np.float64).mean())
        got = float(c3_run["fit"][m])
        assert abs(got - ref) <= 2e-2 * abs(ref), f"member {m}: fitness {got} vs {ref}"


def test_c3_full_member_forward_end_to_end(c3_run):
    # the whole member forward in the oracle (fp32 everywhere, its own spikes)
    cfg, R = c3_run["cfg"], c3_run["cfg"].rows
    c, _dims = oracle_cfg(cfg)
    Ws = [np.ascontiguousarray(w) for w in c3_run["W"]]
    Wp = (O.ctypes.c_void_p * len(Ws))(*[w.ctypes.data for w in Ws])
    keys = (O.c_u64 * len(cfg.keys))(*cfg.keys)
    worst = 0.0
    for m in MEMBERS:
        rows = c3_run["idx"][m * R:(m + 1) * R]
        probs = np.ascontiguousarray(c3_run["pool"][rows], np.float32)
        lab = np.ascontiguousarray(c3_run["labels"][rows], np.int32)
        out = np.zeros(1, np.float32)
        O.load().or_snn_forward_member(O.ctypes.byref(c), Wp, keys, probs, lab, m, out)
        rel = abs(float(c3_run["fit"][m]) - float(out[0])) / abs(float(out[0]))
        worst = max(worst, rel)
        assert rel <= 5e-2, f"member {m}: {c3_run['fit'][m]} vs oracle {out[0]}"
    print(f"end-to-end member fitness: worst rel difference {worst:.2e}")


@pytest.mark.parametrize("layer", [0, 1, 2, 3])
def test_c3_full_layer_gradient(c3_run, layer):
    # each layer's ES gradient over all 8192 members (fc1 from 4096 pairs in 512
    # split-K slices, the operand scale taken from max|f| over the whole
    # population) against the double-accumulated oracle on the same z-scored
    # fitness
    cfg = c3_run["cfg"]
    z, _, _ = O.convert_fitnesses(c3_run["fit"])
    a, b = cfg.dims[layer + 1], cfg.dims[layer]
    g = O.lora_grad_f64(cfg.sigma, cfg.keys[layer], cfg.rank, 0, z, a, b, nthreads=16)
    got = c3_run["grads"][layer]
    assert got.shape == g.shape
    err = np.abs(got - g).max()
    print(f"layer {layer}: gradient max err {err:.3e} of max {np.abs(g).max():.3e}")
    assert err <= 1e-5 * np.abs(g).max(), f"layer {layer} gradient err {err:.3e}"
