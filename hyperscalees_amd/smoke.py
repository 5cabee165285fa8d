"""One tiny EggRoll ES step of the SNN-MLP on cuda:0 through the product path
(bit-packed Poisson, factors drawn ahead, member weights, fp32-accurate
split-operand forward with the LIF fused, count-plane readout, ES update from
the factor record),
checked against the CPU oracle (the oracle is only the checker here; every
computation runs in libhses.so).  Raises AssertionError on a mismatch."""
import math

import numpy as np
import torch

from . import kernels as K
from . import snn
from ._lib import MATH_F32X, SGD


def run_smoke():
    from tests import oracle_lib as O   # checker only

    if not torch.cuda.is_available():
        raise RuntimeError("smoke() needs a GPU")
    K.init(0)
    cfg = snn.SnnConfig(dims=(784, 64, 64, 10), T=8, rows=32, n=16, rank=32, sigma=0.02,
                        math=MATH_F32X, solver=SGD, lr=0.05, poisson_seed=(3, 1, 4, 1))
    pool, labels = snn.synthetic_pool(500, cfg.dims[0], cfg.dims[-1], seed=1)
    idx = snn.sample_index(1, cfg.n, cfg.rows, 500)
    W = snn.init_weights(cfg.dims, 1, gain=snn.ACTIVE_GAIN)
    es = snn.SnnEs(cfg, W, pool, labels, idx)
    assert es.split and es.ahead and es.mw, "the smoke step runs the product path"

    # Poisson spikes: bit-exact
    es.poisson()
    torch.cuda.synchronize()
    words = es.spikes_tm(0).contiguous().cpu().numpy().view(np.uint64)
    bits = ((words[..., None] >> np.arange(64, dtype=np.uint64)) & np.uint64(1)).astype(np.float32)
    got = bits.reshape(cfg.T, cfg.n * cfg.rows, -1)[..., : cfg.dims[0]]
    ref = O.poisson(pool[idx], cfg.T, cfg.poisson_seed)
    assert np.array_equal(got, ref), "Poisson spikes differ from the oracle"

    # full step: fitness, then the ES gradient on the GPU's fitness
    fit = es.forward(0)
    torch.cuda.synchronize()
    fit_gpu = fit.cpu().numpy()
    assert np.all(np.isfinite(fit_gpu))
    # every member's whole forward against the oracle's fp32 one
    dims = np.array(cfg.dims, np.int32)
    c = O.SnnCfg()
    c.n_layers = len(cfg.dims) - 1
    c.dims = dims.ctypes.data_as(O.ctypes.POINTER(O.c_i32))
    c.T, c.rows, c.tau_m, c.v_th, c.sigma = cfg.T, cfg.rows, cfg.tau_m, cfg.v_th, cfg.sigma
    c.rank, c.noise_reuse, c.epoch = cfg.rank, cfg.noise_reuse, 0
    for i in range(4):
        c.poisson_seed[i] = cfg.poisson_seed[i]
    Ws = [np.ascontiguousarray(w) for w in W]
    Wp = (O.ctypes.c_void_p * len(Ws))(*[w.ctypes.data for w in Ws])
    keys = (O.c_u64 * len(cfg.keys))(*cfg.keys)
    for m in range(cfg.n):
        rows = idx[m * cfg.rows:(m + 1) * cfg.rows]
        probs = np.ascontiguousarray(pool[rows], np.float32)
        lab = np.ascontiguousarray(labels[rows], np.int32)
        out = np.zeros(1, np.float32)
        O.load().or_snn_forward_member(O.ctypes.byref(c), Wp, keys, probs, lab, m, out)
        rel = abs(float(fit_gpu[m]) - float(out[0])) / abs(float(out[0]))
        assert rel <= 1e-4, f"member {m}: fitness {fit_gpu[m]} vs oracle {out[0]}"
    es.update(fit, 0)
    torch.cuda.synchronize()
    z, _, _ = O.convert_fitnesses(fit_gpu)
    for l in range(es.L):
        a, b = W[l].shape
        g_ref = O.lora_grad_f64(cfg.sigma, cfg.keys[l], cfg.rank, 0, z, a, b, nthreads=4)
        g = es.grads[l].cpu().numpy()
        err = float(np.abs(g - g_ref).max())
        assert err <= 1e-5 * float(np.abs(g_ref).max()), f"layer {l} ES gradient err {err}"
    print(f"smoke ok: N={cfg.n} r={cfg.rank} fitness mean {fit_gpu.mean():.4f}, member "
          f"forwards within 1e-4 and gradients within 1e-5 of the oracle", flush=True)
