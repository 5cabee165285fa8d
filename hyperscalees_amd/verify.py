"""The K-chunk equivalence check of the reference's ES driver (`--verify`,
accumulate_train.rs:381-559), on the GPU path.

Four ways to take one ES step over the same members, from the same parameters:
  A  one batch: forward of all members, global z-score, do_updates;
  B  the forward in K chunks with frozen parameters, the raw fitness
     concatenated, then one global z-score and do_updates;
  D  the driver's path: K chunks, each chunk's ES gradient accumulated on its
     raw fitness, the global z-score applied afterwards by combine_affine_grads
     (accumulated_update, eggroll.rs:550-702);
  C  the negative control: per chunk a forward with the parameters left by the
     previous chunk, a z-score over that chunk alone and its own do_updates.
B and D must equal A (max |delta param| < 1e-3, accumulate_train.rs:537-548);
C must not (> 1e-3, accumulate_train.rs:549-552): the chunk-local z-score
breaks the linearity the accumulation relies on.

    python -m hyperscalees_amd.verify [--n 256] [--chunks 4]
"""
import argparse
import math
import sys

import numpy as np
import torch

from . import kernels as K
from . import snn
from ._lib import ADAMW

THRESHOLD = 1e-3  # accumulate_train.rs:537-552


def _fresh(cfg_kwargs, pool, labels, idx, W, **over):
    cfg = snn.SnnConfig(**dict(cfg_kwargs, **over))
    return snn.SnnEs(cfg, W, pool, labels, idx)


def _max_delta(Pa, Pb):
    return max(float((a - b).abs().max()) for a, b in zip(Pa, Pb))


def verify_paths(cfg_kwargs, chunks, pool, labels, idx, W, epoch=0):
    """Returns {"d_ab", "d_ad", "d_ac", "pass"} for one step of the four paths."""
    n = cfg_kwargs["n"]
    if n % chunks:
        raise ValueError("n must be a multiple of the chunk count")
    # A: one batch
    a = _fresh(cfg_kwargs, pool, labels, idx, W)
    a.step(epoch)
    # B: chunked forward with frozen parameters, one global z-score and update
    b = _fresh(cfg_kwargs, pool, labels, idx, W, accumulate=chunks)
    for k in range(chunks):
        b.forward(epoch, k * b.cfg.chunk)
    b.update(b.raw, epoch)
    # D: the driver's chunked accumulation with the affine z-score
    d = _fresh(cfg_kwargs, pool, labels, idx, W, accumulate=chunks)
    d.step(epoch)
    # C: chunk-local z-score and an update per chunk (parameters move between chunks)
    c = _fresh(cfg_kwargs, pool, labels, idx, W, accumulate=chunks)
    cc = c.cfg
    m = cc.chunk
    scale = np.float32(-math.sqrt(m) / m)
    for k in range(chunks):
        lo = k * m
        raw = c.forward(epoch, lo)
        z, _ = K.convert_fitnesses(raw)
        c.step_t += 1
        for l in range(c.L):
            rows, cols = c.W[l].shape
            K.es_update(z, lo, cc.keys[l], cc.rank, cc.sigma, epoch, cc.noise_reuse, rows, cols,
                        scale, out=c.grads[l])
            K.solver_step(cc.solver, cc.lr, c.W[l], c.grads[l], c.m[l], c.v[l], step_t=c.step_t,
                          beta1=cc.beta1, beta2=cc.beta2, eps=cc.eps,
                          wd=cc.weight_decay if cc.solver == ADAMW else 0.0)
    torch.cuda.synchronize()
    out = {"d_ab": _max_delta(a.W, b.W), "d_ad": _max_delta(a.W, d.W),
           "d_ac": _max_delta(a.W, c.W)}
    out["pass"] = out["d_ab"] < THRESHOLD and out["d_ad"] < THRESHOLD and out["d_ac"] > THRESHOLD
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--n", type=int, default=256)
    ap.add_argument("--chunks", type=int, default=4)
    ap.add_argument("--rank", type=int, default=4)
    ap.add_argument("--lr", type=float, default=0.05)
    args = ap.parse_args(argv)
    from ._lib import MATH_F32, SGD
    cfg = dict(dims=(784, 128, 128, 128, 10), T=8, rows=16, n=args.n, rank=args.rank, sigma=0.02,
               tau_m=10.0, v_th=1.0, math=MATH_F32, solver=SGD, lr=args.lr,
               poisson_seed=(1, 2, 3, 4))
    pool, labels = snn.synthetic_pool(3000, 784, 10, 0)
    idx = snn.sample_index(0, args.n, cfg["rows"], 3000)
    W = snn.init_weights(cfg["dims"], 0, gain=snn.ACTIVE_GAIN)
    K.init(0)
    r = verify_paths(cfg, args.chunks, pool, labels, idx, W)
    print(f"[verify] n={args.n} K={args.chunks}: chunked vs one batch {r['d_ab']:.3e}, "
          f"accumulated vs one batch {r['d_ad']:.3e}, chunk-local z-score vs one batch "
          f"{r['d_ac']:.3e} -> {'PASS' if r['pass'] else 'FAIL'}")
    return 0 if r["pass"] else 1


if __name__ == "__main__":
    sys.exit(main())
