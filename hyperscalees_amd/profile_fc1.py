"""Profiling target for the dominant kernel of the C3 ES step.

Runs, on cuda:0 with synthetic data of the C3 shape (bench.py's workload):
  * a device-to-device copy of a known size (1 GiB), the calibration point for
    the FETCH_SIZE / WRITE_SIZE hardware counters;
  * the fc1 layer of the SNN step as the step runs it: the factor draw into
    the record (hses_pair_factors, once), every member's weights from it
    (hses_member_weights, once) and then the GEMM on them
    (hses_perturbed_linear_lif_mw: x W_m^T on split fp16 operands, fused with
    the LIF scan), N = 8192 members, r = 128, T = 16, 64 rows per member,
    b = 784, a = 128; with --math bf16 the bf16 forms; with --factored the
    factored forward on a drawn operand image instead
    (hses_perturbed_linear_lif_pre[_x]: x[W^T|B] + (xB)A^T).
The copy and the GEMM are launched --reps times.  Use under rocprofv3, e.g.
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -- python3 -m hyperscalees_amd.profile_fc1
"""
import argparse

import torch

from . import kernels as K
from . import snn


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--math", choices=("f32x", "bf16"), default="f32x")
    ap.add_argument("--factored", action="store_true")
    args = ap.parse_args()
    split = args.math == "f32x"
    math = K.MATH_F32X if split else K.MATH_BF16
    K.init(0)
    cfg = snn.SnnConfig(poisson_seed=(1, 2, 3, 4))
    M = cfg.n * cfg.rows
    g = torch.Generator(device="cuda").manual_seed(0)
    words_in = K.fmt_width(K.FMT_BITS, cfg.dims[0])
    # spikes in the step's time-inner layout, (M, T, words)
    x = torch.randint(0, 2**62, (M, cfg.T, words_in), dtype=torch.int64, device="cuda", generator=g)
    W = torch.randn(cfg.dims[1], cfg.dims[0], device="cuda", generator=g) * 0.05
    spk = torch.empty((M, cfg.T, K.fmt_width(K.FMT_BITS, cfg.dims[1])), dtype=torch.int64,
                      device="cuda")
    a, b = cfg.dims[1], cfg.dims[0]
    rec = K.factor_record(a, b, cfg.rank, 0, cfg.n)
    if args.factored:
        img = (K.pair_image_x if split else K.pair_image)(a, b, cfg.rank, 0, cfg.n)
        K.pair_factors(cfg.keys[0], cfg.rank, cfg.sigma, 0, cfg.noise_reuse, 0, cfg.n, a, b, rec,
                       img, split=split)
    else:
        K.pair_factors(cfg.keys[0], cfg.rank, cfg.sigma, 0, cfg.noise_reuse, 0, cfg.n, a, b, rec,
                       None)
        wm = K.member_weights(W, cfg.rank, cfg.sigma, 0, cfg.n, rec, math=math)
    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda")  # 1 GiB
    dst = torch.empty_like(src)
    src.fill_(1.0)
    torch.cuda.synchronize()
    for _ in range(args.reps):
        dst.copy_(src)
    for s in range(args.reps):
        if args.factored:
            K.perturbed_linear_lif(x, W, cfg.keys[0], cfg.rank, cfg.sigma, 0, cfg.noise_reuse, 0,
                                   cfg.n, cfg.rows, cfg.T, cfg.tau_m, cfg.v_th, spikes=spk,
                                   rec=rec, img=img, time_inner=True, math=math)
        else:
            K.perturbed_linear_lif_mw(x, wm, a, b, 0, cfg.n, cfg.rows, cfg.T, cfg.tau_m, cfg.v_th,
                                      math=math, spikes=spk, time_inner=True)
    torch.cuda.synchronize()
    print("profile_fc1: copy 1 GiB x", args.reps, "; fc1 draw x 1;",
          "" if args.factored else "member weights x 1;", "fc1 GEMM x", args.reps,
          "(" + args.math + (", factored" if args.factored else ", member weights") + ")",
          flush=True)


if __name__ == "__main__":
    main()
