"""Standalone timing of the HBM-streaming kernels at the C3 shapes.

  * LIF scan (hses_lif_scan): currents (T=16, M=524288, h=128) fp32 ->
    bit-packed spikes, and -> fp32 spikes;
  * Poisson encode (hses_poisson_encode): p (M=524288, 784) fp32 with 70% exact
    zeros -> bit-packed spikes (T=16), and -> fp32 spikes for T=4;
  * the C3 step's encode (hses_poisson_encode_pool): the batch of 8192 members x
    64 rows gathered from a prepared 60000 x 784 pool -> bit-packed spikes (T=16,
    each row's 16 words adjacent);
  * torch's device copy of the LIF input (a reference point for the bandwidth
    a plain read + write stream reaches);
  * the exact normal generator (hses_lora_factors) over every pair's factors
    of C3 fc1 (4096 pairs x (128 + 784) stream rows x 128 ranks = 478 M
    normals): normals per second, the bound of the factor-drawing kernels.
Each case runs --reps times after a warm-up, timed with events on the launch
stream; the median is reported with the algorithmic bytes (inputs read once,
outputs written once) and the fraction of the 8 TB/s HBM peak, one JSON line
per case.  Also a profiling target:
    rocprofv3 --kernel-trace --stats -d OUT -- python3 -m hyperscalees_amd.profile_kernels
"""
import argparse
import json

import torch

from . import kernels as K

PEAK_HBM_GBPS = 8000.0


def timed(fn, reps):
    fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    ts.sort()
    return ts[len(ts) // 2]


def report(name, ms, nbytes, **extra):
    gbps = nbytes / (ms * 1e-3) / 1e9
    line = {"kernel": name, "ms": round(ms, 4), "algorithmic_bytes": int(nbytes),
            "GBps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_HBM_GBPS, 4)}
    line.update(extra)
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    K.init(0)
    g = torch.Generator(device="cuda").manual_seed(0)
    T, M, h, d = 16, 8192 * 64, 128, 784

    cur = torch.randn((T, M, h), device="cuda", generator=g) * 0.6 + 0.35
    # reference point: torch's device copy of the same 4.3 GB (read + write)
    cpy = torch.empty_like(cur)
    ms = timed(lambda: cpy.copy_(cur), args.reps)
    report("device copy (torch)", ms, 2 * cur.numel() * 4, shape=[T, M, h])
    del cpy
    ms = timed(lambda: cur.sum(), args.reps)
    report("device read (torch sum)", ms, cur.numel() * 4, shape=[T, M, h])
    for fmt, name, out_b in ((K.FMT_BITS, "lif_scan f32 -> bits", T * M * 2 * 8),
                             (K.FMT_F32, "lif_scan f32 -> f32", T * M * h * 4)):
        spk = torch.empty((T, M, K.fmt_width(fmt, h)), dtype=K._FMT_DTYPE[fmt], device="cuda")
        ms = timed(lambda: K.lif_scan(cur, 10.0, 1.0, fmt=fmt, out=spk), args.reps)
        report(name, ms, T * M * h * 4 + out_b, shape=[T, M, h])
    del cur, spk

    p = torch.rand((M, d), device="cuda", generator=g)
    p[torch.rand((M, d), device="cuda", generator=g) < 0.7] = 0.0
    bits = torch.empty((T, M, K.fmt_width(K.FMT_BITS, d)), dtype=torch.int64, device="cuda")
    ms = timed(lambda: K.poisson_encode(p, T, (1, 2, 3, 4), K.FMT_BITS, out=bits), args.reps)
    report("poisson_encode -> bits", ms, M * d * 4 + T * M * bits.shape[2] * 8, shape=[T, M, d],
           zero_frac=0.7)
    T4 = 4
    f32 = torch.empty((T4, M, d), dtype=torch.float32, device="cuda")
    ms = timed(lambda: K.poisson_encode(p, T4, (1, 2, 3, 4), K.FMT_F32, out=f32), args.reps)
    report("poisson_encode -> f32", ms, M * d * 4 + T4 * M * d * 4, shape=[T4, M, d],
           zero_frac=0.7)
    del p, bits, f32

    import numpy as np
    from . import snn
    pool, _ = snn.synthetic_pool(60000, d, 10, seed=0)
    idx = snn.sample_index(0, 8192, 64, 60000)
    pp = K.PoissonPool(torch.from_numpy(pool).cuda())
    it = torch.as_tensor(idx, dtype=torch.int32).cuda()
    words = K.fmt_width(K.FMT_BITS, d)
    ti = torch.empty((M, T, words), dtype=torch.int64, device="cuda")
    ms = timed(lambda: K.poisson_encode_pool(pp, T, (1, 2, 3, 4), out=ti, rows_index=it,
                                             time_inner=True), args.reps)
    # bytes each gathered row reads: its counts, a u32 threshold and u16 column
    # per active element, a u16 column per saturated one; plus the row index
    act = ((pool > 0) & (pool < 1)).sum(axis=1)
    sat = (pool >= 1).sum(axis=1)
    per_row = 8 + 6 * act + 2 * sat
    report("poisson_encode_pool -> bits (prepared pool, gathered rows)", ms,
           int(per_row[idx].sum()) + 4 * M + T * M * words * 8, shape=[M, T, d],
           pool_rows=60000, active_per_row=round(float(act[idx].mean()), 1))
    del pp, ti

    pairs, a, b, r = 4096, 128, 784, 128
    ms = timed(lambda: K.lora_factors(0.01, 12345, r, 0, 0, (0, pairs), a, b), args.reps)
    normals = pairs * (a + b) * r
    report("lora_factors (exact normals)", ms, normals * 4, shape=[pairs, a + b, r],
           g_normals_per_s=round(normals / (ms * 1e-3) / 1e9, 1))


if __name__ == "__main__":
    main()
