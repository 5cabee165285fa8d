"""Benchmark of the EggRoll SNN-MLP hot path on one MI355X.

Metric: perturbed member-evals/sec + ES-update GB/s, SNN-MLP
N=8192 r=128.  One step = one full ES step of the population:
Poisson encode -> 3 perturbed hidden layers with LIF -> rate readout ->
log-likelihood fitness -> z-score -> ES gradient of the 4 layers -> AdamW.
`value` = N / (time per step): member evaluations per second including the
update.  Inputs are synthetic and resident in HBM before timing starts.

With --workload c5 it measures the RWKV-7 LM configuration instead:
one step = one ES step of N=2048 members at r=1, each scoring the next-token
log-likelihood of its own 128-token sequence (bf16 MFMA linears), then the
z-score and the ES update of every matrix.

Prints one JSON line.  --gpus N > 1 is refused: this build runs on one GPU.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "perturbed member-evals/sec + ES-update GB/s, SNN-MLP N=8192 r=128"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3      # MI355X dense fp32 MFMA
PEAK_HBM_GBPS = 8000.0
# HBM bytes per launch of fc1's GEMM on member weights (k_mw_bits), from two rocprofv3 PMC runs
# of `python3 -m hyperscalees_amd.profile_fc1` (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, factors
# from a 1 GiB copy in the same process; profiles/fc1_c3_traffic.md), keyed by (math, member
# weights).  Measured on the k_mw_bits source of commit 821b0d8; refreshed whenever the kernel
# changes, and the bench line names the source it was measured on.
FC1_TRAFFIC = {
    ("f32x", True): (4.534e9, "rocprofv3 PMC of profile_fc1, k_mw_bits of commit 9357756: "
                              "4.400e9 B read + 0.134e9 B written"),
    ("bf16", True): (2.771e9, "rocprofv3 PMC of profile_fc1 --math bf16, k_mw_bits of commit "
                              "9357756: 2.636e9 B read + 0.134e9 B written"),
}


def layer_flops(cfg, l):
    """Algorithmic forward FLOPs of layer l: 2Mba + 2Mbr + 2Mra."""
    b, a = cfg.dims[l], cfg.dims[l + 1]
    M = cfg.n * cfg.rows * (cfg.T if l < len(cfg.dims) - 2 else 1)
    return 2 * M * b * a + 2 * M * b * cfg.rank + 2 * M * cfg.rank * a


def update_bytes(cfg):
    """ES-update bytes, materialized-factor convention: sum_l N r (a+b) 4 + 2 a b 4."""
    tot = 0
    for l in range(len(cfg.dims) - 1):
        b, a = cfg.dims[l], cfg.dims[l + 1]
        tot += cfg.n * cfg.rank * (a + b) * 4 + 2 * a * b * 4
    return tot


def host_cpu():
    """(threads this process may use, logical CPUs of the host, CPU model name).
    The thread count is the process's CPU affinity, capped by OMP_NUM_THREADS
    when set (the box's per-GPU CPU share)."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = nproc
    cap = os.environ.get("OMP_NUM_THREADS")
    threads = min(avail, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else avail
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return threads, nproc, model


def cpu_baseline(cfg, pool, labels, idx, W, members, threads, label="C3"):
    """The oracle (C restatement of the reference CPU path) on `members` members,
    forward + their share of the ES update, extrapolated linearly in N when
    members < N."""
    from tests import oracle_lib as O
    L = O.load()
    dims = np.array(cfg.dims, np.int32)
    c = O.SnnCfg()
    c.n_layers = len(cfg.dims) - 1
    c.dims = dims.ctypes.data_as(O.ctypes.POINTER(O.c_i32))
    c.T, c.rows, c.tau_m, c.v_th, c.sigma = cfg.T, cfg.rows, cfg.tau_m, cfg.v_th, cfg.sigma
    c.rank, c.noise_reuse, c.epoch = cfg.rank, cfg.noise_reuse, 0
    for i in range(4):
        c.poisson_seed[i] = cfg.poisson_seed[i]
    R = members * cfg.rows
    probs = np.ascontiguousarray(pool[idx[:R]], np.float32)
    lab = np.ascontiguousarray(labels[idx[:R]], np.int32)
    Ws = [np.ascontiguousarray(w) for w in W]
    Wp = (O.ctypes.c_void_p * len(Ws))(*[w.ctypes.data for w in Ws])
    keys = (O.c_u64 * len(cfg.keys))(*cfg.keys)
    fit = np.zeros(members, np.float32)
    t0 = time.perf_counter()
    L.or_snn_forward_members(O.ctypes.byref(c), Wp, keys, probs, lab, 0, members, threads, fit)
    t1 = time.perf_counter()
    z, _, _ = O.convert_fitnesses(fit)
    for l in range(len(cfg.dims) - 1):
        a, b = cfg.dims[l + 1], cfg.dims[l]
        O.lora_grad_f64(cfg.sigma, cfg.keys[l], cfg.rank, 0, z, a, b, nthreads=threads)
    t2 = time.perf_counter()
    per_member = (t2 - t0) / members
    _, nproc, model = host_cpu()
    scope = ("all N members (no extrapolation)" if members == cfg.n else
             f"{members} of {cfg.n} members, extrapolated linearly in N")
    return {"value": 1.0 / per_member, "unit": "member-evals/s", "cores": threads,
            "kind": "port", "host_nproc": nproc, "cpu_model": model,
            "sample": (f"{label} ES step (forward + ES update) of {scope}, oracle (C, -O3, OpenMP) on "
                       f"{threads} host threads; fwd {t1 - t0:.2f}s, update {t2 - t1:.2f}s"),
            "seconds": round(t2 - t0, 2)}


def bench_c5(args):
    """The C5 workload: RWKV-7 LM (4 layers, d=512, vocab 256), N=2048, r=1."""
    import torch
    from hyperscalees_amd import kernels as K
    from hyperscalees_amd import rwkv, rwkv_lm
    from hyperscalees_amd._lib import ACT_RELU_SQ

    n = args.population if args.population != 8192 else 2048
    cfg = rwkv_lm.RwkvLmConfig(n=n)
    params = rwkv_lm.init_params(cfg, seed=0)
    K.init(0)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    tok = torch.randint(0, cfg.vocab, (cfg.n, cfg.seq_len + 1), dtype=torch.int32, device="cuda",
                        generator=g)
    for i in range(args.warmup):
        es.step(tok, epoch=i)
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    marks = []
    t0 = time.perf_counter()
    for s_ in range(args.steps):
        e = [ev() for _ in range(3)]
        e[0].record()
        fit = es.forward(tok, epoch=s_)
        e[1].record()
        es.update(fit, s_)
        e[2].record()
        marks.append(e)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    t_fwd = float(np.mean([e[0].elapsed_time(e[1]) for e in marks]))
    t_upd = float(np.mean([e[1].elapsed_time(e[2]) for e in marks]))

    # Dominant single launch: ChannelMixing key of layer 0 (x (N*T, 512) -> relu^2 (N*T, 2048),
    # bf16 in and out as in the step), timed alone with events on the launch stream.
    B0 = es.blocks[0]
    C, F, T = cfg.d_model, cfg.ffn_mult * cfg.d_model, cfg.seq_len
    x = torch.randn((cfg.n, T, C), device="cuda", generator=g).to(torch.bfloat16)
    ek = es._es(0, 0, 0, cfg.n)["ffn_key"]
    lk = []
    for _ in range(3):
        e0, e1 = ev(), ev()
        e0.record()
        rwkv.linear(x, B0["ffn_key"], ek, cfg.math, act=ACT_RELU_SQ, out_bf16=True)
        e1.record()
        torch.cuda.synchronize()
        lk.append(e0.elapsed_time(e1))
    lk_ms = float(np.median(lk))
    rows = cfg.n * T
    lk_flops = 2 * rows * C * F + 2 * rows * cfg.rank * (C + F)
    achieved = lk_flops / (lk_ms * 1e-3) / 1e12
    out = {
        "metric": "perturbed member-evals/sec, RWKV-7 LM N=2048 r=1 (configs[4])",
        "value": round(cfg.n / (ms_per_step * 1e-3), 1),
        "unit": "member-evals/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 MFMA linears (fp32 accumulate), fp32 activations and recurrence",
        "data": "synthetic",
        "config": {"workload": ("C5: RWKV-7 LM, 4 layers, d=512, head 64, vocab 256, 128-token "
                                "uniform random sequences, N=2048 members x 1 sequence, r=1, "
                                "init N(0, 0.02), fitness = mean next-token log-likelihood, full "
                                "ES step (forward + fitness + z-score + ES update + SGD)"),
                   "population": cfg.n, "rank": cfg.rank, "seq_len": T,
                   "parallelism": "single GPU"},
        "phase_ms": {"forward": round(t_fwd, 3), "es_update": round(t_upd, 3)},
        "fwd_tflops": round(rwkv_lm.forward_flops(cfg) / (t_fwd * 1e-3) / 1e12, 1),
        "roofline": {"kernel": ("k_gemm_bf16<BF16 x, rank 1, relu^2, bf16 y> with its W->bf16 "
                                "conversion and factor draw (ChannelMixing key, 262144 x 512 -> "
                                "2048)"),
                     "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": None, "launch_ms": round(lk_ms, 3),
                     "algorithmic_flop_per_launch": lk_flops},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_c5(cfg, params, es, tok, args.cpu_members)
    print(json.dumps(out), flush=True)


def cpu_baseline_c5(cfg, params, es, tok, members):
    """The oracle's LM (a C restatement of the reference's forward) for a sample
    of members, each on its own materialised parameters W + A_m B_m^T, in
    parallel over the host threads (ctypes releases the GIL), plus the sample's
    share of the ES update (the oracle's double-accumulated gradient of every
    matrix over the sample's members)."""
    from concurrent.futures import ThreadPoolExecutor
    from tests import oracle_lib as O
    threads, nproc, model = host_cpu()
    ns = max(1, min(members, 4 * threads, cfg.n))
    tk = tok[:ns].cpu().numpy()
    H = cfg.d_model // cfg.head_size
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    names = list(es.keys)  # (layer, matrix) of every MM parameter

    def member(m):
        P = {k: v for k, v in params.items() if k != "blocks"}
        P["blocks"] = []
        for l, B in enumerate(params["blocks"]):
            Bm = dict(B)
            for name in (nm for (l2, nm) in names if l2 == l):
                a, b = B[name].shape
                A, Bf = O.lora_factors(bs, es.keys[(l, name)], cfg.rank, 0, [m], a, b)
                Bm[name] = B[name] + A[0] @ Bf[0].T
            P["blocks"].append(Bm)
        O.rwkv_lm_forward(P, tk[m, :-1], H)

    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(member, range(ns)))
    t1 = time.perf_counter()
    z = np.random.default_rng(0).standard_normal(ns).astype(np.float32)
    for (l, name) in names:
        a, b = params["blocks"][l][name].shape
        O.lora_grad_f64(cfg.sigma, es.keys[(l, name)], cfg.rank, 0, z, a, b, nthreads=threads)
    t2 = time.perf_counter()
    return {"value": round(ns / (t2 - t0), 4), "unit": "member-evals/s", "cores": threads,
            "kind": "port", "host_nproc": nproc, "cpu_model": model,
            "sample": (f"oracle LM forward of {ns} of {cfg.n} members ({cfg.seq_len}-token sequences, "
                       f"each on its materialised W + A_m B_m^T) in parallel on {threads} host "
                       f"threads, plus the ES update of every matrix over those members; fwd "
                       f"{t1 - t0:.2f}s, update {t2 - t1:.2f}s; extrapolated linearly in N"),
            "seconds": round(t2 - t0, 2)}


def _events(n):
    import torch
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _time_launch(fn, reps=5):
    """Mean duration (ms) of fn's launches: `reps` back-to-back calls between two
    HIP events on the launch stream, after one untimed call.  The host enqueues
    ahead of the GPU, so its per-call overhead does not show as GPU idle time."""
    import torch
    fn()
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _timed_steps(step, steps, warmup):
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s_ in range(steps):
        step(s_)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000.0 / steps


def bench_c4(args):
    """the spiking self-attention transformer (d_model 64, 4 heads, 2
    blocks, 64 tokens, LIF on Q/K/V) at N=1024, r=8, fp32.  One step = the
    population forward (Poisson-encoded tokens of a random 256-way vocabulary,
    one sequence per member), log-likelihood fitness, z-score, do_updates of
    every leaf and AdamW."""
    import torch
    from hyperscalees_amd import kernels as K
    from hyperscalees_amd import snn_attention as sa
    cfg = sa.SaConfig()
    K.init(0)
    P = sa.init_params(cfg, 0)
    vocab = sa.synthetic_vocab(cfg, 0)
    es = sa.SpikingAttentionEs(cfg, P, vocab)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    tok = torch.randint(0, cfg.vocab, (cfg.n, cfg.ntok), dtype=torch.int32, device="cuda", generator=g)
    lab = torch.randint(0, cfg.classes, (cfg.n,), dtype=torch.int32, device="cuda", generator=g)
    ms = _timed_steps(lambda i: es.step(tok, lab, epoch=i), args.steps, args.warmup)
    fwd_ms = _time_launch(lambda: es.forward(tok, lab, epoch=0), reps=3)
    # dominant kernel: the attention competition of one block (all members and heads)
    att_ms = _time_launch(lambda: es.attention_block(0, 0), reps=3)
    att = lambda: K._lib.call("hses_sa_attention", K._p(es.Q), K._p(es.Kt), K._p(es.V),
                              cfg.d_model, cfg.n, cfg.ntok, cfg.heads, cfg.head_dim,
                              K._p(es.th["beta"]), K._p(es.th["attn_th"]), cfg.g_inh, cfg.tau_m,
                              cfg.n_iter, K._p(es.O), K._stream())
    core_ms = _time_launch(att, reps=5)
    # algorithmic work of the competition: n_iter LIF steps over R x R key
    # neurons per (member, head) plus the scores and A V products (fp32 VALU)
    R, hd = cfg.ntok, cfg.head_dim
    core_flop = cfg.n * cfg.heads * (2 * R * R * hd * 2 + cfg.n_iter * R * R * 6)
    achieved = core_flop / (core_ms * 1e-3) / 1e12
    peak_vector_fp32 = 157.3  # MI355X fp32 vector (FMA) peak, TFLOP/s
    fl = sa.forward_flops(cfg)
    out = {
        "metric": "perturbed member-evals/sec, spiking self-attention N=1024 r=8 fp32 (configs[3])",
        "value": round(cfg.n / (ms * 1e-3), 1), "unit": "member-evals/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (fp32 MFMA projections, fp32 VALU spiking stages, fp32 ES update)",
        "data": "synthetic",
        "config": {"workload": ("C4: spiking self-attention transformer (snn_self_attention_heads), "
                                "d_model 64, 4 heads, 2 blocks, 64 tokens of a random 256-way "
                                "vocabulary (16-value intensity vectors, Poisson T=8), LIF on Q/K/V, "
                                "N=1024 members x 1 sequence, r=8, sigma 0.02; full ES step "
                                "(forward + fitness + z-score + ES update of every leaf + AdamW)"),
                   "population": cfg.n, "rank": cfg.rank, "tokens": cfg.ntok,
                   "parallelism": "single GPU"},
        "phase_ms": {"forward": round(fwd_ms, 4), "attention_block": round(att_ms, 4)},
        "fwd_flop": fl,
        "roofline": {"kernel": "k_sa_attention (row_softmax_lif over 1024 members x 4 heads x 64 rows)",
                     "bound": "valu", "achieved": round(achieved, 2), "peak": peak_vector_fp32,
                     "unit": "TFLOP/s", "frac": round(achieved / peak_vector_fp32, 4),
                     "traffic": None, "launch_ms": round(core_ms, 4),
                     "algorithmic_flop_per_launch": core_flop},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_c4(cfg, P, es, tr_spikes(es, tok, lab), args.cpu_members)
    print(json.dumps(out), flush=True)


def tr_spikes(es, tok, lab):
    """The population's input spikes (T, M, tin) on the host."""
    tr = {}
    es.forward(tok, lab, epoch=0, trace=tr)
    return tr["spk"].cpu().numpy()


def cpu_baseline_c4(cfg, P, es, spk, members):
    """The oracle's member forward (C restatement of the JAX model) on each
    sampled member's materialised parameters, in parallel over the host threads,
    plus the sample's share of the ES update of every leaf."""
    from concurrent.futures import ThreadPoolExecutor
    from tests import oracle_lib as O
    threads, nproc, model = host_cpu()
    ns = max(1, min(members, 8 * threads, cfg.n))
    R = cfg.ntok

    def member(m):
        Pm = O.sa_member_params(P, es.keys, es.leaves, cfg.sigma, cfg.rank, m)
        O.sa_forward_member(cfg, Pm, spk[:, m * R:(m + 1) * R])

    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(member, range(ns)))
    t1 = time.perf_counter()
    z = np.random.default_rng(0).standard_normal(ns).astype(np.float32)
    for name, (a, b), cls in es.leaves:
        if cls == 1:
            O.lora_grad_f64(cfg.sigma, es.keys[name], cfg.rank, 0, z, a, b, nthreads=threads)
    t2 = time.perf_counter()
    return {"value": round(ns / (t2 - t0), 3), "unit": "member-evals/s", "cores": threads,
            "kind": "port", "host_nproc": nproc, "cpu_model": model,
            "sample": (f"oracle forward of {ns} of {cfg.n} members (each on its materialised "
                       f"parameters) in parallel on {threads} host threads, plus the ES update of "
                       f"every MM leaf over those members; fwd {t1 - t0:.2f}s, update "
                       f"{t2 - t1:.2f}s; extrapolated linearly in N"),
            "seconds": round(t2 - t0, 2)}


def bench_c1(args):
    """SNN-MLP 784-128-128-128-10, T=8, N=256, r=4, sigma 0.02, fp32; every
    member evaluates the same 64 synthetic inputs.  One step = the full ES step."""
    import torch
    from hyperscalees_amd import kernels as K
    from hyperscalees_amd import snn
    from hyperscalees_amd._lib import MATH_F32, SGD
    cfg = snn.SnnConfig(T=8, rows=64, n=256, rank=4, sigma=0.02, math=MATH_F32, solver=SGD,
                        lr=0.05, poisson_seed=(1, 2, 3, 4))
    pool, labels = snn.synthetic_pool(64, cfg.dims[0], cfg.dims[-1], seed=0)
    idx = np.tile(np.arange(64, dtype=np.int32), cfg.n)  # the same 64 inputs for every member
    W = snn.init_weights(cfg.dims, 0, gain=snn.ACTIVE_GAIN)
    K.init(0)
    es = snn.SnnEs(cfg, W, pool, labels, idx)
    ms = _timed_steps(lambda i: es.step(epoch=i), args.steps, args.warmup)
    # dominant kernel: fc1's perturbed forward (k_factors + k_gemm_f32, fp32 MFMA)
    fc1 = lambda: K.perturbed_linear(es.spk[0], es.W[0], cfg.keys[0], cfg.rank, cfg.sigma, 0,
                                     cfg.noise_reuse, 0, cfg.n, cfg.rows, x_fmt=K.FMT_BITS,
                                     n_time=cfg.T, math=cfg.math, out=es.cur)
    fc1_ms = _time_launch(fc1)
    fl = layer_flops(cfg, 0)
    achieved = fl / (fc1_ms * 1e-3) / 1e12
    out = {
        "metric": "perturbed member-evals/sec, SNN-MLP N=256 r=4 T=8 fp32 (configs[0])",
        "value": round(cfg.n / (ms * 1e-3), 1), "unit": "member-evals/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (fp32 MFMA forward and ES update)", "data": "synthetic",
        "config": {"workload": ("C1: SNN-MLP 784-128-128-128-10, LIF decay 0.9 v_th 1.0, Poisson "
                                "T=8, N=256, r=4, sigma 0.02, the same 64 inputs (70% zeros) for "
                                "every member, full ES step (forward + fitness + z-score + ES "
                                "update + SGD)"),
                   "population": cfg.n, "rank": cfg.rank, "T": cfg.T, "parallelism": "single GPU"},
        "fwd_flop_per_step": sum(layer_flops(cfg, l) for l in range(len(cfg.dims) - 1)),
        "roofline": {"kernel": ("k_factors + k_gemm_f32<BITS x, 128 columns, rank 4> (fc1, 8 x 16384 "
                                "rows, 784 -> 128)"),
                     "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
                     "traffic": None, "launch_ms": round(fc1_ms, 4),
                     "algorithmic_flop_per_launch": fl},
    }
    if not args.no_cpu_baseline:
        threads, _, _ = host_cpu()
        out["cpu_baseline"] = cpu_baseline(cfg, pool, labels, idx, W, cfg.n, threads, label="C1")
    print(json.dumps(out), flush=True)


def bench_c2(args):
    """one EggRoll layer W 1024x1024 fp32, N=4096, r=1, 16 rows per member,
    x ~ N(0,1); one step = the perturbed forward, then the ES update on z-scored
    N(0,1) fitness (noise from seed 0: the layer key of layer 0)."""
    import torch
    from hyperscalees_amd import kernels as K
    from hyperscalees_amd._lib import MATH_F32
    n, rpm, a, b, r, sigma = 4096, 16, 1024, 1024, 1, 0.02
    key = 0x9E3779B97F4A7C15
    K.init(0)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    W = (torch.randn((a, b), device="cuda", generator=g) / 32.0).contiguous()
    x = torch.randn((n * rpm, b), device="cuda", generator=g)
    fit = torch.randn(n, device="cuda", generator=g)
    y = torch.empty((n * rpm, a), device="cuda")
    grad = torch.empty((a, b), device="cuda")
    scale = np.float32(-math.sqrt(n) / n)

    def step(i):
        K.perturbed_linear(x, W, key, r, sigma, i, 0, 0, n, rpm, math=MATH_F32, out=y)
        z, _ = K.convert_fitnesses(fit)
        K.es_update(z, 0, key, r, sigma, i, 0, a, b, scale, out=grad)

    ms = _timed_steps(step, args.steps, args.warmup)
    fwd_ms = _time_launch(lambda: K.perturbed_linear(x, W, key, r, sigma, 0, 0, 0, n, rpm,
                                                     math=MATH_F32, out=y))
    z, _ = K.convert_fitnesses(fit)
    upd_ms = _time_launch(lambda: K.es_update(z, 0, key, r, sigma, 0, 0, a, b, scale, out=grad))
    M = n * rpm
    fwd_fl = 2 * M * b * a + 2 * M * b * r + 2 * M * r * a
    upd_fl = 2 * a * b * n * r
    achieved = fwd_fl / (fwd_ms * 1e-3) / 1e12
    out = {
        "metric": "perturbed member-evals/sec, EggRoll layer 1024x1024 N=4096 r=1 fp32 (configs[1])",
        "value": round(n / (ms * 1e-3), 1), "unit": "member-evals/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (fp32 MFMA forward and ES update)", "data": "synthetic",
        "config": {"workload": ("C2: W 1024x1024 ~ N(0, 1/32^2), N=4096, r=1, 16 rows per member, "
                                "x ~ N(0,1); perturbed forward + z-score of N(0,1) fitness + ES "
                                "update"),
                   "population": n, "rank": r, "parallelism": "single GPU"},
        "phase_ms": {"forward": round(fwd_ms, 4), "es_update": round(upd_ms, 4)},
        "es_update_tflops": round(upd_fl / (upd_ms * 1e-3) / 1e12, 2),
        "roofline": {"kernel": ("k_factors + k_gemm_f32<F32 x, 128 columns, rank 1> (65536 x 1024 "
                                "-> 1024)"),
                     "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
                     "traffic": None, "launch_ms": round(fwd_ms, 4),
                     "algorithmic_flop_per_launch": fwd_fl},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_c2(W.cpu().numpy(), x.cpu().numpy(),
                                              z.cpu().numpy(), n, rpm, r, sigma, key)
    print(json.dumps(out), flush=True)


def cpu_baseline_c2(W, x, z, n, rpm, r, sigma, key):
    """The oracle's do_mm for every member (its factors from the noiser stream),
    in parallel over the host threads, then the double-accumulated ES update."""
    from concurrent.futures import ThreadPoolExecutor
    from tests import oracle_lib as O
    threads, nproc, model = host_cpu()
    a, b = W.shape
    bs = O.load().or_base_sigma(sigma, r)

    def member(m):
        A, B = O.lora_factors(bs, key, r, 0, [m], a, b)
        O.do_mm(np.ascontiguousarray(x[m * rpm:(m + 1) * rpm]), W, A[0], B[0])

    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(member, range(n)))
    t1 = time.perf_counter()
    O.lora_grad_f64(sigma, key, r, 0, z, a, b, nthreads=threads)
    t2 = time.perf_counter()
    return {"value": round(n / (t2 - t0), 2), "unit": "member-evals/s", "cores": threads,
            "kind": "port", "host_nproc": nproc, "cpu_model": model,
            "sample": (f"C2 step of all {n} members (no extrapolation): oracle do_mm per member in "
                       f"parallel on {threads} host threads, then the ES update; fwd "
                       f"{t1 - t0:.2f}s, update {t2 - t1:.2f}s"),
            "seconds": round(t2 - t0, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--population", type=int, default=8192)
    ap.add_argument("--cpu-members", type=int, default=8192)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("c1", "c2", "c3", "c4", "c5"), default="c3")
    ap.add_argument("--math", choices=("bf16", "f32x"), default="f32x",
                    help="C3 forward arithmetic: fp32-accurate split fp16 operands (the "
                         "reference's fp32 results), or the faster bf16 MFMA")
    ap.add_argument("--noise-cache", action="store_true",
                    help="C3: keep the factor records across steps (the reference's "
                         "LoraNoiseCache for noise_reuse = 0) instead of redrawing them every "
                         "step as its training binary does; not the default measurement")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU "
              "(across GPUs the population would shard by member, one slice of members per GPU)", file=sys.stderr)
        sys.exit(2)
    if args.workload in ("c1", "c2", "c4", "c5"):
        {"c1": bench_c1, "c2": bench_c2, "c4": bench_c4, "c5": bench_c5}[args.workload](args)
        return

    import torch
    from hyperscalees_amd import kernels as K
    from hyperscalees_amd import snn

    from hyperscalees_amd._lib import MATH_BF16, MATH_F32X
    cfg = snn.SnnConfig(n=args.population, poisson_seed=(1, 2, 3, 4),
                        math=MATH_F32X if args.math == "f32x" else MATH_BF16)
    pool_size = 60000
    pool, labels = snn.synthetic_pool(pool_size, cfg.dims[0], cfg.dims[-1], seed=0)
    idx = snn.sample_index(0, cfg.n, cfg.rows, pool_size)
    W = snn.init_weights(cfg.dims, 0, gain=snn.ACTIVE_GAIN)
    K.init(0)
    es = snn.SnnEs(cfg, W, pool, labels, idx, noise_cache=args.noise_cache)
    L = len(cfg.dims) - 1

    for i in range(args.warmup):
        es.step(epoch=i)
    torch.cuda.synchronize()

    ev = lambda: torch.cuda.Event(enable_timing=True)
    # Whole ES steps (es.step), consecutive epochs; stage events recorded on
    # the stream as the stages are issued.
    marks = []
    t0 = time.perf_counter()
    for s in range(args.steps):
        evs = {}

        def mark(name, evs=evs):
            e = ev()
            e.record()
            evs[name] = e
        mark("start")
        es.step(epoch=args.warmup + s, mark=mark)
        marks.append(evs)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1000.0 / args.steps

    def span(e, i, j):
        return e[i].elapsed_time(e[j])
    stages = ["poisson"] + [f"hidden{l}" for l in range(L - 1)] + ["readout"]
    t_poisson = np.mean([span(e, "start", "poisson") for e in marks])
    t_hidden = [np.mean([span(e, stages[l], stages[l + 1]) for e in marks]) for l in range(L - 1)]
    t_readout = np.mean([span(e, stages[L - 1], "readout") for e in marks])
    t_fwd = np.mean([span(e, "start", "readout") for e in marks])
    t_upd = np.mean([span(e, "readout", "update") for e in marks])

    # Dominant kernel: fc1's forward GEMM with the LIF fused, timed alone with
    # events on the launch stream.  On member weights (the C3 step's path):
    # k_pair_bits<.., MW> computing x W_m^T, beside the two launches that feed
    # it, the factor draw (k_pair_gen, the record alone) and the member-weight
    # product (k_member_weights); on the factored forward, the GEMM on the
    # drawn factors x[W^T|B] + (xB)A^T (or the kernel that draws inline).
    a1, b1 = es.W[0].shape
    kp1 = (b1 + 63) // 64 * 64
    draw = None
    wm_info = None
    normals = (cfg.n // 2) * cfg.rank * (a1 + b1)
    if es.mw:
        fc1_draw = lambda: K.pair_factors(cfg.keys[0], cfg.rank, cfg.sigma, 0, cfg.noise_reuse, 0,
                                          cfg.n, a1, b1, es.rec[0], None)
        draw_ms = _time_launch(fc1_draw, reps=3)
        wbytes = normals * 4
        nwm = K._lib.load().hses_member_weights_bytes(a1, b1, cfg.n, cfg.math) // 2
        wm1 = es.wm[:nwm]
        fc1_wm = lambda: K.member_weights(es.W[0], cfg.rank, cfg.sigma, 0, cfg.n, es.rec[0],
                                          math=cfg.math, out=wm1)
        wm_ms = _time_launch(fc1_wm, reps=3)
        wm_bytes = nwm * 2 + normals * 4  # written + the record read
        wm_info = {"kernel": ("k_member_weights<" + ("split" if es.split else "bf16")
                              + "> (fc1: every member's W + sign (sigma/sqrt(r)) A B^T from the "
                              "factor record, " + ("fp16 high and low parts"
                                                   if es.split else "bf16") + ")"),
                   "bound": "hbm", "launch_ms": round(wm_ms, 4),
                   "hbm_bytes": wm_bytes, "written_bytes": nwm * 2,
                   "achieved_GBps": round(wm_bytes / (wm_ms * 1e-3) / 1e9, 1),
                   "frac": round(wm_bytes / (wm_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                   "mfma_flop_per_launch": 2 * (cfg.n // 2) * a1 * kp1 * cfg.rank * 3}
        fc1_draw()
        fc1_wm()
    elif es.ahead:
        img1 = es.img_x[0] if es.split else es.img[0]
        fc1_draw = lambda: K.pair_factors(cfg.keys[0], cfg.rank, cfg.sigma, 0, cfg.noise_reuse, 0,
                                          cfg.n, a1, b1, es.rec[0], img1, split=es.split)
        draw_ms = _time_launch(fc1_draw, reps=3)
        parts = 2 if es.split else 1  # the split image holds high and low parts
        wbytes = normals * 4 + parts * (cfg.n // 2) * (cfg.rank * kp1 + a1 * 136) * 2
        fc1_draw()
    if es.ahead:
        draw = {"kernel": ("k_pair_gen (fc1 factors: every pair's exact Box-Muller normals into "
                           "the factor record"
                           + ("" if es.mw else (" and the split fp16 operand image" if es.split
                                                else " and the bf16 operand image")) + ")"),
                "bound": "valu", "launch_ms": round(draw_ms, 4), "normals_per_launch": normals,
                "g_normals_per_s": round(normals / (draw_ms * 1e-3) / 1e9, 1),
                "hbm_bytes_written": wbytes,
                "hbm_frac": round(wbytes / (draw_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
    fc1_ms = []
    for s in range(3):
        e0, e1 = ev(), ev()
        e0.record()
        if es.mw:
            K.perturbed_linear_lif_mw(es.spk[0], wm1, a1, b1, 0, cfg.n, cfg.rows, cfg.T,
                                      cfg.tau_m, cfg.v_th, math=cfg.math, spikes=es.spk[1],
                                      time_inner=es.time_inner)
        elif es.ahead:
            K.perturbed_linear_lif(es.spk[0], es.W[0], cfg.keys[0], cfg.rank, cfg.sigma, 0,
                                   cfg.noise_reuse, 0, cfg.n, cfg.rows, cfg.T, cfg.tau_m,
                                   cfg.v_th, spikes=es.spk[1], rec=es.rec[0],
                                   img=img1,
                                   time_inner=es.time_inner, math=cfg.math)
        elif es.fused:
            K.perturbed_linear_lif(es.spk[0], es.W[0], cfg.keys[0], cfg.rank, cfg.sigma, s,
                                   cfg.noise_reuse, 0, cfg.n, cfg.rows, cfg.T, cfg.tau_m,
                                   cfg.v_th, spikes=es.spk[1],
                                   rec=es.rec[0] if es.rec else None, time_inner=es.time_inner)
        else:
            K.perturbed_linear(es.spk[0], es.W[0], cfg.keys[0], cfg.rank, cfg.sigma, s,
                               cfg.noise_reuse, 0, cfg.n, cfg.rows, x_fmt=K.FMT_BITS,
                               n_time=cfg.T, math=cfg.math, out=es.cur)
        e1.record()
        torch.cuda.synchronize()
        fc1_ms.append(e0.elapsed_time(e1))
    fc1_ms = float(np.median(fc1_ms))
    M1 = cfg.n * cfg.rows * cfg.T
    # algorithmic FLOPs of the kernel: x W_m^T on member weights, else the
    # factored product (layer_flops)
    fc1_flops = 2 * M1 * b1 * a1 if es.mw else layer_flops(cfg, 0)
    # matrix-core FLOPs it issues: K padded to whole 64-k tiles (on member
    # weights with split operands, 32-k tiles: 800 at b = 784), twice for the
    # split operands (and the factored form's 256 staged columns and rank
    # product)
    if es.mw:
        kmw = (b1 + 31) // 32 * 32 if es.split else kp1
        mfma_flops = 2 * M1 * kmw * a1 * (2 if es.split else 1)
    else:
        mfma_flops = (2 * M1 * kp1 * (a1 + cfg.rank) * (2 if es.split else 1)
                      + 2 * M1 * cfg.rank * a1 * (3 if es.split else 1))
    achieved = fc1_flops / (fc1_ms * 1e-3) / 1e12
    traffic_key = ("f32x" if es.split else "bf16", bool(es.mw))

    # fc1's ES update from the factor record (HBM-bound): algorithmic bytes are
    # the record (pairs x r x (a + b) fp32) plus the gradient written.
    upd_roof = None
    if es.rec is not None:
        zf = torch.randn(cfg.n, device="cuda")
        scale1 = np.float32(-math.sqrt(cfg.n) / cfg.n)
        upd1_ms = _time_launch(lambda: K.es_update_rec(zf, 0, es.rec[0], cfg.rank, cfg.sigma, a1,
                                                       b1, scale1, out=es.grads[0]), reps=5)
        rec_bytes = (cfg.n // 2) * cfg.rank * (a1 + b1) * 4 + a1 * b1 * 4
        gbs = rec_bytes / (upd1_ms * 1e-3) / 1e9
        upd_roof = {"kernel": "k_es_rows<.., record> + k_es_reduce (fc1 ES update from the factor record)",
                    "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBPS,
                    "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBPS, 4),
                    "launch_ms": round(upd1_ms, 4), "algorithmic_bytes_per_launch": rec_bytes}

    fwd_flops = sum(layer_flops(cfg, l) for l in range(L))
    out = {
        "metric": METRIC,
        "value": round(cfg.n / (ms_per_step * 1e-3), 1),
        "unit": "member-evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": (("fp32-accurate forward: fp16 split-operand MFMA (hi*hi + hi*lo + lo*hi, fp32 "
                   "accumulate)" if es.split else "bf16 forward MFMA (fp32 accumulate)")
                  + "; ES update as fp16 split-operand MFMA (hi*hi + hi*lo + lo*hi, fp32 "
                  "accumulate; fp32-accurate)"),
        "data": "synthetic",
        "config": {
            "workload": ("C3: SNN-MLP 784-128-128-128-10, LIF decay 0.9 v_th 1.0, Poisson T=16, "
                         "N=8192, r=128, 64 samples/member from a 60000x784 pool (70% zeros), "
                         "full ES step (forward + fitness + z-score + ES update + AdamW)"),
            "population": cfg.n, "rank": cfg.rank, "T": cfg.T, "samples_per_member": cfg.rows,
            "parallelism": "single GPU",
            **({"noise_cache": ("factor records kept across steps (LoraNoiseCache, "
                                "noise_reuse = 0): the timed steps draw no factors")}
               if args.noise_cache else {}),
        },
        "fwd_member_evals_per_s": round(cfg.n / (t_fwd * 1e-3), 1),
        "es_update_GBps": round(update_bytes(cfg) / (t_upd * 1e-3) / 1e9, 2),
        "phase_ms": {"poisson": round(float(t_poisson), 3),
                     "hidden_layers": [round(float(x), 3) for x in t_hidden],
                     "readout_fitness": round(float(t_readout), 3),
                     "forward": round(float(t_fwd), 3), "es_update": round(float(t_upd), 3)},
        "fwd_tflops": round(fwd_flops / (t_fwd * 1e-3) / 1e12, 1),
        "roofline": {"kernel": (("k_mw_bits<LIF, T=16, spikes"
                                 + (", split fp16 operands" if es.split else "")
                                 + "> (fc1: x W_m^T, T=16 x 524288 rows, LIF fused)")
                                if es.mw else
                                (("k_pair_bits<LIF, T=16, spikes, factors drawn ahead"
                                  + (", split fp16 operands" if es.split else "") + "> (fc1 GEMM: "
                                  if es.ahead else "k_pair_bits (fc1: ")
                                 + "x[W^T|B] + (xB)A^T, T=16 x 524288 rows"
                                 + (", LIF fused)" if es.fused else ")"))),
                     "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": FC1_TRAFFIC.get(traffic_key, (None, None))[0],
                     "traffic_source": FC1_TRAFFIC.get(traffic_key, (None, None))[1],
                     "launch_ms": round(fc1_ms, 3),
                     "algorithmic_flop_per_launch": fc1_flops,
                     # the matrix-core work the kernel issues (split operands:
                     # each product twice) against the same fp16/bf16 peak
                     "mfma_flop_per_launch": mfma_flops,
                     "mfma_issue_frac": round(mfma_flops / (fc1_ms * 1e-3) / 1e12
                                              / PEAK_BF16_TFLOPS, 4)},
    }
    if wm_info is not None:
        out["member_weights"] = wm_info
    if draw is not None:
        out["draw"] = draw
    if upd_roof is not None:
        out["es_update_roofline"] = upd_roof
    if not args.no_cpu_baseline:
        threads, _, _ = host_cpu()
        out["cpu_baseline"] = cpu_baseline(cfg, pool, labels, idx, W, args.cpu_members, threads)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
