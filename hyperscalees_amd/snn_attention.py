"""Spiking self-attention transformer (C4) ES step on the GPU, composed from the
libhses kernels.

The model is SNNSelfAttentionHeadsModel (src/hyperscalees/models/
snn_self_attention_heads.py), the JAX model with LIF on Q/K/V that the C4
configuration names:

  x (T, R tokens, tin) Poisson spikes
    -> per token three perturbed projections in_q/in_k/in_v, each integrated by
       a LIF over T into a spike rate; X = mean of the three rates + pos_emb
    -> L blocks: per head h perturbed q_h/k_h/v_h projections of X, attention
       weights from row_softmax_lif (a LIF competition of the key neurons), head
       outputs A V concatenated and projected by o; X += that; then ff1, the
       LIF-gated lif_single, ff2; X += that
    -> mean over tokens -> perturbed readout `out` -> * out_gain -> logits.

Every matrix is an MM leaf perturbed with this noiser's rank-r factors
(do_mm, eggroll.rs:419-446) generated in the forward kernels; every Parameter
leaf (pos_emb, out_gain, beta and the raw thresholds q_th, k_th, v_th, attn_th,
b{b}_ff_th) is perturbed per member with dense noise (get_noisy_standard_impl,
eggroll.rs:480-503).  Leaf i has the base key (i+1)*0x9E3779B97F4A7C15 in the
order of `leaf_names` (the JAX model splits a threefry tree key per leaf, which
no reference path restates bit for bit).  The ES step z-scores the fitness,
takes do_updates of every leaf (the LoRA update for MM leaves, the dense
update for Parameter leaves) and one solver step.

The input vocabulary: each of `vocab` token ids stands for a fixed random
intensity vector of `tin` values in [0, 1]; a member's tokens are Poisson
encoded (poisson_encode_fused_oxide.rs:61-106 with a row gather).
"""
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from . import kernels as K
from ._lib import ADAMW, FMT_F32, MATH_F32, REWARD_LOGLIK, SGD

KEY_MUL = 0x9E3779B97F4A7C15
MM, PARAM = 1, 0   # es_map classes (common.py:6-7)


@dataclass
class SaConfig:
    tin: int = 16            # values per token
    ntok: int = 64           # tokens per sequence (R)
    d_model: int = 64
    heads: int = 4
    blocks: int = 2
    classes: int = 10
    vocab: int = 256
    T: int = 8               # Poisson / LIF time steps
    n: int = 1024            # population size N (one sequence per member)
    rank: int = 8
    sigma: float = 0.02
    tau_m: float = 20.0      # rand_init default (snn_self_attention_heads.py:96)
    v_th: float = 0.05       # initial thresholds (softplus of the raw leaves)
    g_inh: float = 0.5       # DEFAULT_CORE_ARGS (snn_self_attention_heads.py:28-32)
    n_iter: int = 8
    noise_reuse: int = 0
    solver: int = ADAMW
    lr: float = 0.01
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 1e-4
    poisson_seed: tuple = (9, 10, 11, 12)

    def __post_init__(self):
        if self.d_model % self.heads:
            raise ValueError("d_model must be a multiple of heads")
        if self.ntok > 64 or self.head_dim > 64:
            raise ValueError("at most 64 tokens per member and 64 channels per head")

    @property
    def head_dim(self):
        return self.d_model // self.heads


def leaf_names(cfg):
    """(name, shape, class) of every leaf in key order: the Rust model's params()
    order (snn_transformer.rs:223-249) followed by the JAX model's thresholds."""
    d, hd, tin = cfg.d_model, cfg.head_dim, cfg.tin
    L = [("in_q", (d, tin), MM), ("in_k", (d, tin), MM), ("in_v", (d, tin), MM),
         ("pos_emb", (cfg.ntok, d), PARAM)]
    for b in range(cfg.blocks):
        for kind in "qkv":
            L += [(f"b{b}_{kind}{h}", (hd, d), MM) for h in range(cfg.heads)]
        L += [(f"b{b}_o", (d, d), MM), (f"b{b}_ff1", (d, d), MM), (f"b{b}_ff2", (d, d), MM)]
    L += [("out", (cfg.classes, d), MM), ("out_gain", (1, 1), PARAM), ("beta", (1, 1), PARAM)]
    L += [(n, (1, 1), PARAM) for n in ("q_th", "k_th", "v_th", "attn_th")]
    L += [(f"b{b}_ff_th", (1, 1), PARAM) for b in range(cfg.blocks)]
    return L


def leaf_keys(cfg):
    return {name: ((i + 1) * KEY_MUL) % 2**64 for i, (name, _, _) in enumerate(leaf_names(cfg))}


def init_params(cfg, seed=0):
    """rand_init (snn_self_attention_heads.py:96-151): MM leaves N(0, 1/in),
    pos_emb 0, out_gain 1, raw thresholds log(exp(v_th) - 1), raw beta
    log(exp(1/sqrt(head_dim)) - 1); host fp32 arrays from a seeded fixture RNG."""
    rng = np.random.default_rng(seed)
    P = {}
    raw_vth = np.float32(np.log(np.expm1(np.float32(cfg.v_th))))
    raw_beta = np.float32(np.log(np.expm1(np.float32(1.0 / np.sqrt(cfg.head_dim)))))
    for name, shape, cls in leaf_names(cfg):
        if cls == MM:
            P[name] = (rng.standard_normal(shape) / np.sqrt(shape[1])).astype(np.float32)
        elif name == "pos_emb":
            P[name] = np.zeros(shape, np.float32)
        elif name == "out_gain":
            P[name] = np.ones(shape, np.float32)
        elif name == "beta":
            P[name] = np.full(shape, raw_beta, np.float32)
        else:
            P[name] = np.full(shape, raw_vth, np.float32)
    return P


def synthetic_vocab(cfg, seed=0):
    """Intensity vectors (vocab, tin) in [0, 1) standing for the token ids."""
    return np.random.default_rng(seed + 100).random((cfg.vocab, cfg.tin), dtype=np.float32)


class SpikingAttentionEs:
    """Device-resident population forward and ES step of the C4 model."""

    def __init__(self, cfg, params, vocab, device="cuda"):
        self.cfg = c = cfg
        self.dev = torch.device(device)
        self.streams = None  # side streams of the ES update, made on first use
        self.leaves = leaf_names(cfg)
        self.keys = leaf_keys(cfg)
        self.P = {k: torch.from_numpy(np.ascontiguousarray(v)).to(self.dev) for k, v in params.items()}
        self.vocab = torch.from_numpy(np.ascontiguousarray(vocab, np.float32)).to(self.dev)
        n, R, d = c.n, c.ntok, c.d_model
        M = n * R
        self.M = M
        f32 = dict(dtype=torch.float32, device=self.dev)
        self.spk = torch.empty((c.T, M, c.tin), **f32)
        self.cur = [torch.empty((c.T, M, d), **f32) for _ in range(3)]
        self.X = torch.empty((M, d), **f32)
        self.Q, self.Kt, self.V, self.O, self.D = (torch.empty((M, d), **f32) for _ in range(5))
        self.pooled = torch.empty((n, d), **f32)
        self.logits = torch.empty((n, c.classes), **f32)
        self.raw = torch.empty(n, **f32)
        self.noisy = {}     # per-member Parameter leaves (n, a, b)
        self.th = {}        # per-member softplus of the raw thresholds / beta (n,)
        self.grads = {k: torch.zeros_like(v) for k, v in self.P.items()}
        adam = c.solver != SGD
        self.m = {k: torch.zeros_like(v) if adam else None for k, v in self.P.items()}
        self.v = {k: torch.zeros_like(v) if adam else None for k, v in self.P.items()}
        self.step_t = 0

    # -- pieces ---------------------------------------------------------------
    def _side_streams(self):
        if self.streams is None:
            self.streams = [torch.cuda.Stream(device=self.dev) for _ in range(4)]
        return self.streams

    def _fan_out(self, calls):
        """Independent launches round-robin on the side streams (default priority,
        a workspace per stream), joined into the current stream afterwards."""
        main = torch.cuda.current_stream()
        ready = torch.cuda.Event()
        ready.record(main)
        sides = self._side_streams()
        for side in sides:
            side.wait_event(ready)
        for i, fn in enumerate(calls):
            with torch.cuda.stream(sides[i % len(sides)]):
                fn()
        for side in sides:
            main.wait_stream(side)

    def _linear(self, x, x_stride, x_plane, n_time, name, rpm, n, y, y_off, y_stride, y_plane,
                epoch):
        """Perturbed do_mm of MM leaf `name` over the population (fp32 math), rows
        of member m at [m rpm, (m+1) rpm) of each time plane, written into
        y[:, y_off:] with row stride y_stride."""
        c = self.cfg
        W = self.P[name]
        a, b = W.shape
        lib = _lib.load()
        wbytes = int(lib.hses_perturbed_linear_workspace(a, b, c.rank, n, rpm, n_time, MATH_F32))
        work = K._workspace(wbytes, self.dev)
        yp = y.data_ptr() + 4 * y_off
        _lib.call("hses_perturbed_linear", K._p(x), FMT_F32, x_stride, x_plane, n_time, K._p(W),
                  a, b, self.keys[name], c.rank, c.sigma, epoch, c.noise_reuse, 0, n, rpm, yp,
                  y_stride, y_plane, MATH_F32, K._p(work), wbytes, K._stream())

    def perturb_params(self, epoch):
        """Every member's Parameter leaves (get_noisy_standard) and the softplus
        of its thresholds and beta."""
        c = self.cfg
        for name, _shape, cls in self.leaves:
            if cls != PARAM:
                continue
            self.noisy[name] = K.noisy_standard(self.P[name], self.keys[name], c.sigma, epoch,
                                                c.noise_reuse, (0, c.n))
            if name.endswith("_th") or name == "beta":
                y = torch.empty(c.n, dtype=torch.float32, device=self.dev)
                _lib.call("hses_softplus", K._p(self.noisy[name]), c.n, K._p(y), K._stream())
                self.th[name] = y

    def encode(self, epoch):
        """Poisson spikes, the three encoder projections and their LIF rates -> X."""
        c = self.cfg
        R, d, M = c.ntok, c.d_model, self.M
        self._fan_out([
            (lambda i=i, name=name: self._linear(self.spk, c.tin, M * c.tin, c.T, name, R, c.n,
                                                 self.cur[i], 0, d, M * d, epoch))
            for i, name in enumerate(("in_q", "in_k", "in_v"))])
        _lib.call("hses_sa_encode", K._p(self.cur[0]), K._p(self.cur[1]), K._p(self.cur[2]), c.T,
                  M, d, R, K._p(self.th["q_th"]), K._p(self.th["k_th"]), K._p(self.th["v_th"]),
                  c.tau_m, K._p(self.noisy["pos_emb"]), 1, K._p(self.X), K._stream())

    def attention_block(self, b, epoch, trace=None):
        c = self.cfg
        R, d, M, hd = c.ntok, c.d_model, self.M, c.head_dim
        # the 3 x heads projections are independent
        self._fan_out([
            (lambda kind=kind, buf=buf, h=h: self._linear(self.X, d, 0, 1, f"b{b}_{kind}{h}", R,
                                                          c.n, buf, h * hd, d, 0, epoch))
            for kind, buf in (("q", self.Q), ("k", self.Kt), ("v", self.V))
            for h in range(c.heads)])
        _lib.call("hses_sa_attention", K._p(self.Q), K._p(self.Kt), K._p(self.V), d, c.n, R,
                  c.heads, hd, K._p(self.th["beta"]), K._p(self.th["attn_th"]), c.g_inh, c.tau_m,
                  c.n_iter, K._p(self.O), K._stream())
        if trace is not None:
            trace[f"b{b}_in"] = self.X.clone()
            for nm, t in (("q", self.Q), ("k", self.Kt), ("v", self.V), ("att", self.O)):
                trace[f"b{b}_{nm}"] = t.clone()
        self._linear(self.O, d, 0, 1, f"b{b}_o", R, c.n, self.D, 0, d, 0, epoch)
        _lib.call("hses_add_inplace", K._p(self.X), K._p(self.D), M * d, K._stream())
        if trace is not None:
            trace[f"b{b}_x_att"] = self.X.clone()
        self._linear(self.X, d, 0, 1, f"b{b}_ff1", R, c.n, self.D, 0, d, 0, epoch)
        _lib.call("hses_sa_ffn_spike", K._p(self.D), M, d, R, K._p(self.th[f"b{b}_ff_th"]),
                  K._p(self.O), K._stream())
        if trace is not None:
            trace[f"b{b}_ff1"] = self.D.clone()
            trace[f"b{b}_act"] = self.O.clone()
        self._linear(self.O, d, 0, 1, f"b{b}_ff2", R, c.n, self.D, 0, d, 0, epoch)
        _lib.call("hses_add_inplace", K._p(self.X), K._p(self.D), M * d, K._stream())

    def readout(self, epoch):
        c = self.cfg
        _lib.call("hses_sa_pool", K._p(self.X), c.n, c.ntok, c.d_model, K._p(self.pooled),
                  K._stream())
        self._linear(self.pooled, c.d_model, 0, 1, "out", 1, c.n, self.logits, 0, c.classes, 0,
                     epoch)
        _lib.call("hses_scale_rows", K._p(self.logits), c.n, c.classes,
                  K._p(self.noisy["out_gain"]), K._stream())

    # -- step -----------------------------------------------------------------
    def forward(self, tokens, labels, epoch=0, trace=None):
        """tokens (n, ntok) int32 and labels (n,) int32 on the device -> raw fitness
        (n,): each member's log-likelihood of its label.  With a dict `trace`
        the stage outputs are copied into it."""
        c = self.cfg
        K._dev(tokens, torch.int32, "tokens")
        K._dev(labels, torch.int32, "labels")
        if tokens.shape != (c.n, c.ntok):
            raise ValueError(f"tokens must be ({c.n}, {c.ntok})")
        self.perturb_params(epoch)
        K.poisson_encode(self.vocab, c.T, c.poisson_seed, FMT_F32, out=self.spk,
                         rows_index=tokens.view(-1))
        self.encode(epoch)
        if trace is not None:
            trace["spk"] = self.spk.clone()
            for i, q in enumerate("qkv"):
                trace[f"cur_{q}"] = self.cur[i].clone()
            trace["x_enc"] = self.X.clone()
        for b in range(c.blocks):
            self.attention_block(b, epoch, trace)
        if trace is not None:
            trace["x_out"] = self.X.clone()
        self.readout(epoch)
        if trace is not None:
            trace["pooled"] = self.pooled.clone()
            trace["logits"] = self.logits.clone()
        return K.member_fitness(self.logits, labels, c.n, 1, REWARD_LOGLIK, out=self.raw)

    def update(self, raw_fit, epoch=0):
        """z-score, do_updates of every leaf and one solver step."""
        c = self.cfg
        z, _ = K.convert_fitnesses(raw_fit)
        scale = np.float32(-math.sqrt(c.n) / c.n)   # -g sqrt(N), g = (1/N) sum (eggroll.rs:403)
        self.step_t += 1
        # The leaves' updates are independent and each is a few tens of microseconds
        # on a small part of the GPU: they run round-robin on side streams (default
        # priority, each with its own workspace), joined before the next forward.
        main = torch.cuda.current_stream()
        ready = torch.cuda.Event()
        ready.record(main)
        for side in self._side_streams():
            side.wait_event(ready)
            z.record_stream(side)
        for i, (name, (a, b), cls) in enumerate(self.leaves):
            with torch.cuda.stream(self.streams[i % len(self.streams)]):
                if cls == MM:
                    K.es_update(z, 0, self.keys[name], c.rank, c.sigma, epoch, c.noise_reuse, a,
                                b, scale, out=self.grads[name])
                else:
                    K.full_update(z, 0, self.keys[name], c.sigma, epoch, c.noise_reuse, a, b,
                                  scale, out=self.grads[name])
                K.solver_step(c.solver, c.lr, self.P[name], self.grads[name], self.m[name],
                              self.v[name], step_t=self.step_t, beta1=c.beta1, beta2=c.beta2,
                              eps=c.eps, wd=c.weight_decay if c.solver == ADAMW else 0.0)
        for side in self.streams:
            main.wait_stream(side)
        return z

    def step(self, tokens, labels, epoch=0):
        fit = self.forward(tokens, labels, epoch)
        self.update(fit, epoch)
        return fit


def forward_flops(cfg):
    """Multiply-add FLOPs (x2) of one population forward: the perturbed
    projections (shared product + rank-r terms), the attention scores and A V."""
    c = cfg
    R, d, hd, r, H = c.ntok, c.d_model, c.head_dim, c.rank, c.heads
    rows = c.n * R
    fl = 3 * c.T * rows * (2 * c.tin * d + 2 * r * (c.tin + d))
    per_block = (3 * H * (2 * d * hd + 2 * r * (d + hd)) + 3 * (2 * d * d + 4 * r * d))
    fl += c.blocks * rows * per_block
    fl += c.blocks * c.n * H * (2 * R * R * hd) * 2      # scores and A V
    fl += c.n * (2 * d * c.classes + 2 * r * (d + c.classes))
    return fl
