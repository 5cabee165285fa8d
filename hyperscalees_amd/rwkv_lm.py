"""RWKV-7 language model EggRoll ES step on the GPU (the C5 workload).

The model is BaseRWKV (src/hyperscalees/models/llm/rwkv7.py:117-253) with the
burn port's components (burn_impl/hyperscalees-models/src/llm.rs):
  x = ln0(emb[tokens]); per block x += att(ln1(x)), x += ffn(ln2(x)), the
  value of block 0 carried to the later blocks as v_first; logits =
  ln_out(x) head^T.
The ES map is rwkv7.py:161-180: every matrix (the Linear receptance / key /
value / output, the Tmm low-rank branches w1..g2, the ChannelMixing key /
value) is an MM parameter, perturbed per member by its rank-r factors
(do_mm / do_Tmm); emb and head are excluded; the vectors are full-rank
parameters held frozen, as the reference's LLM evolution drivers run them
(freeze_nonlora = True, llm_experiments/general_do_evolution.py:74).  So one
ES step is: the population's forward, the next-token log-likelihood fitness
averaged over each member's positions, the z-score (eggroll.rs:967-992), and
per MM parameter the ES gradient -sqrt(N) (1/N) sum_i z_i A_i B_i^T
(eggroll.rs:384-404) with one solver step (noiser.rs:155-225).

Activations are (sequences, T, C) fp32, one or more sequences per member;
the linears run on MFMA in cfg.math (bf16 operands with fp32 accumulation by
default, as the C5 configuration asks).
"""
import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import kernels as K
from . import rwkv
from ._lib import ADAMW, MATH_BF16, REWARD_LOGLIK, SGD
from . import _lib

TM_MATRICES = ("receptance", "key", "value", "output", "w1", "w2", "v1", "v2", "a1", "a2",
               "g1", "g2")
TM_VECTORS = ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "v0", "a0", "k_k", "k_a", "r_k",
              "ln_w", "ln_b")
FFN_MATRICES = ("ffn_key", "ffn_value")
BLOCK_VECTORS = ("ffn_x_k", "ln1_w", "ln1_b", "ln2_w", "ln2_b")
KEY_MUL = 0x9E3779B97F4A7C15


def lora_widths(C):
    """The low-rank widths of RWKV-7's decay, value, in-context-rate and gate
    branches for model width C (the RWKV-7 release's sizing rule)."""
    def r32(v):
        return max(32, int(round(v / 32)) * 32)
    return r32(1.8 * C ** 0.5), r32(1.3 * C ** 0.5), r32(1.8 * C ** 0.5), r32(0.6 * C ** 0.8)


@dataclass
class RwkvLmConfig:
    n_layer: int = 4
    d_model: int = 512
    head_size: int = 64
    vocab: int = 256
    ffn_mult: int = 4
    seq_len: int = 128             # input positions per sequence (targets are the next tokens)
    seqs_per_member: int = 1
    n: int = 2048                  # population size N
    rank: int = 1
    sigma: float = 0.01
    noise_reuse: int = 0
    math: int = MATH_BF16
    solver: int = SGD
    lr: float = 1e-3
    beta1: float = 0.9             # Adam / AdamW (Solver::adam, noiser.rs:101-108)
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 1e-4     # AdamW only (Solver::adamw, noiser.rs:111-119)
    init_std: float = 0.02
    widths: tuple = field(default=None)

    def __post_init__(self):
        if self.widths is None:
            self.widths = lora_widths(self.d_model)
        if self.d_model % self.head_size or self.head_size > 64:
            raise ValueError("d_model must be heads of at most 64 channels")


def init_params(cfg, seed=0):
    """Random-init weights: matrices and mixing vectors N(0, init_std^2), the
    norms' weights 1 and biases 0.  Returns host fp32 arrays: a dict with
    emb, ln0_w, ln0_b, ln_out_w, ln_out_b, head and `blocks`, a list of dicts
    with the TimeMixing names, ffn_x_k, ffn_key (F, C), ffn_value (C, F) and
    ln1/ln2.  Linear weights are (out, in), Tmm weights (in, out)."""
    rng = np.random.default_rng(seed)
    C, V, F = cfg.d_model, cfg.vocab, cfg.ffn_mult * cfg.d_model
    dw, dv, da, dg = cfg.widths

    def nrm(*shape):
        return (rng.standard_normal(shape) * cfg.init_std).astype(np.float32)

    P = {"emb": nrm(V, C), "head": nrm(V, C), "ln0_w": np.ones(C, np.float32),
         "ln0_b": np.zeros(C, np.float32), "ln_out_w": np.ones(C, np.float32),
         "ln_out_b": np.zeros(C, np.float32), "blocks": []}
    for _ in range(cfg.n_layer):
        B = {n: nrm(C) for n in TM_VECTORS + ("ffn_x_k",)}
        for n in ("ln_w", "ln1_w", "ln2_w"):
            B[n] = np.ones(C, np.float32)
        for n in ("ln_b", "ln1_b", "ln2_b"):
            B[n] = np.zeros(C, np.float32)
        for n in ("receptance", "key", "value", "output"):
            B[n] = nrm(C, C)
        for n1, n2, d in (("w1", "w2", dw), ("v1", "v2", dv), ("a1", "a2", da), ("g1", "g2", dg)):
            B[n1], B[n2] = nrm(C, d), nrm(d, C)
        B["ffn_key"], B["ffn_value"] = nrm(F, C), nrm(C, F)
        P["blocks"].append(B)
    return P


def mm_names(n_layer):
    """(layer, name) of every MM parameter, in key order."""
    return [(l, n) for l in range(n_layer) for n in TM_MATRICES + FFN_MATRICES]


class RwkvLmEs:
    """The population forward and the ES step of the RWKV-7 LM on one GPU."""

    def __init__(self, cfg, params, device="cuda", key_seed=0):
        self.cfg = cfg
        self.dev = torch.device(device)

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(self.dev)

        self.P = {k: dev(v) for k, v in params.items() if k != "blocks"}
        self.blocks = [{k: dev(v) for k, v in b.items()} for b in params["blocks"]]
        # one base key per MM parameter (the JAX model splits a tree key per leaf)
        self.keys = {ln: ((i + 1 + key_seed) * KEY_MUL) % 2**64
                     for i, ln in enumerate(mm_names(cfg.n_layer))}
        self.grads = {ln: torch.empty_like(self.blocks[ln[0]][ln[1]]) for ln in self.keys}
        # Adam / AdamW moments m = v = 0 per parameter (Solver::init_state, noiser.rs:126-149)
        adam = cfg.solver != SGD
        self.m = {ln: torch.zeros_like(self.blocks[ln[0]][ln[1]]) if adam else None
                  for ln in self.keys}
        self.v = {ln: torch.zeros_like(self.blocks[ln[0]][ln[1]]) if adam else None
                  for ln in self.keys}
        self.step_t = 0
        self.streams = None
        S, C = cfg.head_size, cfg.d_model
        nseq = cfg.n * cfg.seqs_per_member
        self.state0 = torch.zeros((nseq, 2 + S, C), dtype=torch.float32, device=self.dev)
        self.vf0 = torch.zeros((nseq, cfg.seq_len, C), dtype=torch.float32, device=self.dev)

    def _es(self, l, epoch, tid_lo, n):
        c = self.cfg
        return {name: rwkv.EsLinear(key=self.keys[(l, name)], rank=c.rank, sigma=c.sigma,
                                    epoch=epoch, noise_reuse=c.noise_reuse, tid_lo=tid_lo, n=n,
                                    seqs_per_member=c.seqs_per_member)
                for name in TM_MATRICES + FFN_MATRICES}

    def logits(self, tokens, epoch=0, tid_lo=0, perturb=True, state=None):
        """tokens (n * seqs_per_member, T) int32 on the device -> logits
        (n * seqs_per_member * T, V) fp32; every member's sequences run with its
        perturbed MM parameters (perturb False: the plain model).  With `state`
        (n_layer, sequences, 2 + S, C) -- per layer row 0 the ChannelMixing shift,
        rows 1.. TimeMixing's state (rwkv7.py:182-187) -- the sequences continue
        from it and (logits, new state) is returned."""
        c = self.cfg
        nseq, T = tokens.shape
        n = nseq // c.seqs_per_member
        if n * c.seqs_per_member != nseq:
            raise ValueError("sequences are not a whole number of members")
        C, H, V = c.d_model, c.d_model // c.head_size, c.vocab
        rows = nseq * T
        K._dev(tokens, torch.int32, "tokens")
        x = torch.empty((rows, C), dtype=torch.float32, device=self.dev)
        h = torch.empty_like(x)
        _lib.call("hses_embed_layer_norm", K._p(tokens), rows, K._p(self.P["emb"]), V, C,
                  K._p(self.P["ln0_w"]), K._p(self.P["ln0_b"]), 1e-5, K._p(x), K._stream())
        bf = c.math == MATH_BF16
        x3 = x.view(nseq, T, C)
        carry = state is not None
        if carry:
            if state.shape != (c.n_layer, nseq, 2 + c.head_size, C):
                raise ValueError("state must be (n_layer, sequences, 2 + S, C)")
            new_state = torch.empty_like(state)
        if T == c.seq_len and nseq == self.state0.shape[0]:
            zero, vf = self.state0, self.vf0
        else:
            zero = torch.zeros((nseq, 2 + c.head_size, C), dtype=torch.float32, device=self.dev)
            vf = torch.zeros((nseq, T, C), dtype=torch.float32, device=self.dev)
        # Each LayerNorm that feeds a token shift is formed with that shift (and the
        # residual add before it) in one pass: the normalised rows never go to memory.
        def tm_mixes(B, delta, st):
            mixes = torch.stack([B[nm] for nm in rwkv.TM_MIXES])
            return rwkv.add_layer_norm_shift(x3, delta, B["ln1_w"], B["ln1_b"], 1e-5, st[:, 1, :],
                                             mixes, bf16=bf, want_last=carry)

        d = None  # block 0's ln1 reads the embedding (no residual add)
        st = state[0] if carry else zero
        xm, xm_last = tm_mixes(self.blocks[0], d, st)
        for l, B in enumerate(self.blocks):
            es = self._es(l, epoch, tid_lo, n) if perturb else {}
            d, st_tm, vf = rwkv.time_mixing(B, None, st[:, 1:, :] if carry else None, vf, H, T, l,
                                            es=es, math=c.math, want_state=carry, xm=xm,
                                            x_last=xm_last)
            xk, xk_last = rwkv.add_layer_norm_shift(x3, d.view(nseq, T, C), B["ln2_w"], B["ln2_b"],
                                                    1e-5, st[:, 0, :], B["ffn_x_k"].reshape(1, -1),
                                                    bf16=bf, want_last=carry)
            d, last = rwkv.channel_mixing(None, None, B["ffn_x_k"], B["ffn_key"], B["ffn_value"], T,
                                          es_key=es.get("ffn_key"), es_value=es.get("ffn_value"),
                                          math=c.math, want_last=carry, xk=xk[0], last=xk_last)
            if carry:
                new_state[l][:, 1:, :] = st_tm
                new_state[l][:, 0, :] = last
            if l + 1 < len(self.blocks):
                st = state[l + 1] if carry else zero
                xm, xm_last = tm_mixes(self.blocks[l + 1], d.view(nseq, T, C), st)
            else:
                _lib.call("hses_add_layer_norm", K._p(x), K._p(d), rows, C, K._p(self.P["ln_out_w"]),
                          K._p(self.P["ln_out_b"]), 1e-5, K._p(h), K._stream())
        lg = rwkv.linear(h.view(1, rows, C), self.P["head"], None, c.math).view(rows, V)
        return (lg, new_state) if carry else lg

    def forward(self, tokens, epoch=0, tid_lo=0):
        """tokens (n * seqs_per_member, T + 1) int32: inputs are the first T ids,
        targets the next ones.  Returns the raw fitness (n,): each member's mean
        next-token log-likelihood."""
        c = self.cfg
        nseq = tokens.shape[0]
        inp = tokens[:, :-1].contiguous()
        tgt = tokens[:, 1:].contiguous()
        lg = self.logits(inp, epoch, tid_lo)
        n = nseq // c.seqs_per_member
        return K.member_fitness(lg, tgt.view(-1), n, tgt.numel() // n, REWARD_LOGLIK)

    def update(self, raw_fit, epoch=0):
        c = self.cfg
        z, _ = K.convert_fitnesses(raw_fit)
        n = raw_fit.numel()
        scale = np.float32(-math.sqrt(n) / n)   # -g sqrt(N), g = (1/N) sum (eggroll.rs:403)
        self.step_t += 1
        # The parameters' updates are independent and each fills only part of the GPU
        # at r = 1: they run round-robin on side streams (default priority, each with
        # its own workspace), joined before the next forward.
        if self.streams is None:
            self.streams = [torch.cuda.Stream(device=self.dev) for _ in range(4)]
        main = torch.cuda.current_stream()
        ready = torch.cuda.Event()
        ready.record(main)
        for side in self.streams:
            side.wait_event(ready)
            z.record_stream(side)
        for i, ((l, name), key) in enumerate(self.keys.items()):
            with torch.cuda.stream(self.streams[i % len(self.streams)]):
                W = self.blocks[l][name]
                a, b = W.shape
                K.es_update(z, 0, key, c.rank, c.sigma, epoch, c.noise_reuse, a, b, scale,
                            out=self.grads[(l, name)])
                K.solver_step(c.solver, c.lr, W, self.grads[(l, name)], self.m[(l, name)],
                              self.v[(l, name)], step_t=self.step_t, beta1=c.beta1,
                              beta2=c.beta2, eps=c.eps,
                              wd=c.weight_decay if c.solver == ADAMW else 0.0)
        for side in self.streams:
            main.wait_stream(side)
        return z

    def step(self, tokens, epoch=0):
        """One ES step on the given token batch; returns the raw fitness (n,)."""
        fit = self.forward(tokens, epoch)
        self.update(fit, epoch)
        return fit


def forward_flops(cfg, n_seq=None):
    """Multiply-add FLOPs (x2) of one population forward: the shared-weight
    products, the rank-r corrections of the MM parameters and the head."""
    c = cfg
    n_seq = c.n * c.seqs_per_member if n_seq is None else n_seq
    rows = n_seq * c.seq_len
    C, F, V, r = c.d_model, c.ffn_mult * c.d_model, c.vocab, c.rank
    dw, dv, da, dg = c.widths
    per_row = 0
    for l in range(c.n_layer):
        mats = [(C, C)] * 4 + [(C, dw), (dw, C), (C, da), (da, C), (C, dg), (dg, C), (F, C), (C, F)]
        if l > 0:
            mats += [(C, dv), (dv, C)]
        for a, b in mats:
            per_row += 2 * a * b + 2 * r * (a + b)
    per_row += 2 * V * C
    return rows * per_row
