"""RWKV-7 components on the GPU (burn_impl/hyperscalees-models/src/llm.rs).

Wrappers over libhses.so's RWKV entry points and the ChannelMixing
composition (llm.rs:182-213).  Activations are batched over sequences:
x (nseq, T, C) fp32, one sequence per (member, sample); the recurrence state
(nseq, H, S, S).  The linear layers are the noiser's do_mm on every member's
perturbed weights (hses_perturbed_linear; sigma = 0 gives the reference's
plain Linear forward).
"""
from dataclasses import dataclass

import torch

from . import _lib
from . import kernels as K
from ._lib import MATH_F32


def _stream():
    return K._stream()


def _p(t):
    return K._p(t)


def layer_norm(x, w, b, eps=1e-5, out=None):
    """llm.rs:66-83 over the last axis of x."""
    K._dev(x, torch.float32, "x")
    out = torch.empty_like(x) if out is None else out
    C = x.shape[-1]
    _lib.call("hses_layer_norm", _p(x), x.numel() // C, C, _p(w), _p(b), eps, _p(out), _stream())
    return out


def group_norm(x, groups, w, b, eps=1e-5, out=None):
    """llm.rs:97-150: x (n, C) or (n, C, L)."""
    K._dev(x, torch.float32, "x")
    out = torch.empty_like(x) if out is None else out
    L = x.shape[2] if x.dim() == 3 else 1
    _lib.call("hses_group_norm", _p(x), x.shape[0], x.shape[1], L, groups, _p(w), _p(b), eps,
              _p(out), _stream())
    return out


def token_shift_mix(x, state, mixes, new_starts=None, out=None):
    """x (nseq, T, C), state (nseq, C), mixes (n_mix, C) -> (n_mix, nseq, T, C):
    x + ([state, x[:-1]] (0 at new starts) - x) * mix."""
    K._dev(x, torch.float32, "x")
    nseq, T, C = x.shape
    n_mix = mixes.shape[0]
    if new_starts is not None:
        K._dev(new_starts, torch.uint8, "new_starts")
    out = torch.empty((n_mix, nseq, T, C), dtype=torch.float32, device=x.device) if out is None else out
    _lib.call("hses_token_shift_mix", _p(x), _p(state), _p(new_starts), _p(mixes), n_mix, nseq, T, C,
              _p(out), _stream())
    return out


def relu_sq_(x):
    K._dev(x, torch.float32, "x")
    _lib.call("hses_relu_sq", _p(x), x.numel(), _stream())
    return x


def wkv7(r, w, k, v, a, b, s_in, length, new_starts=None, out=None, s_out=None):
    """rwkv7_inner_loop (llm.rs:235-300) for every sequence: r..b (nseq, T, H, S),
    s_in (nseq, H, S, S) -> (out (nseq, T, H, S), s_out (nseq, H, S, S))."""
    for name, t in (("r", r), ("w", w), ("k", k), ("v", v), ("a", a), ("b", b), ("s_in", s_in)):
        K._dev(t, torch.float32, name)
    nseq, T, H, S = r.shape
    if new_starts is not None:
        K._dev(new_starts, torch.uint8, "new_starts")
    out = torch.empty_like(r) if out is None else out
    s_out = torch.empty_like(s_in) if s_out is None else s_out
    _lib.call("hses_rwkv7_wkv", _p(r), _p(w), _p(k), _p(v), _p(a), _p(b), _p(s_in),
              _p(new_starts), nseq, T, H, S, length, _p(out), _p(s_out), _stream())
    return out, s_out


@dataclass
class EsLinear:
    """The noiser context of one Linear (MM) parameter: its key and the
    population layout (n members, seqs_per_member sequences each)."""
    key: int
    rank: int
    sigma: float
    epoch: int = 0
    noise_reuse: int = 0
    tid_lo: int = 0
    n: int = 1
    seqs_per_member: int = 1


def linear(x, W, es=None, math=MATH_F32):
    """x (nseq, T, in) @ W^T for W (out, in): the plain Linear (es None) or every
    member's perturbed do_mm (eggroll.rs:419-446) on its own sequences."""
    nseq, T, cin = x.shape
    if es is None:
        es = EsLinear(key=0, rank=0, sigma=0.0, n=nseq, seqs_per_member=1)
    y = K.perturbed_linear(x.reshape(1, nseq * T, cin), W, es.key, es.rank, es.sigma, es.epoch,
                           es.noise_reuse, es.tid_lo, es.n, es.seqs_per_member * T, n_time=1,
                           math=math)
    return y.reshape(nseq, T, W.shape[0])


def channel_mixing(x, state, x_k, Wk, Wv, length, new_starts=None, es_key=None, es_value=None,
                   math=MATH_F32):
    """ChannelMixing::forward (llm.rs:191-213) on every sequence:
    xk = x + ([state, x[:-1]] - x) * x_k; out = relu(xk Wk^T)^2 Wv^T; last = x[length-1].
    x (nseq, T, C), state (nseq, C), Wk (F, C), Wv (C, F)."""
    xk = token_shift_mix(x, state, x_k.reshape(1, -1), new_starts)[0]
    kk = relu_sq_(linear(xk, Wk, es_key, math))
    out = linear(kk, Wv, es_value, math)
    last = x[:, length - 1, :].contiguous()
    return out, last
