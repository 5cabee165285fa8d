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
from ._lib import ACT_RELU_SQ, ACT_SIGMOID, ACT_TANH, FMT_BF16, FMT_F32, MATH_BF16, MATH_F32


_SIDE = {}  # device index -> side streams (default priority)


def _side_streams(dev):
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _SIDE:
        _SIDE[key] = [torch.cuda.Stream(device=dev) for _ in range(4)]
    return _SIDE[key]


def _fan_out(jobs, inputs):
    """Run independent launches round-robin on side streams, joined into the
    current stream.  `inputs` (made on the current stream) is recorded on the
    side streams and every job's output on the current stream, so the caching
    allocator reuses neither block before the stream that reads it is done."""
    main = torch.cuda.current_stream()
    ready = torch.cuda.Event()
    ready.record(main)
    sides = _side_streams(inputs.device)
    for side in sides:
        side.wait_event(ready)
        inputs.record_stream(side)
    out = {}
    for i, (name, fn) in enumerate(jobs.items()):
        with torch.cuda.stream(sides[i % len(sides)]):
            out[name] = fn()
    for side in sides:
        main.wait_stream(side)
    for t in out.values():
        t.record_stream(main)
    return out


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


def token_shift_mix(x, state, mixes, new_starts=None, out=None, bf16=False):
    """x (nseq, T, C), state (nseq, C), mixes (n_mix, C) -> (n_mix, nseq, T, C):
    x + ([state, x[:-1]] (0 at new starts) - x) * mix, in fp32 or (bf16) rounded
    to bfloat16 for a bf16-math forward."""
    K._dev(x, torch.float32, "x")
    nseq, T, C = x.shape
    n_mix = mixes.shape[0]
    if new_starts is not None:
        K._dev(new_starts, torch.uint8, "new_starts")
    dt = torch.bfloat16 if bf16 else torch.float32
    out = torch.empty((n_mix, nseq, T, C), dtype=dt, device=x.device) if out is None else out
    K._dev(out, dt, "out")
    _lib.call("hses_token_shift_mix", _p(x), _p(state), _p(new_starts), _p(mixes), n_mix, nseq, T, C,
              _p(out), FMT_BF16 if bf16 else FMT_F32, _stream())
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


def _fmt(x):
    return FMT_BF16 if x.dtype == torch.bfloat16 else FMT_F32


def linear(x, W, es=None, math=MATH_F32, act=0, out_bf16=False):
    """x (nseq, T, in) (fp32 or bf16) @ W^T for W (out, in): the plain Linear (es
    None) or every member's perturbed do_mm (eggroll.rs:419-446) on its own
    sequences; `act` (hses_act) applies the elementwise op that follows."""
    nseq, T, cin = x.shape
    if es is None:
        es = EsLinear(key=0, rank=0, sigma=0.0, n=nseq, seqs_per_member=1)
    y = K.perturbed_linear(x.reshape(1, nseq * T, cin), W, es.key, es.rank, es.sigma, es.epoch,
                           es.noise_reuse, es.tid_lo, es.n, es.seqs_per_member * T, n_time=1,
                           math=math, act=act, x_fmt=_fmt(x), out_bf16=out_bf16)
    return y.reshape(nseq, T, W.shape[0])


def add_layer_norm_shift(x, delta, w, b, eps, state, mixes, new_starts=None, bf16=False,
                         length=None, want_last=False):
    """A block's residual add (x += delta in place; delta None: x only read), the
    LayerNorm y of x, and the next module's token shift of y with the mixing
    vectors mixes (n_mix, C): returns (out (n_mix, nseq, T, C), y[:, length-1]
    or None).  x (nseq, T, C), state (nseq, C) the previous token's y.  One fused
    kernel where it applies (C 256 / 512 / 1024, 1 or 6 mixes), else the two
    steps; the values are the same bit for bit."""
    K._dev(x, torch.float32, "x")
    nseq, T, C = x.shape
    length = T if length is None else length
    n_mix = mixes.shape[0]
    dt = torch.bfloat16 if bf16 else torch.float32
    state = state.contiguous()
    mixes = mixes.contiguous()
    if C in (256, 512, 1024) and n_mix in (1, 6):
        out = torch.empty((n_mix, nseq, T, C), dtype=dt, device=x.device)
        last = torch.empty((nseq, C), dtype=torch.float32, device=x.device) if want_last else None
        if new_starts is not None:
            K._dev(new_starts, torch.uint8, "new_starts")
        _lib.call("hses_add_ln_shift", _p(x), _p(delta), nseq, T, C, _p(w), _p(b), eps, _p(state),
                  _p(new_starts), _p(mixes), n_mix, _p(out), FMT_BF16 if bf16 else FMT_F32,
                  _p(last), length, _stream())
        return out, last
    y = torch.empty_like(x)
    if delta is None:
        layer_norm(x, w, b, eps, out=y)
    else:
        _lib.call("hses_add_layer_norm", _p(x), _p(delta), nseq * T, C, _p(w), _p(b), eps, _p(y),
                  _stream())
    out = token_shift_mix(y, state, mixes, new_starts, bf16=bf16)
    return out, (y[:, length - 1, :].contiguous() if want_last else None)


def channel_mixing(x, state, x_k, Wk, Wv, length, new_starts=None, es_key=None, es_value=None,
                   math=MATH_F32, want_last=True, xk=None, last=None):
    """ChannelMixing::forward (llm.rs:191-213) on every sequence:
    xk = x + ([state, x[:-1]] - x) * x_k; out = relu(xk Wk^T)^2 Wv^T; last = x[length-1].
    x (nseq, T, C), state (nseq, C), Wk (F, C), Wv (C, F).  With xk (and last)
    given -- the shift formed by add_layer_norm_shift -- x may be None."""
    # with bf16 math the intermediates only feed the next bf16 product, which
    # would round them the same way: store them as bf16
    bf = math == MATH_BF16
    if xk is None:
        xk = token_shift_mix(x, state, x_k.reshape(1, -1), new_starts, bf16=bf)[0]
    kk = linear(xk, Wk, es_key, math, act=ACT_RELU_SQ, out_bf16=bf)
    out = linear(kk, Wv, es_value, math)
    if last is None and want_last:
        last = x[:, length - 1, :].contiguous()
    return out, (last if want_last else None)


def linear_t(x, W, es=None, math=MATH_F32, act=0, out_bf16=False):
    """x (nseq, T, in) @ W for W (in, out): the plain Tmm (es None) or every
    member's perturbed do_Tmm (common.rs:156-159, eggroll.rs:450-477), then
    the activation `act` (hses_act)."""
    nseq, T, cin = x.shape
    if es is None:
        es = EsLinear(key=0, rank=0, sigma=0.0, n=nseq, seqs_per_member=1)
    y = K.perturbed_linear_t(x.reshape(1, nseq * T, cin), W, es.key, es.rank, es.sigma, es.epoch,
                             es.noise_reuse, es.tid_lo, es.n, es.seqs_per_member * T, n_time=1,
                             math=math, act=act, x_fmt=_fmt(x), out_bf16=out_bf16)
    return y.reshape(nseq, T, W.shape[1])


def rwkv_act_(x, kind):
    """In place: kind 0 tanh, kind 1 sigmoid."""
    K._dev(x, torch.float32, "x")
    _lib.call("hses_rwkv_act", _p(x), x.numel(), kind, _stream())
    return x


TM_MIXES = ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")


def time_mixing(P, x, state, v_first, H, length, layer_id, new_starts=None, es=None,
                math=MATH_F32, want_state=True, xm=None, x_last=None):
    """TimeMixing::forward (llm.rs:348-480) on every sequence.

    P maps the module's parameter names to device tensors: x_r..x_g, w0, v0,
    a0, k_k, k_a, r_k, ln_w, ln_b (C); receptance, key, value, output (C, C)
    Linear weights (out, in); w1, v1, a1, g1 (C, D) and w2, v2, a2, g2 (D, C)
    Tmm weights (in, out).  es optionally maps a matrix name to its EsLinear
    (the member's perturbation of that parameter).  x (nseq, T, C); state
    (nseq, 1 + S, C): row 0 the previous token, rows 1.. the (H, S, S) WKV
    state; v_first (nseq, T, C).  Returns (out, state, v_first), new tensors.  With
    xm (the six mixes, (6, nseq, T, C), as add_layer_norm_shift forms them) and,
    for want_state, x_last (x[:, length-1]) given, x may be None, and then state
    may be None for the zero state (no state returned)."""
    es = es or {}
    nseq, T, C = x.shape if xm is None else xm.shape[1:]
    S = C // H
    if S * H != C or S > 64:
        raise ValueError(f"C={C} is not H={H} heads of at most 64 channels")
    if (state is not None and state.shape != (nseq, 1 + S, C)) or v_first.shape != (nseq, T, C):
        raise ValueError("state must be (nseq, 1 + S, C) and v_first (nseq, T, C)")
    if not 1 <= length <= T:
        raise ValueError("length must be in [1, T]")
    bf = math == MATH_BF16  # bf16-only consumers get bf16 inputs (the same rounding)
    if xm is None:
        if x is None or state is None:
            raise ValueError("x and state are needed to form the mixes")
        mixes = torch.stack([P[n] for n in TM_MIXES])
        xm = token_shift_mix(x, state[:, 0, :].contiguous(), mixes, new_starts, bf16=bf)

    def lin(i, name):
        return linear(xm[i], P[name], es.get(name), math)

    def low(inp, n1, n2, act):
        h = linear_t(inp, P[n1], es.get(n1), math, act=act, out_bf16=bf)
        return linear_t(h, P[n2], es.get(n2), math)

    # the projections and the low-rank branches only read the mixes: they run
    # side by side (the write-bound narrow products overlap the wide ones)
    jobs = {"r": lambda: lin(0, "receptance"), "k": lambda: lin(2, "key"),
            "v": lambda: lin(3, "value"),
            "g": lambda: low(xm[5], "g1", "g2", ACT_SIGMOID),
            "w": lambda: low(xm[1], "w1", "w2", ACT_TANH),   # w2 output; the gate makes w
            "a": lambda: low(xm[4], "a1", "a2", ACT_TANH)}   # a2 output; the gate makes a
    if layer_id != 0:
        jobs["v2o"] = lambda: low(xm[3], "v1", "v2", ACT_TANH)
    res = _fan_out(jobs, xm)
    r, w, k, v, a, g = (res[n] for n in ("r", "w", "k", "v", "a", "g"))
    if layer_id == 0:
        v_first = v  # only read from here on
        v2o = None
    else:
        v2o = res["v2o"]
    # state None: the zero WKV state (the kernel starts from zeros, nothing is copied)
    s_in = None if state is None else state[:, 1:, :].reshape(nseq, H, S, S).contiguous()
    # the gates, the kk normalisation and k update, the recurrence, ln_x, the readout and
    # the gate in one kernel, from the raw projections
    gn = torch.empty(r.shape, dtype=torch.bfloat16 if bf else torch.float32, device=r.device)
    s_new = torch.empty((nseq, H, S, S), dtype=torch.float32, device=r.device) if want_state else None
    if new_starts is not None:
        K._dev(new_starts, torch.uint8, "new_starts")
    _lib.call("hses_tm_fused", _p(r), _p(w), _p(k), _p(v), _p(a), _p(v2o), _p(v_first),
              _p(P["w0"]), _p(P["a0"]), _p(P["v0"]), _p(P["k_k"]), _p(P["k_a"]), _p(s_in),
              _p(new_starts), nseq, T, H, S, length, _p(g), _p(P["ln_w"]), _p(P["ln_b"]), 64e-5,
              _p(P["r_k"]), _p(gn), FMT_BF16 if bf else FMT_F32, _p(s_new), _stream())
    state_out = None
    if want_state:
        if state is None:
            raise ValueError("want_state needs the incoming state")
        state_out = torch.empty_like(state)
        state_out[:, 0, :] = x[:, length - 1, :] if x_last is None else x_last
        state_out[:, 1:, :] = s_new.view(nseq, S, C)
    out = linear(gn.view(nseq, T, C), P["output"], es.get("output"), math)
    return out, state_out, v_first
