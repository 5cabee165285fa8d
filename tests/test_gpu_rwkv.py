"""GPU parity of the RWKV-7 components (llm.rs) against the oracle
(tests/test_oracle_rwkv.py pins it on the reference's hand-computed cases).

Norms and the token shift: elementwise order as the reference, reductions over
64-lane waves (rel 1e-5).  The WKV-7 recurrence: per-element order as the
reference and ascending-j sums, with the device's exp (rel 1e-4 of the output
scale over 32 steps).  ChannelMixing: fp32 MFMA linears (rel 1e-5)."""
import numpy as np
import pytest
import torch

from hyperscalees_amd import rwkv
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu


def cuda(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()


def close(got, ref, rel):
    ref = np.asarray(ref, np.float64)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    assert err <= rel * max(np.abs(ref).max(), 1e-30), f"max err {err:.3e} vs scale {np.abs(ref).max():.3e}"


@pytest.mark.parametrize("rows,C", [(2, 4), (37, 512), (5, 1000)])
def test_layer_norm(hses_gpu, rows, C):
    rng = np.random.default_rng(C)
    x = (rng.standard_normal((rows, C)) * 3 + 1).astype(np.float32)
    w, b = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    got = rwkv.layer_norm(cuda(x), cuda(w), cuda(b), 1e-5)
    torch.cuda.synchronize()
    close(got.cpu().numpy(), O.layer_norm(x, w, b, 1e-5), 1e-5)


@pytest.mark.parametrize("shape,G", [((2, 4, 2), 2), ((128, 512), 8), ((7, 96, 3), 4)])
def test_group_norm(hses_gpu, shape, G):
    rng = np.random.default_rng(G)
    x = (rng.standard_normal(shape) * 2 - 0.5).astype(np.float32)
    C = shape[1]
    w, b = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    got = rwkv.group_norm(cuda(x), G, cuda(w), cuda(b), 64e-5)
    torch.cuda.synchronize()
    close(got.cpu().numpy(), O.group_norm(x, G, w, b, 64e-5), 1e-5)


@pytest.mark.parametrize("C", [40, 38])   # four-channel vector path, scalar path
def test_token_shift_mix(hses_gpu, C):
    rng = np.random.default_rng(3)
    nseq, T, n_mix = 3, 9, 6
    x = rng.standard_normal((nseq, T, C)).astype(np.float32)
    st = rng.standard_normal((nseq, C)).astype(np.float32)
    mix = rng.random((n_mix, C)).astype(np.float32)
    ns = np.zeros((nseq, T), np.uint8)
    ns[1, 4] = 1
    got = rwkv.token_shift_mix(cuda(x), cuda(st), cuda(mix), cuda(ns, torch.uint8)).cpu().numpy()
    prev = np.concatenate([st[:, None, :], x[:, :-1, :]], 1)
    prev[ns.astype(bool)] = 0.0
    sx = prev - x
    ref = x[None] + sx[None] * mix[:, None, None, :]
    np.testing.assert_array_equal(got, ref.astype(np.float32))  # same elementwise ops
    got16 = rwkv.token_shift_mix(cuda(x), cuda(st), cuda(mix), cuda(ns, torch.uint8), bf16=True)
    assert torch.equal(got16, torch.from_numpy(ref.astype(np.float32)).cuda().to(torch.bfloat16))


@pytest.mark.parametrize("nseq,T,H,S,length", [(3, 32, 2, 64, 32), (2, 17, 3, 32, 9), (4, 5, 1, 16, 0)])
def test_wkv7_matches_oracle(hses_gpu, nseq, T, H, S, length):
    rng = np.random.default_rng(nseq * T + S)
    shp = (nseq, T, H, S)
    r = rng.standard_normal(shp).astype(np.float32)
    w = (rng.standard_normal(shp) * 0.5 - 0.6).astype(np.float32)   # decays 0.3 .. 0.9
    k = (rng.standard_normal(shp) * 0.3).astype(np.float32)
    v = rng.standard_normal(shp).astype(np.float32)
    kk = rng.standard_normal(shp).astype(np.float32)
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    a_ = (-kk).astype(np.float32)                                      # a = -kk, b = kk * gate
    b_ = (kk * rng.random(shp)).astype(np.float32)
    s0 = (rng.standard_normal((nseq, H, S, S)) * 0.1).astype(np.float32)
    ns = np.zeros((nseq, T), np.uint8)
    if T > 3:
        ns[0, 3] = 1
    out, s_out = rwkv.wkv7(*(cuda(t) for t in (r, w, k, v, a_, b_, s0)), length,
                           new_starts=cuda(ns, torch.uint8))
    torch.cuda.synchronize()
    out, s_out = out.cpu().numpy(), s_out.cpu().numpy()
    for q in range(nseq):
        ro, rs = O.rwkv7_inner_loop(r[q], w[q], k[q], v[q], a_[q], b_[q], s0[q], length, ns[q])
        close(out[q], ro, 1e-4)
        close(s_out[q], rs, 1e-4)


@pytest.mark.parametrize("nseq,T,C,F,length", [(2, 16, 64, 256, 16), (3, 7, 40, 96, 5)])
def test_channel_mixing_matches_oracle(hses_gpu, nseq, T, C, F, length):
    rng = np.random.default_rng(C + F)
    x = rng.standard_normal((nseq, T, C)).astype(np.float32)
    st = rng.standard_normal((nseq, C)).astype(np.float32)
    x_k = rng.random(C).astype(np.float32)
    Wk = (rng.standard_normal((F, C)) / np.sqrt(C)).astype(np.float32)
    Wv = (rng.standard_normal((C, F)) / np.sqrt(F)).astype(np.float32)
    ns = np.zeros((nseq, T), np.uint8)
    ns[-1, 2] = 1
    out, last = rwkv.channel_mixing(cuda(x), cuda(st), cuda(x_k), cuda(Wk), cuda(Wv), length,
                                    new_starts=cuda(ns, torch.uint8))
    torch.cuda.synchronize()
    out, last = out.cpu().numpy(), last.cpu().numpy()
    for q in range(nseq):
        ro, rl = O.channel_mixing(x[q], st[q], x_k, Wk, Wv, length, ns[q])
        close(out[q], ro, 1e-5)
        np.testing.assert_array_equal(last[q], rl)


def tm_params(rng, C, D):
    P = {}
    for n in O.TM_VECTORS + ("k_a",):
        P[n] = rng.random(C).astype(np.float32)
    for n in ("w0", "v0", "a0", "r_k", "ln_b"):
        P[n] = (rng.standard_normal(C) * 0.5).astype(np.float32)
    P["k_k"] = (1 + 0.2 * rng.standard_normal(C)).astype(np.float32)
    P["ln_w"] = (1 + 0.2 * rng.standard_normal(C)).astype(np.float32)
    for n in O.TM_LINEAR:
        P[n] = (rng.standard_normal((C, C)) / np.sqrt(C)).astype(np.float32)
    for n in ("w1", "v1", "a1", "g1"):
        P[n] = (rng.standard_normal((C, D)) / np.sqrt(C)).astype(np.float32)
    for n in ("w2", "v2", "a2", "g2"):
        P[n] = (rng.standard_normal((D, C)) / np.sqrt(D)).astype(np.float32)
    return P


@pytest.mark.parametrize("nseq,T,H,S,D,length,layer_id", [
    (2, 8, 2, 16, 8, 8, 0),
    (3, 7, 4, 32, 16, 5, 1),
    (2, 4, 2, 64, 32, 4, 2),
])
def test_time_mixing_matches_oracle(hses_gpu, nseq, T, H, S, D, length, layer_id):
    # fp32 linears, elementwise gates in the reference's order with the device's
    # exp/log/tanh, the recurrence's 1e-4 bound: rel 1e-4 of each output's scale.
    C = H * S
    rng = np.random.default_rng(C + T + layer_id)
    P = tm_params(rng, C, D)
    x = rng.standard_normal((nseq, T, C)).astype(np.float32)
    st = (rng.standard_normal((nseq, 1 + S, C)) * 0.3).astype(np.float32)
    vf = rng.standard_normal((nseq, T, C)).astype(np.float32)
    ns = np.zeros((nseq, T), np.uint8)
    ns[-1, T // 2] = 1
    Pd = {n: cuda(t) for n, t in P.items()}
    out, so, vfo = rwkv.time_mixing(Pd, cuda(x), cuda(st), cuda(vf), H, length, layer_id,
                                    new_starts=cuda(ns, torch.uint8))
    torch.cuda.synchronize()
    out, so, vfo = out.cpu().numpy(), so.cpu().numpy(), vfo.cpu().numpy()
    for q in range(nseq):
        ro, rs, rv = O.time_mixing(P, x[q], st[q], vf[q], H, length, layer_id, ns[q])
        close(out[q], ro, 1e-4)
        close(so[q, 1:], rs[1:], 1e-4)
        np.testing.assert_array_equal(so[q, 0], rs[0])
        if layer_id == 0:
            close(vfo[q], rv, 1e-5)
        else:
            np.testing.assert_array_equal(vfo[q], vf[q])


def test_time_mixing_perturbed_members(hses_gpu):
    # n = 2 members of 2 sequences each, perturbing the Linear `key` and `output`
    # and the Tmm `w1` and `g2`: member m's sequences equal the plain module with
    # W + A_m B_m^T (the do_mm / do_Tmm identity).
    n, spm, T, H, S, D, r, sigma = 2, 2, 5, 2, 32, 16, 2, 0.1
    C, nseq = H * S, n * spm
    rng = np.random.default_rng(11)
    P = tm_params(rng, C, D)
    x = rng.standard_normal((nseq, T, C)).astype(np.float32)
    st = (rng.standard_normal((nseq, 1 + S, C)) * 0.3).astype(np.float32)
    vf = np.zeros((nseq, T, C), np.float32)
    keys = {"key": 0x1234, "output": 0x5678, "w1": 0x9ABC, "g2": 0xDEF0}
    es = {name: rwkv.EsLinear(key=kk, rank=r, sigma=sigma, n=n, seqs_per_member=spm)
          for name, kk in keys.items()}
    Pd = {nm: cuda(t) for nm, t in P.items()}
    out, so, _ = rwkv.time_mixing(Pd, cuda(x), cuda(st), cuda(vf), H, T, 0, es=es)
    torch.cuda.synchronize()
    out, so = out.cpu().numpy(), so.cpu().numpy()
    bs = O.load().or_base_sigma(sigma, r)
    for m in range(n):
        Pm = dict(P)
        for name, kk in keys.items():
            a, b = P[name].shape
            A, B = O.lora_factors(bs, kk, r, 0, [m], a, b)
            Pm[name] = (P[name].astype(np.float64) + A[0].astype(np.float64) @ B[0].T).astype(np.float32)
        for q in range(m * spm, (m + 1) * spm):
            ro, rs, _ = O.time_mixing(Pm, x[q], st[q], vf[q], H, T, 0)
            close(out[q], ro, 1e-4)
            close(so[q, 1:], rs[1:], 1e-4)


def test_bf16_intermediates_are_exact(hses_gpu):
    # With bf16 math the forward rounds its input to bf16 (nearest even) before the
    # MFMAs, so a bf16 token-shift output and a bf16 linear output feed the next
    # product with exactly the values the fp32 path would: the results are equal.
    from hyperscalees_amd._lib import ACT_RELU_SQ, MATH_BF16
    rng = np.random.default_rng(21)
    nseq, T, C, F = 4, 128, 64, 256
    x = cuda(rng.standard_normal((nseq, T, C)))
    st = cuda(rng.standard_normal((nseq, C)))
    mixes = cuda(rng.random((6, C)))
    o32 = rwkv.token_shift_mix(x, st, mixes)
    o16 = rwkv.token_shift_mix(x, st, mixes, bf16=True)
    assert torch.equal(o32.to(torch.bfloat16), o16)
    W = cuda(rng.standard_normal((F, C)) / 8)
    es = rwkv.EsLinear(key=0x77, rank=1, sigma=0.1, n=nseq, seqs_per_member=1)
    y32 = rwkv.linear(o32[1], W, es, MATH_BF16, act=ACT_RELU_SQ)
    y16 = rwkv.linear(o16[1], W, es, MATH_BF16, act=ACT_RELU_SQ)
    assert torch.equal(y32, y16)
    yb = rwkv.linear(o16[1], W, es, MATH_BF16, act=ACT_RELU_SQ, out_bf16=True)
    assert torch.equal(y32.to(torch.bfloat16), yb)
    W2 = cuda(rng.standard_normal((C, F)) / 16)
    assert torch.equal(rwkv.linear(y32, W2, es, MATH_BF16), rwkv.linear(yb, W2, es, MATH_BF16))


@pytest.mark.parametrize("S", [64, 32, 16])
def test_fused_wkv_post_equals_chain(hses_gpu, S):
    # hses_tm_wkv_post == hses_rwkv7_wkv -> hses_group_norm(G = H) -> hses_tm_post, bit for bit
    from hyperscalees_amd import _lib, kernels as K
    nseq, T, H, length = 3, 9, 2, 7
    C = H * S
    rng = np.random.default_rng(S)
    shp = (nseq, T, H, S)
    r, k, v, g = (cuda(rng.standard_normal(shp)) for _ in range(4))
    w = cuda(rng.standard_normal(shp) * 0.5 - 0.6)
    kk = rng.standard_normal(shp)
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    a_, b_ = cuda(-kk), cuda(kk * rng.random(shp))
    s0 = cuda(rng.standard_normal((nseq, H, S, S)) * 0.1)
    ln_w, ln_b, r_k = (cuda(rng.standard_normal(C)) for _ in range(3))
    ns = np.zeros((nseq, T), np.uint8)
    ns[1, 4] = 1
    nsd = cuda(ns, torch.uint8)
    wkv, s_a = rwkv.wkv7(r, w, k, v, a_, b_, s0, length, new_starts=nsd)
    gn = rwkv.group_norm(wkv.view(nseq * T, C), H, ln_w, ln_b, 64e-5)
    _lib.call("hses_tm_post", K._p(gn), K._p(r), K._p(k), K._p(v), K._p(g), K._p(r_k), nseq * T,
              H, S, K._stream())
    out = torch.empty_like(r)
    s_b = torch.empty_like(s0)
    _lib.call("hses_tm_wkv_post", K._p(r), K._p(w), K._p(k), K._p(v), K._p(a_), K._p(b_), K._p(s0),
              K._p(nsd), nseq, T, H, S, length, K._p(g), K._p(ln_w), K._p(ln_b), 64e-5, K._p(r_k),
              K._p(out), 0, K._p(s_b), K._stream())
    out16 = torch.empty(r.shape, dtype=torch.bfloat16, device="cuda")
    s_c = torch.empty_like(s0)
    _lib.call("hses_tm_wkv_post", K._p(r), K._p(w), K._p(k), K._p(v), K._p(a_), K._p(b_), K._p(s0),
              K._p(nsd), nseq, T, H, S, length, K._p(g), K._p(ln_w), K._p(ln_b), 64e-5, K._p(r_k),
              K._p(out16), 1, K._p(s_c), K._stream())
    torch.cuda.synchronize()
    assert torch.equal(out.view(nseq * T, C), gn)
    assert torch.equal(s_a, s_b)
    assert torch.equal(out16, out.to(torch.bfloat16))


@pytest.mark.parametrize("S,with_v", [(64, True), (32, False)])
def test_gates_kk_equals_chain(hses_gpu, S, with_v):
    # hses_tm_gates_kk == hses_tm_gates -> hses_tm_kk, bit for bit
    from hyperscalees_amd import _lib, kernels as K
    rows, H = 37, 3
    C = H * S
    rng = np.random.default_rng(S + with_v)
    w2o, a2o, v2o, v, vf, k = (rng.standard_normal((rows, C)).astype(np.float32) for _ in range(6))
    w0, a0, v0, k_k, k_a = (rng.standard_normal(C).astype(np.float32) for _ in range(5))
    d = {n: cuda(x) for n, x in dict(w2o=w2o, a2o=a2o, v2o=v2o, v=v, vf=vf, k=k, w0=w0, a0=a0,
                                       v0=v0, k_k=k_k, k_a=k_a).items()}
    e = {n: t.clone() for n, t in d.items()}
    v2 = d["v2o"] if with_v else None
    ai1, bi1, ai2, bi2 = (torch.empty((rows, C), device="cuda") for _ in range(4))
    _lib.call("hses_tm_gates", K._p(d["w2o"]), K._p(d["a2o"]), K._p(v2), K._p(d["v"]), K._p(d["vf"]),
              K._p(d["w0"]), K._p(d["a0"]), K._p(d["v0"]), rows, C, K._stream())
    _lib.call("hses_tm_kk", K._p(d["k"]), K._p(d["k_k"]), K._p(d["k_a"]), K._p(d["a2o"]), rows, H, S,
              K._p(ai1), K._p(bi1), K._stream())
    v2e = e["v2o"] if with_v else None
    _lib.call("hses_tm_gates_kk", K._p(e["w2o"]), K._p(e["a2o"]), K._p(v2e), K._p(e["v"]),
              K._p(e["vf"]), K._p(e["w0"]), K._p(e["a0"]), K._p(e["v0"]), K._p(e["k"]),
              K._p(e["k_k"]), K._p(e["k_a"]), rows, H, S, K._p(ai2), K._p(bi2), K._stream())
    torch.cuda.synchronize()
    for n in ("w2o", "v", "k"):
        assert torch.equal(d[n], e[n]), n
    assert torch.equal(ai1, ai2) and torch.equal(bi1, bi2)


@pytest.mark.parametrize("C,n_mix,add,bf16", [(512, 6, True, True), (512, 1, True, True),
                                              (256, 6, False, False), (1024, 1, True, False),
                                              (512, 6, False, True)])
def test_add_ln_shift_equals_chain(hses_gpu, C, n_mix, add, bf16):
    # the fused residual add + LayerNorm + token shift == hses_add_layer_norm (a zero
    # delta without add) then hses_token_shift_mix, bit for bit, with new starts, a
    # carried state and the last normalised row at length < T
    from hyperscalees_amd import _lib, kernels as K
    from hyperscalees_amd._lib import FMT_BF16, FMT_F32
    nseq, T, length = 5, 37, 30
    rng = np.random.default_rng(C + n_mix + 2 * add)
    x = rng.standard_normal((nseq, T, C)).astype(np.float32) * 2 + 0.5
    dl = rng.standard_normal((nseq, T, C)).astype(np.float32)
    w, b = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    st = rng.standard_normal((nseq, C)).astype(np.float32)
    mix = rng.random((n_mix, C)).astype(np.float32)
    ns = np.zeros((nseq, T), np.uint8)
    ns[1, 0] = ns[2, 17] = 1
    fmt, dt = (FMT_BF16, torch.bfloat16) if bf16 else (FMT_F32, torch.float32)
    wd, bd, sd, md, nsd = cuda(w), cuda(b), cuda(st), cuda(mix), cuda(ns, torch.uint8)
    # the chain
    x1, d1 = cuda(x), cuda(dl if add else np.zeros_like(dl))
    y1 = torch.empty_like(x1)
    _lib.call("hses_add_layer_norm", K._p(x1), K._p(d1), nseq * T, C, K._p(wd), K._p(bd), 1e-5,
              K._p(y1), K._stream())
    o1 = torch.empty((n_mix, nseq, T, C), dtype=dt, device="cuda")
    _lib.call("hses_token_shift_mix", K._p(y1), K._p(sd), K._p(nsd), K._p(md), n_mix, nseq, T, C,
              K._p(o1), fmt, K._stream())
    # fused
    x2, d2 = cuda(x), cuda(dl)
    o2 = torch.empty((n_mix, nseq, T, C), dtype=dt, device="cuda")
    last = torch.empty((nseq, C), device="cuda")
    _lib.call("hses_add_ln_shift", K._p(x2), K._p(d2) if add else None, nseq, T, C, K._p(wd),
              K._p(bd), 1e-5, K._p(sd), K._p(nsd), K._p(md), n_mix, K._p(o2), fmt, K._p(last),
              length, K._stream())
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(last, y1[:, length - 1, :])
    assert torch.equal(x2, x1 if add else cuda(x))


@pytest.mark.parametrize("C", [512, 256, 40])   # vector paths and the scalar path
def test_add_layer_norm(hses_gpu, C):
    from hyperscalees_amd import _lib, kernels as K
    rows = 70
    rng = np.random.default_rng(C)
    x = rng.standard_normal((rows, C)).astype(np.float32) * 2 + 0.5
    dl = rng.standard_normal((rows, C)).astype(np.float32)
    w, b = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    xd, dd, y = cuda(x), cuda(dl), torch.empty((rows, C), device="cuda")
    wd, bd = cuda(w), cuda(b)   # held: a temporary's memory could be handed to the next tensor
    _lib.call("hses_add_layer_norm", K._p(xd), K._p(dd), rows, C, K._p(wd), K._p(bd), 1e-5,
              K._p(y), K._stream())
    torch.cuda.synchronize()
    s = x + dl
    np.testing.assert_array_equal(xd.cpu().numpy(), s)       # the residual, one fp32 add
    close(y.cpu().numpy(), O.layer_norm(s, w, b, 1e-5), 1e-5)


@pytest.mark.parametrize("S,with_v,bf", [(64, True, False), (32, False, False), (64, True, True)])
def test_tm_fused_equals_chain(hses_gpu, S, with_v, bf):
    # hses_tm_fused == hses_tm_gates_kk -> hses_tm_wkv_post, bit for bit
    from hyperscalees_amd import _lib, kernels as K
    nseq, T, H, length = 3, 9, 2, 7
    C = H * S
    rng = np.random.default_rng(S + 2 * with_v + bf)
    shp = (nseq, T, H, S)
    raw = {n: cuda(rng.standard_normal(shp)) for n in ("r", "w2o", "k", "v", "a2o", "v2o", "vf", "g")}
    par = {n: cuda(rng.standard_normal(C)) for n in ("w0", "a0", "v0", "k_k", "k_a", "ln_w", "ln_b", "r_k")}
    s0 = cuda(rng.standard_normal((nseq, H, S, S)) * 0.1)
    ns = np.zeros((nseq, T), np.uint8)
    ns[2, 3] = 1
    nsd = cuda(ns, torch.uint8)
    odt = torch.bfloat16 if bf else torch.float32
    c = {n: t.clone() for n, t in raw.items()}
    v2 = c["v2o"] if with_v else None
    ai, bi = torch.empty(shp, device="cuda"), torch.empty(shp, device="cuda")
    _lib.call("hses_tm_gates_kk", K._p(c["w2o"]), K._p(c["a2o"]), K._p(v2), K._p(c["v"]),
              K._p(c["vf"]), K._p(par["w0"]), K._p(par["a0"]), K._p(par["v0"]), K._p(c["k"]),
              K._p(par["k_k"]), K._p(par["k_a"]), nseq * T, H, S, K._p(ai), K._p(bi), K._stream())
    out1, s1 = torch.empty(shp, dtype=odt, device="cuda"), torch.empty_like(s0)
    _lib.call("hses_tm_wkv_post", K._p(c["r"]), K._p(c["w2o"]), K._p(c["k"]), K._p(c["v"]),
              K._p(ai), K._p(bi), K._p(s0), K._p(nsd), nseq, T, H, S, length, K._p(c["g"]),
              K._p(par["ln_w"]), K._p(par["ln_b"]), 64e-5, K._p(par["r_k"]), K._p(out1), int(bf),
              K._p(s1), K._stream())
    f = {n: t.clone() for n, t in raw.items()}
    v2f = f["v2o"] if with_v else None
    out2, s2 = torch.empty(shp, dtype=odt, device="cuda"), torch.empty_like(s0)
    _lib.call("hses_tm_fused", K._p(f["r"]), K._p(f["w2o"]), K._p(f["k"]), K._p(f["v"]),
              K._p(f["a2o"]), K._p(v2f), K._p(f["vf"] if with_v else None), K._p(par["w0"]),
              K._p(par["a0"]), K._p(par["v0"]), K._p(par["k_k"]), K._p(par["k_a"]), K._p(s0),
              K._p(nsd), nseq, T, H, S, length, K._p(f["g"]), K._p(par["ln_w"]), K._p(par["ln_b"]),
              64e-5, K._p(par["r_k"]), K._p(out2), int(bf), K._p(s2), K._stream())
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(s1, s2)
    for n in raw:   # the fused kernel only reads its inputs
        assert torch.equal(f[n], raw[n]), n
