"""GPU parity of the spiking self-attention transformer (C4) against the oracle.

Stage kernels (encoder LIF rates, the row_softmax_lif attention, the ffn gate,
pooling) are bit-exact against the oracle's functions on the same inputs: they
use the same f32 operations in the same order.  The whole population forward
is checked stage by stage on the GPU's own stage inputs, member by member: the
perturbed projections (this noiser's factors, every leaf with its own key)
within fp32 rel 1e-5, every spiking stage bit for bit, so a rounding-level
difference of a projection cannot cascade through the thresholds.  At the full
C4 size (N = 1024, r = 8) sampled members go through the same checks, and the
ES gradients of an MM leaf and of a Parameter leaf are compared with the
oracle's double-accumulated sums.
"""
import math

import numpy as np
import pytest
import torch

from hyperscalees_amd import _lib
from hyperscalees_amd import kernels as K
from hyperscalees_amd import snn_attention as sa
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def test_softplus_matches_oracle(hses_gpu):
    x = np.concatenate([np.linspace(-40, 40, 4001), [0.0, -1e-8, 1e-8]]).astype(np.float32)
    y = torch.empty(x.size, dtype=torch.float32, device="cuda")
    xd = dev(x)
    _lib.call("hses_softplus", K._p(xd), x.size, K._p(y), K._stream())
    got = y.cpu().numpy()
    ref = np.array([O.load().or_sa_softplus(float(v)) for v in x], np.float32)
    ulp = np.spacing(np.abs(ref))
    assert np.all(np.abs(got - ref) <= 2 * ulp)


def test_encode_stage_bit_exact(hses_gpu):
    rng = np.random.default_rng(1)
    n, R, d, T = 3, 64, 64, 8
    M = n * R
    cur = [rng.normal(0.4, 0.4, (T, M, d)).astype(np.float32) for _ in range(3)]
    th = [rng.uniform(0.03, 0.08, n).astype(np.float32) for _ in range(3)]
    pos = rng.standard_normal((n, R, d)).astype(np.float32)
    X = torch.empty((M, d), dtype=torch.float32, device="cuda")
    cd = [dev(c) for c in cur]
    thd = [dev(t) for t in th]
    posd = dev(pos)
    _lib.call("hses_sa_encode", K._p(cd[0]), K._p(cd[1]), K._p(cd[2]), T, M, d, R, K._p(thd[0]),
              K._p(thd[1]), K._p(thd[2]), 20.0, K._p(posd), 1, K._p(X), K._stream())
    torch.cuda.synchronize()
    got = X.cpu().numpy()
    for m in range(n):
        rows = slice(m * R, (m + 1) * R)
        ref = np.zeros((R, d), np.float32)
        O.load().or_sa_encode(*[np.ascontiguousarray(c[:, rows]) for c in cur], T, R, d,
                              float(th[0][m]), float(th[1][m]), float(th[2][m]), 20.0,
                              np.ascontiguousarray(pos[m]), ref)
        np.testing.assert_array_equal(got[rows], ref, err_msg=f"member {m}")
    assert 0.05 < (got - pos.reshape(M, d)).mean() < 0.95   # rates neither all 0 nor all 1


@pytest.mark.parametrize("R,H,hd", [(64, 4, 16), (50, 2, 24), (7, 3, 5)])
def test_attention_stage_bit_exact(hses_gpu, R, H, hd):
    rng = np.random.default_rng(R + H)
    n, d = 3, H * hd + 3           # a row stride wider than the heads
    M = n * R
    Q, Kk, V = (rng.uniform(0, 1, (M, d)).astype(np.float32) for _ in range(3))
    beta = rng.uniform(0.2, 0.3, n).astype(np.float32)
    vth = rng.uniform(0.03, 0.08, n).astype(np.float32)
    out = torch.zeros((M, d), dtype=torch.float32, device="cuda")
    keep = [dev(a) for a in (Q, Kk, V, beta, vth)]   # alive until the kernel has run
    _lib.call("hses_sa_attention", K._p(keep[0]), K._p(keep[1]), K._p(keep[2]), d, n, R, H, hd,
              K._p(keep[3]), K._p(keep[4]), 0.5, 20.0, 8, K._p(out), K._stream())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for m in range(n):
        for h in range(H):
            rows = slice(m * R, (m + 1) * R)
            q = np.ascontiguousarray(Q[rows])
            k = np.ascontiguousarray(Kk[rows])
            v = np.ascontiguousarray(V[rows])
            ref = np.zeros((R, d), np.float32)
            off = 4 * h * hd
            O.load().or_sa_attention_head(q.ctypes.data + off, k.ctypes.data + off,
                                          v.ctypes.data + off, R, hd, d, float(beta[m]),
                                          float(vth[m]), 0.5, 20.0, 8, ref.ctypes.data + off)
            np.testing.assert_array_equal(got[rows, h * hd:(h + 1) * hd],
                                          ref[:, h * hd:(h + 1) * hd], err_msg=f"m{m} h{h}")
    assert got[:, :H * hd].any()


def test_ffn_gate_pool_and_row_scale_bit_exact(hses_gpu):
    rng = np.random.default_rng(5)
    n, R, d = 4, 64, 96
    M = n * R
    c = rng.standard_normal((M, d)).astype(np.float32)
    c[3] = 0.0                                     # an all-zero row
    vth = rng.uniform(0.2, 0.6, n).astype(np.float32)
    act = torch.empty((M, d), dtype=torch.float32, device="cuda")
    cd, vthd = dev(c), dev(vth)
    _lib.call("hses_sa_ffn_spike", K._p(cd), M, d, R, K._p(vthd), K._p(act), K._stream())
    pooled = torch.empty((n, d), dtype=torch.float32, device="cuda")
    _lib.call("hses_sa_pool", K._p(cd), n, R, d, K._p(pooled), K._stream())
    y = dev(c[:n, :10])
    g = rng.uniform(0.5, 2, n).astype(np.float32)
    gd = dev(g)
    _lib.call("hses_scale_rows", K._p(y), n, 10, K._p(gd), K._stream())
    torch.cuda.synchronize()
    for m in range(n):
        ref = np.zeros((R, d), np.float32)
        O.load().or_sa_ffn_spike(np.ascontiguousarray(c[m * R:(m + 1) * R]), R, d, float(vth[m]), ref)
        np.testing.assert_array_equal(act.cpu().numpy()[m * R:(m + 1) * R], ref)
        s = np.zeros(d, np.float32)
        for i in range(R):
            s = s + c[m * R + i]
        np.testing.assert_array_equal(pooled.cpu().numpy()[m], s / np.float32(R))
    np.testing.assert_array_equal(y.cpu().numpy(), c[:n, :10] * g[:, None])


# -- the whole forward, stage by stage ---------------------------------------

def mm_member(x, W, key, cfg, m, epoch=0):
    """do_mm of member m: x (rows, b) -> (rows, a), oracle factors, float32."""
    a, b = W.shape
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    A, B = O.lora_factors(bs, key, cfg.rank, epoch, [m], a, b, noise_reuse=cfg.noise_reuse)
    return O.do_mm(np.ascontiguousarray(x, np.float32), W, A[0], B[0])


def close(got, ref, rel, what):
    err = np.abs(got.astype(np.float64) - ref).max()
    scale = max(np.abs(ref).max(), 1e-30)
    assert err <= rel * scale, f"{what}: err {err:.3e} vs scale {scale:.3e}"


def check_stages(es, tr, members, epoch=0):
    c = es.cfg
    R, d, hd, T = c.ntok, c.d_model, c.head_dim, c.T
    P = {k: v.cpu().numpy() for k, v in es.P.items()}
    th = {k: v.cpu().numpy() for k, v in es.th.items()}
    pos = es.noisy["pos_emb"].cpu().numpy()
    gain = es.noisy["out_gain"].cpu().numpy().ravel()
    t = {k: v.cpu().numpy() for k, v in tr.items()}
    L = O.load()
    for m in members:
        rows = slice(m * R, (m + 1) * R)
        # thresholds and beta: softplus of the member's perturbed raw leaves
        for name in th:
            raw = float(es.noisy[name].cpu().numpy().ravel()[m])
            ref = np.float32(L.or_sa_softplus(raw))
            assert abs(th[name][m] - ref) <= 2 * np.spacing(abs(ref)), (name, m)
        x = t["spk"][:, rows]
        for i, (q, name) in enumerate((("q", "in_q"), ("k", "in_k"), ("v", "in_v"))):
            ref = mm_member(x.reshape(-1, c.tin), P[name], es.keys[name], c, m, epoch)
            close(t[f"cur_{q}"][:, rows].reshape(-1, d), ref, 1e-5, f"m{m} {name}")
        Xe = np.zeros((R, d), np.float32)
        L.or_sa_encode(*[np.ascontiguousarray(t[f"cur_{q}"][:, rows]) for q in "qkv"], T, R, d,
                       float(th["q_th"][m]), float(th["k_th"][m]), float(th["v_th"][m]), c.tau_m,
                       np.ascontiguousarray(pos[m]), Xe)
        np.testing.assert_array_equal(t["x_enc"][rows], Xe, err_msg=f"m{m} encode")
        for b in range(c.blocks):
            Xb = t[f"b{b}_in"][rows]
            for kind in "qkv":
                for h in range(c.heads):
                    nm = f"b{b}_{kind}{h}"
                    ref = mm_member(Xb, P[nm], es.keys[nm], c, m, epoch)
                    close(t[f"b{b}_{kind}"][rows, h * hd:(h + 1) * hd], ref, 1e-5, f"m{m} {nm}")
            q, k, v = (np.ascontiguousarray(t[f"b{b}_{kind}"][rows]) for kind in "qkv")
            att = np.zeros((R, d), np.float32)
            for h in range(c.heads):
                off = 4 * h * hd
                L.or_sa_attention_head(q.ctypes.data + off, k.ctypes.data + off, v.ctypes.data + off,
                                       R, hd, d, float(th["beta"][m]), float(th["attn_th"][m]),
                                       c.g_inh, c.tau_m, c.n_iter, att.ctypes.data + off)
            np.testing.assert_array_equal(t[f"b{b}_att"][rows], att, err_msg=f"m{m} b{b} attention")
            ref = Xb + mm_member(att, P[f"b{b}_o"], es.keys[f"b{b}_o"], c, m, epoch)
            close(t[f"b{b}_x_att"][rows], ref, 1e-5, f"m{m} b{b} attention residual")
            xa = t[f"b{b}_x_att"][rows]
            ref = mm_member(xa, P[f"b{b}_ff1"], es.keys[f"b{b}_ff1"], c, m, epoch)
            close(t[f"b{b}_ff1"][rows], ref, 1e-5, f"m{m} b{b} ff1")
            act = np.zeros((R, d), np.float32)
            L.or_sa_ffn_spike(np.ascontiguousarray(t[f"b{b}_ff1"][rows]), R, d,
                              float(th[f"b{b}_ff_th"][m]), act)
            np.testing.assert_array_equal(t[f"b{b}_act"][rows], act, err_msg=f"m{m} b{b} gate")
            nxt = t[f"b{b + 1}_in"][rows] if b + 1 < c.blocks else t["x_out"][rows]
            ref = xa + mm_member(act, P[f"b{b}_ff2"], es.keys[f"b{b}_ff2"], c, m, epoch)
            close(nxt, ref, 1e-5, f"m{m} b{b} ffn residual")
        s = np.zeros(d, np.float32)
        for i in range(R):
            s = s + t["x_out"][m * R + i]
        np.testing.assert_array_equal(t["pooled"][m], s / np.float32(R), err_msg=f"m{m} pool")
        ref = mm_member(t["pooled"][m:m + 1], P["out"], es.keys["out"], c, m, epoch)[0] * gain[m]
        close(t["logits"][m], ref, 1e-5, f"m{m} readout")


def make_es(cfg, seed=0):
    P = sa.init_params(cfg, seed)
    vocab = sa.synthetic_vocab(cfg, seed)
    es = sa.SpikingAttentionEs(cfg, P, vocab)
    rng = np.random.default_rng(seed + 7)
    tok = torch.from_numpy(rng.integers(0, cfg.vocab, (cfg.n, cfg.ntok)).astype(np.int32)).cuda()
    lab = torch.from_numpy(rng.integers(0, cfg.classes, cfg.n).astype(np.int32)).cuda()
    return es, P, vocab, tok, lab


def test_forward_stages_small_population(hses_gpu):
    cfg = sa.SaConfig(n=6)
    es, P, vocab, tok, lab = make_es(cfg, seed=1)
    tr = {}
    fit = es.forward(tok, lab, epoch=0, trace=tr)
    torch.cuda.synchronize()
    # input spikes: the Poisson encode of each token's intensity vector
    ref = O.poisson(vocab[tok.cpu().numpy().ravel()], cfg.T, cfg.poisson_seed)
    np.testing.assert_array_equal(tr["spk"].cpu().numpy(), ref)
    check_stages(es, tr, range(cfg.n))
    # fitness: the log-likelihood of each member's label
    lg = tr["logits"].cpu().numpy().astype(np.float64)
    ll = lg - lg.max(1, keepdims=True)
    ll = ll - np.log(np.exp(ll).sum(1, keepdims=True))
    ref = ll[np.arange(cfg.n), lab.cpu().numpy()]
    np.testing.assert_allclose(fit.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    # the layers are active: encoder rates, attention weights and ffn gates
    x_enc = tr["x_enc"].cpu().numpy() - es.noisy["pos_emb"].cpu().numpy().reshape(-1, cfg.d_model)
    assert 0.02 < x_enc.mean() < 0.98
    assert tr["b0_att"].abs().sum() > 0 and 0.01 < float(tr["b1_act"].mean()) < 0.99


def test_member_forward_end_to_end(hses_gpu):
    # each member against the oracle's whole forward on its materialised
    # parameters; thresholds may flip on rounding-level differences, so the
    # bar is on the median member, and flips are reported
    cfg = sa.SaConfig(n=6)
    es, P, vocab, tok, lab = make_es(cfg, seed=2)
    tr = {}
    es.forward(tok, lab, epoch=0, trace=tr)
    torch.cuda.synchronize()
    spk = tr["spk"].cpu().numpy()
    lg = tr["logits"].cpu().numpy()
    rels = []
    for m in range(cfg.n):
        Pm = O.sa_member_params(P, es.keys, es.leaves, cfg.sigma, cfg.rank, m)
        ref = O.sa_forward_member(cfg, Pm, spk[:, m * cfg.ntok:(m + 1) * cfg.ntok])
        rels.append(np.abs(lg[m] - ref).max() / np.abs(ref).max())
    print("end-to-end logits rel differences:", ["%.1e" % r for r in rels])
    assert np.median(rels) <= 1e-4


def test_full_size_sampled_members_and_gradients(hses_gpu):
    cfg = sa.SaConfig()          # C4: N = 1024, r = 8, d 64, 4 heads, 2 blocks, 64 tokens
    es, P, vocab, tok, lab = make_es(cfg, seed=3)
    tr = {}
    fit = es.forward(tok, lab, epoch=0, trace=tr)
    torch.cuda.synchronize()
    check_stages(es, tr, (0, 1, 511, 1022, 1023))
    fit_h = fit.cpu().numpy()
    es.update(fit, 0)
    torch.cuda.synchronize()
    z, _, _ = O.convert_fitnesses(fit_h)
    name = "b1_k2"                                   # an MM leaf
    a, b = P[name].shape
    g = O.lora_grad_f64(cfg.sigma, es.keys[name], cfg.rank, 0, z, a, b, nthreads=16)
    close(es.grads[name].cpu().numpy(), g, 1e-5, name)
    # a Parameter leaf: (1/N) sum f_m noise_m, returned as -g sqrt(N)
    name = "attn_th"
    acc = 0.0
    for m in range(cfg.n):
        nz = np.zeros(1, np.float32)
        O.load().or_get_nonlora_update_params(cfg.sigma, es.keys[name], 0, m, 1, 1, 0, nz)
        acc += float(nz[0] * np.float32(z[m]))
    ref = acc * (-math.sqrt(cfg.n) / cfg.n)
    assert abs(float(es.grads[name].cpu()) - ref) <= 1e-5 * abs(ref)
