"""GPU parity of the RWKV-7 LM ES step (hyperscalees_amd.rwkv_lm) against the
oracle's LM forward (rwkv7.py:189-253; pinned in tests/test_oracle_rwkv.py) on
each member's materialised parameters W + A_m B_m^T, the log-likelihood
fitness, and the ES gradient and SGD step of every MM parameter.

fp32 linears: rel 1e-4 of the logits' scale through two blocks (the WKV-7
recurrence's bound); bf16 linears (the C5 precision): rel 2e-2."""
import numpy as np
import pytest
import torch

from hyperscalees_amd import rwkv_lm
from hyperscalees_amd._lib import ADAM, ADAMW, MATH_BF16, MATH_F32, SGD
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu

SMALL = dict(n_layer=2, d_model=64, head_size=32, vocab=50, ffn_mult=4, seq_len=8, n=4, rank=1,
             sigma=0.05, math=MATH_F32, solver=SGD, lr=0.1, init_std=0.2, widths=(16, 8, 16, 32))


def member_params(params, es, m, epoch=0):
    """The oracle's parameter dict of member m: W + A_m B_m^T for every MM parameter."""
    c = es.cfg
    bs = O.load().or_base_sigma(c.sigma, c.rank)
    P = {k: v for k, v in params.items() if k != "blocks"}
    P["blocks"] = []
    for l, B in enumerate(params["blocks"]):
        Bm = dict(B)
        for name in rwkv_lm.TM_MATRICES + rwkv_lm.FFN_MATRICES:
            a, b = B[name].shape
            A, Bf = O.lora_factors(bs, es.keys[(l, name)], c.rank, epoch, [m], a, b,
                                   noise_reuse=c.noise_reuse)
            Bm[name] = (B[name].astype(np.float64) + A[0].astype(np.float64) @ Bf[0].T.astype(np.float64)).astype(np.float32)
        P["blocks"].append(Bm)
    return P


def close(got, ref, rel):
    ref = np.asarray(ref, np.float64)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    assert err <= rel * np.abs(ref).max(), f"max err {err:.3e} vs scale {np.abs(ref).max():.3e}"


def log_softmax(z):
    z = z.astype(np.float64)
    m = z.max(-1, keepdims=True)
    return z - m - np.log(np.exp(z - m).sum(-1, keepdims=True))


@pytest.mark.parametrize("math,spm,rel", [(MATH_F32, 1, 1e-4), (MATH_F32, 2, 1e-4),
                                          (MATH_BF16, 1, 2e-2)])
def test_lm_members_match_oracle(hses_gpu, math, spm, rel):
    cfg = rwkv_lm.RwkvLmConfig(**dict(SMALL, math=math, seqs_per_member=spm))
    params = rwkv_lm.init_params(cfg, seed=3)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    H = cfg.d_model // cfg.head_size
    rng = np.random.default_rng(4)
    nseq, T = cfg.n * spm, cfg.seq_len
    tok = rng.integers(0, cfg.vocab, (nseq, T + 1)).astype(np.int32)
    tok_d = torch.from_numpy(tok).cuda()
    lg = es.logits(tok_d[:, :-1].contiguous()).cpu().numpy().reshape(nseq, T, cfg.vocab)
    fit = es.forward(tok_d).cpu().numpy()
    torch.cuda.synchronize()
    for m in range(cfg.n):
        Pm = member_params(params, es, m)
        lls = []
        for q in range(m * spm, (m + 1) * spm):
            ref, _ = O.rwkv_lm_forward(Pm, tok[q, :-1], H)
            close(lg[q], ref, rel)
            lls.append(log_softmax(ref)[np.arange(T), tok[q, 1:]])
        np.testing.assert_allclose(fit[m], np.mean(lls), rtol=10 * rel, atol=10 * rel)


def test_lm_plain_forward_matches_oracle(hses_gpu):
    cfg = rwkv_lm.RwkvLmConfig(**dict(SMALL, n_layer=3, n=3))
    params = rwkv_lm.init_params(cfg, seed=5)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    rng = np.random.default_rng(6)
    tok = rng.integers(0, cfg.vocab, (3, 11)).astype(np.int32)     # T != seq_len
    lg = es.logits(torch.from_numpy(tok).cuda(), perturb=False).cpu().numpy().reshape(3, 11, -1)
    for q in range(3):
        ref, _ = O.rwkv_lm_forward(params, tok[q], cfg.d_model // cfg.head_size)
        close(lg[q], ref, 1e-4)


def test_lm_es_step_gradients_and_sgd(hses_gpu):
    cfg = rwkv_lm.RwkvLmConfig(**dict(SMALL, n=6))
    params = rwkv_lm.init_params(cfg, seed=7)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    rng = np.random.default_rng(8)
    tok = torch.from_numpy(rng.integers(0, cfg.vocab, (cfg.n, cfg.seq_len + 1)).astype(np.int32)).cuda()
    before = {ln: es.blocks[ln[0]][ln[1]].cpu().numpy().copy() for ln in es.keys}
    vec_before = es.blocks[1]["x_r"].cpu().numpy().copy()
    fit = es.step(tok, epoch=0)
    torch.cuda.synchronize()
    z, _, _ = O.convert_fitnesses(fit.cpu().numpy())
    for (l, name), key in es.keys.items():
        a, b = before[(l, name)].shape
        g = O.lora_grad_f64(cfg.sigma, key, cfg.rank, 0, z, a, b)
        g_gpu = es.grads[(l, name)].cpu().numpy()
        assert np.abs(g_gpu - g).max() <= 1e-5 * np.abs(g).max(), (l, name)
        p_ref = before[(l, name)] - g * np.float32(cfg.lr)
        ulp = np.spacing(np.abs(p_ref).astype(np.float32))
        tol = 2 * ulp + 1e-5 * np.abs(g).max() * cfg.lr
        assert np.all(np.abs(es.blocks[l][name].cpu().numpy() - p_ref) <= tol), (l, name)
    # full-rank vectors are frozen (freeze_nonlora)
    np.testing.assert_array_equal(es.blocks[1]["x_r"].cpu().numpy(), vec_before)


@pytest.mark.parametrize("solver", [ADAM, ADAMW])
def test_lm_es_step_adam(hses_gpu, solver):
    # Adam / AdamW on every MM parameter: the moments start at zero and the
    # step follows Solver::update (noiser.rs:166-214) on the step's own
    # gradient; a second step checks that the moments carry over.
    cfg = rwkv_lm.RwkvLmConfig(**dict(SMALL, n=6, solver=solver, lr=0.01))
    params = rwkv_lm.init_params(cfg, seed=9)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    rng = np.random.default_rng(10)
    tok = torch.from_numpy(rng.integers(0, cfg.vocab, (cfg.n, cfg.seq_len + 1)).astype(np.int32)).cuda()
    p = {ln: es.blocks[ln[0]][ln[1]].cpu().numpy().copy() for ln in es.keys}
    m = {ln: np.zeros_like(v) for ln, v in p.items()}
    v = {ln: np.zeros_like(x) for ln, x in p.items()}
    wd = cfg.weight_decay if solver == ADAMW else 0.0
    for t in (1, 2):
        es.step(tok, epoch=t)
        torch.cuda.synchronize()
        for ln in es.keys:
            g = es.grads[ln].cpu().numpy()
            out = np.zeros_like(p[ln])
            O.load().or_solver_step(solver, cfg.lr, cfg.beta1, cfg.beta2, cfg.eps, wd, t,
                                    p[ln].ravel(), g.ravel(), m[ln].reshape(-1), v[ln].reshape(-1),
                                    p[ln].size, out.reshape(-1))
            got = es.blocks[ln[0]][ln[1]].cpu().numpy()
            # a few ulps of the lr-sized Adam step (p + step may cancel to near zero)
            np.testing.assert_allclose(got, out, rtol=1e-6, atol=1e-6 * cfg.lr, err_msg=str(ln))
            p[ln] = got.copy()


def test_embed_layer_norm_out_of_range_token_gives_nan(hses_gpu):
    from hyperscalees_amd import _lib, kernels as K
    C, V = 64, 10
    emb = torch.randn(V, C, device="cuda")
    w = torch.ones(C, device="cuda")
    b = torch.zeros(C, device="cuda")
    tok = torch.tensor([0, 9, 10, -1, 3], dtype=torch.int32, device="cuda")
    y = torch.empty(5, C, device="cuda")
    _lib.call("hses_embed_layer_norm", K._p(tok), 5, K._p(emb), V, C, K._p(w), K._p(b), 1e-5,
              K._p(y), K._stream())
    y = y.cpu().numpy()
    assert np.isfinite(y[[0, 1, 4]]).all() and np.isnan(y[[2, 3]]).all()
    ref = O.layer_norm(emb.cpu().numpy()[[0, 9, 3]], np.ones(C), np.zeros(C))
    close(y[[0, 1, 4]], ref, 1e-5)


def test_lm_full_width_state_carry_is_exact(hses_gpu):
    # The C5 model at full width and depth (4 layers, d=512, 8 heads of 64, FFN 2048, bf16
    # products, r=1 perturbed members): the LM is recurrent and every kernel computes a
    # token's row independently of the others, so running 128 tokens equals running 64 and
    # then 64 from the carried state, bit for bit (logits and final state).
    cfg = rwkv_lm.RwkvLmConfig(n=64)
    params = rwkv_lm.init_params(cfg, seed=11)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    S, C = cfg.head_size, cfg.d_model
    rng = np.random.default_rng(12)
    tok = torch.from_numpy(rng.integers(0, cfg.vocab, (cfg.n, 128)).astype(np.int32)).cuda()
    st0 = torch.zeros((cfg.n_layer, cfg.n, 2 + S, C), device="cuda")
    full, st_full = es.logits(tok, epoch=3, state=st0)
    a, st_a = es.logits(tok[:, :64].contiguous(), epoch=3, state=st0)
    b, st_b = es.logits(tok[:, 64:].contiguous(), epoch=3, state=st_a)
    torch.cuda.synchronize()
    V = cfg.vocab
    joined = torch.cat([a.view(cfg.n, 64, V), b.view(cfg.n, 64, V)], dim=1)
    assert torch.equal(full.view(cfg.n, 128, V), joined)
    assert torch.equal(st_full, st_b)
    assert torch.isfinite(full).all()


def test_lm_full_size_members_match_oracle(hses_gpu):
    # C5 at its full size (N = 2048 members, 4 layers, d = 512, 128 tokens,
    # bf16 products): sampled members' logits against the oracle LM on their
    # materialised parameters, at the bf16 bar.
    cfg = rwkv_lm.RwkvLmConfig()
    params = rwkv_lm.init_params(cfg, seed=13)
    es = rwkv_lm.RwkvLmEs(cfg, params)
    H = cfg.d_model // cfg.head_size
    rng = np.random.default_rng(14)
    T = cfg.seq_len
    tok = rng.integers(0, cfg.vocab, (cfg.n, T)).astype(np.int32)
    lg = es.logits(torch.from_numpy(tok).cuda(), epoch=2)
    torch.cuda.synchronize()
    for m in (0, 1, 1023, 2047):
        got = lg[m * T:(m + 1) * T].cpu().numpy()
        Pm = member_params(params, es, m, epoch=2)
        ref, _ = O.rwkv_lm_forward(Pm, tok[m], H)
        close(got, ref, 2e-2)
