"""Pins of the oracle's RWKV-7 components (llm.rs) against the reference's own
hand-computed tests (llm.rs:931-1097) and against what the mathematics fixes."""
import numpy as np

from tests import oracle_lib as O

TOL = 1e-4  # the reference tests' tolerance (llm.rs:925)


def test_layer_norm_hand_computed():
    # llm.rs:931-953
    x = np.array([[1, 2, 3, 4], [10, 20, 30, 40]], np.float32)
    w = np.array([2, 1, 0.5, 1], np.float32)
    b = np.array([1, 0, 0.5, -1], np.float32)
    exp = [-1.6832, -0.4472, 0.7236, 0.3416] * 2
    np.testing.assert_allclose(O.layer_norm(x, w, b, 1e-5).ravel(), exp, atol=TOL)


def test_group_norm_hand_computed():
    # llm.rs:973-1003: (2, 4, 2), 2 groups of 2 channels x 2 positions
    x = np.arange(1, 17, dtype=np.float32).reshape(2, 4, 2)
    out = O.group_norm(x, 2, np.ones(4, np.float32), np.zeros(4, np.float32), 1e-5)
    np.testing.assert_allclose(out.ravel(), [-1.34164, -0.44721, 0.44721, 1.34164] * 4, atol=TOL)


def test_group_norm_rank2_is_layer_norm_per_group():
    # rank-2 GroupNorm with G groups == layer norm of each group's C/G channels
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 12)).astype(np.float32) * 3 + 1
    w, b = rng.standard_normal(12).astype(np.float32), rng.standard_normal(12).astype(np.float32)
    gn = O.group_norm(x, 3, w, b, 64e-5)
    for g in range(3):
        sl = slice(4 * g, 4 * g + 4)
        np.testing.assert_allclose(gn[:, sl], O.layer_norm(x[:, sl], w[sl], b[sl], 64e-5),
                                   rtol=1e-6, atol=1e-6)


def test_channel_mixing_hand_computed():
    # llm.rs:1005-1039: T=2, C=1, identity key/value
    out, last = O.channel_mixing(np.array([[3.0], [5.0]]), np.array([1.0]), np.array([2.0]),
                                 np.array([[1.0]]), np.array([[1.0]]), 2)
    np.testing.assert_allclose(out.ravel(), [0.0, 1.0], atol=TOL)
    assert last[0] == 5.0


def test_channel_mixing_new_start_zeroes_the_shift():
    # a new start at t replaces the shifted row by 0: sx = -x there
    x = np.array([[3.0], [5.0]], np.float32)
    out, _ = O.channel_mixing(x, np.array([1.0]), np.array([2.0]), np.array([[1.0]]),
                              np.array([[1.0]]), 2, new_starts=[False, True])
    # t=1: xk = 5 + (0 - 5) * 2 = -5 -> relu^2 = 0
    np.testing.assert_allclose(out.ravel(), [0.0, 0.0], atol=TOL)


def test_rwkv7_inner_loop_hand_computed():
    # llm.rs:1041-1097: pure decay 0.5 per step (k = v = a = b = 0)
    s0 = np.array([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], np.float32)
    r = np.array([[[1, 0], [0, 1]], [[1, 1], [1, 1]]], np.float32)
    z = np.zeros((2, 2, 2), np.float32)
    w = np.full((2, 2, 2), np.log(np.log(2.0)), np.float32)
    out, out_s = O.rwkv7_inner_loop(r, w, z, z, z, z, s0, 2)
    np.testing.assert_allclose(out.ravel(), [0.5, 1.5, 3.0, 4.0, 0.75, 1.75, 2.75, 3.75], atol=TOL)
    np.testing.assert_allclose(out_s.ravel(), (s0 * 0.25).ravel(), atol=TOL)


def test_rwkv7_inner_loop_rank_one_updates_and_resets():
    # With w -> decay 0 (w large), a = b = 0: the state after step t is exactly
    # v_t k_t^T, so out[t] = v_t (k_t . r_t); a new start discards s0; and
    # length selects which step's state is returned.
    rng = np.random.default_rng(1)
    T, H, S = 3, 2, 4
    r, k, v = (rng.standard_normal((T, H, S)).astype(np.float32) for _ in range(3))
    z = np.zeros((T, H, S), np.float32)
    w = np.full((T, H, S), 10.0, np.float32)  # exp(-exp(10)) == 0 in f32
    s0 = rng.standard_normal((H, S, S)).astype(np.float32)
    out, out_s = O.rwkv7_inner_loop(r, w, k, v, z, z, s0, 2, new_starts=[True, False, False])
    for t in range(T):
        np.testing.assert_allclose(out[t], v[t] * (k[t] * r[t]).sum(-1, keepdims=True),
                                   rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out_s, np.einsum("hi,hj->hij", v[1], k[1]), rtol=1e-6)
    # the a/b term: with s = I (no decay of the diagonal, w -> 1), v = k = 0,
    # one step gives s' = I + (I a) b^T = I + a b^T
    a, b = rng.standard_normal((1, 1, S)).astype(np.float32), rng.standard_normal((1, 1, S)).astype(np.float32)
    wl = np.full((1, 1, S), -30.0, np.float32)  # exp(-exp(-30)) == 1 in f32
    z1 = np.zeros((1, 1, S), np.float32)
    _, s1 = O.rwkv7_inner_loop(z1, wl, z1, z1, a, b, np.eye(S, dtype=np.float32)[None], 1)
    np.testing.assert_allclose(s1[0], np.eye(S) + np.outer(a[0, 0], b[0, 0]), rtol=1e-6, atol=1e-6)


# -- TimeMixing (llm.rs:348-480) ------------------------------------------------
# The reference's own test (llm.rs:1163-1196) checks shapes, finiteness and the
# v_first rule; the closed forms below fix each branch separately, at T = 1 or
# through the state, so that a wrong sign, a transposed operand or a head
# mis-indexing fails one of them.

def tm_zero(C, D):
    P = {n: np.zeros(C, np.float32) for n in O.TM_VECTORS + ("w0", "v0", "a0", "k_k", "k_a",
                                                               "r_k", "ln_b")}
    P["ln_w"] = np.ones(C, np.float32)
    for n in O.TM_LINEAR:
        P[n] = np.zeros((C, C), np.float32)
    for n in ("w1", "v1", "a1", "g1"):
        P[n] = np.zeros((C, D), np.float32)
    for n in ("w2", "v2", "a2", "g2"):
        P[n] = np.zeros((D, C), np.float32)
    return P


def softplus(x):
    return np.logaddexp(0.0, x)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def test_time_mixing_reference_structural_case():
    # llm.rs:1163-1196: T=2, H=2, S=2, C=4, zero weights; layer 1 keeps v_first
    P = tm_zero(4, 4)
    x = np.array([[1, 0, 1, 0], [0, 1, 0, 1]], np.float32)
    out, st, vf = O.time_mixing(P, x, np.zeros((3, 4)), np.zeros((2, 4)), 2, 2, 0)
    assert out.shape == (2, 4) and st.shape == (3, 4) and vf.shape == (2, 4)
    assert np.isfinite(out).all()
    vf_in = np.arange(8, dtype=np.float32).reshape(2, 4)
    _, _, vf2 = O.time_mixing(P, x, np.zeros((3, 4)), vf_in, 2, 2, 1)
    np.testing.assert_array_equal(vf2, vf_in)


def test_time_mixing_readout_and_gate_closed_form():
    # receptance = key = value = output = I, r_k = 1, ln_w = 0 (group norm -> ln_b = 0),
    # g1 = 0 -> sigmoid 0.5, g2 row 0 = 2 -> g = 1:  out = (sum_{s in head} x_s^2) x
    C, H, D, T = 8, 2, 3, 3
    P = tm_zero(C, D)
    for n in O.TM_LINEAR:
        P[n] = np.eye(C, dtype=np.float32)
    P["r_k"][:] = 1
    P["ln_w"][:] = 0
    P["g2"][0] = 2
    rng = np.random.default_rng(1)
    x = rng.standard_normal((T, C)).astype(np.float32)
    out, _, vf = O.time_mixing(P, x, np.zeros((1 + C // H, C)), np.zeros((T, C)), H, T, 0)
    hs = (x.reshape(T, H, -1) ** 2).sum(-1)
    ref = (hs[:, :, None] * x.reshape(T, H, -1)).reshape(T, C)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(vf, x)   # layer 0: v_first = v = x


def test_time_mixing_decay_value_blend_and_state_closed_form():
    # k_k = 0 -> kk = 0, a_i = b_i = 0: the state update is s = s0 diag(exp(-exp(w))) + v k^T
    # with w = -softplus(-(w0 + tanh(xw W1) W2)) - 0.5 (Tmm operands (in, out)), and at a
    # later layer v = value(xv) + (v_first - value(xv)) sigmoid(v0 + tanh(xv V1) V2).
    C, H, D = 8, 2, 3
    S = C // H
    rng = np.random.default_rng(2)
    P = tm_zero(C, D)
    P["key"] = rng.standard_normal((C, C)).astype(np.float32)
    P["value"] = rng.standard_normal((C, C)).astype(np.float32)
    P["w0"] = rng.standard_normal(C).astype(np.float32)
    P["w1"] = rng.standard_normal((C, D)).astype(np.float32)
    P["w2"] = rng.standard_normal((D, C)).astype(np.float32)
    P["v0"] = rng.standard_normal(C).astype(np.float32)
    P["v1"] = rng.standard_normal((C, D)).astype(np.float32)
    P["v2"] = rng.standard_normal((D, C)).astype(np.float32)
    P["x_w"] = rng.random(C).astype(np.float32)
    P["x_k"] = rng.random(C).astype(np.float32)
    P["x_v"] = rng.random(C).astype(np.float32)
    x = rng.standard_normal((1, C)).astype(np.float32)
    state = rng.standard_normal((1 + S, C)).astype(np.float32)
    vf_in = rng.standard_normal((1, C)).astype(np.float32)
    _, st, vf = O.time_mixing(P, x, state, vf_in, H, 1, 1)
    f = np.float64
    sx = state[0].astype(f) - x[0]
    xw, xk, xv = x[0] + sx * P["x_w"], x[0] + sx * P["x_k"], x[0] + sx * P["x_v"]
    w = -softplus(-(P["w0"] + np.tanh(xw @ P["w1"]) @ P["w2"])) - 0.5
    k = P["key"].astype(f) @ xk
    v0 = P["value"].astype(f) @ xv
    v = v0 + (vf_in[0] - v0) * sigmoid(P["v0"] + np.tanh(xv @ P["v1"]) @ P["v2"])
    dec = np.exp(-np.exp(w))
    s0 = state[1:].reshape(H, S, S).astype(f)
    ref = np.stack([s0[h] * dec[h * S:(h + 1) * S][None, :]
                    + np.outer(v[h * S:(h + 1) * S], k[h * S:(h + 1) * S]) for h in range(H)])
    np.testing.assert_allclose(st[1:].reshape(H, S, S), ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_array_equal(st[0], x[0])       # state[0] = x[length - 1]
    np.testing.assert_array_equal(vf, vf_in)          # layer > 0 leaves v_first


def test_time_mixing_delta_rule_closed_form():
    # k_k = 1, a = sigmoid(a0 + tanh(xa A1) A2): kk = k / |k|_head, k' = k (k_a (a - 1) + 1),
    # one step of the RWKV-7 delta rule  S' = S (diag(d) - kk^T (a kk)) + v k'^T  per head.
    C, H, D = 8, 2, 4
    S = C // H
    rng = np.random.default_rng(3)
    P = tm_zero(C, D)
    P["key"] = rng.standard_normal((C, C)).astype(np.float32)
    P["value"] = rng.standard_normal((C, C)).astype(np.float32)
    P["w0"] = rng.standard_normal(C).astype(np.float32)
    P["a0"] = rng.standard_normal(C).astype(np.float32)
    P["a1"] = rng.standard_normal((C, D)).astype(np.float32)
    P["a2"] = rng.standard_normal((D, C)).astype(np.float32)
    P["k_k"][:] = 1
    P["k_a"] = rng.random(C).astype(np.float32)
    P["x_a"] = rng.random(C).astype(np.float32)
    x = rng.standard_normal((1, C)).astype(np.float32)
    state = rng.standard_normal((1 + S, C)).astype(np.float32)
    _, st, _ = O.time_mixing(P, x, state, np.zeros((1, C)), H, 1, 0)
    f = np.float64
    sx = state[0].astype(f) - x[0]
    xa = x[0] + sx * P["x_a"]
    k = P["key"].astype(f) @ x[0]
    v = P["value"].astype(f) @ x[0]
    a = sigmoid(P["a0"] + np.tanh(xa @ P["a1"]) @ P["a2"])
    d = np.exp(-np.exp(-softplus(-P["w0"].astype(f)) - 0.5))
    s0 = state[1:].reshape(H, S, S).astype(f)
    for h in range(H):
        sl = slice(h * S, (h + 1) * S)
        kk = k[sl] / np.linalg.norm(k[sl])
        kp = k[sl] * (P["k_a"][sl] * (a[sl] - 1) + 1)
        ref = s0[h] @ (np.diag(d[sl]) - np.outer(kk, a[sl] * kk)) + np.outer(v[sl], kp)
        np.testing.assert_allclose(st[1:].reshape(H, S, S)[h], ref, rtol=1e-4, atol=1e-5)


def test_time_mixing_group_norm_branch_closed_form():
    # s0 = 0, T = 1: wkv = v (k . r) per head; out = GroupNorm_H(wkv) g with output = I,
    # g = sigmoid(xg G1) G2, r_k = 0 (no readout).
    C, H, D = 8, 2, 3
    S = C // H
    rng = np.random.default_rng(4)
    P = tm_zero(C, D)
    for n in ("receptance", "key", "value"):
        P[n] = rng.standard_normal((C, C)).astype(np.float32)
    P["output"] = np.eye(C, dtype=np.float32)
    P["ln_w"] = rng.standard_normal(C).astype(np.float32)
    P["ln_b"] = rng.standard_normal(C).astype(np.float32)
    P["g1"] = rng.standard_normal((C, D)).astype(np.float32)
    P["g2"] = rng.standard_normal((D, C)).astype(np.float32)
    P["x_g"] = rng.random(C).astype(np.float32)
    x = rng.standard_normal((1, C)).astype(np.float32)
    state = np.zeros((1 + S, C), np.float32)
    state[0] = rng.standard_normal(C)
    out, _, _ = O.time_mixing(P, x, state, np.zeros((1, C)), H, 1, 0)
    f = np.float64
    r, k, v = (P[n].astype(f) @ x[0] for n in ("receptance", "key", "value"))
    xg = x[0] + (state[0] - x[0].astype(f)) * P["x_g"]
    g = sigmoid(xg @ P["g1"]) @ P["g2"]
    ref = np.empty(C)
    for h in range(H):
        sl = slice(h * S, (h + 1) * S)
        y = v[sl] * (k[sl] @ r[sl])
        ref[sl] = (y - y.mean()) / np.sqrt(y.var() + 64e-5) * P["ln_w"][sl] + P["ln_b"][sl]
    np.testing.assert_allclose(out[0], ref * g, rtol=1e-4, atol=1e-5)


def test_time_mixing_length_and_new_starts():
    # state[0] = x[length - 1]; a new start at t zeroes the shifted row (t = 0 uses state[0])
    C, H, D, T = 4, 1, 2, 4
    rng = np.random.default_rng(5)
    P = tm_zero(C, D)
    P["receptance"] = np.eye(C, dtype=np.float32)
    P["key"] = np.eye(C, dtype=np.float32)
    P["value"] = np.eye(C, dtype=np.float32)
    P["output"] = np.eye(C, dtype=np.float32)
    P["x_r"][:] = 1     # xr = shifted row: r_t = x_{t-1} (state[0] at t = 0, 0 at a new start)
    P["r_k"][:] = 1
    P["ln_w"][:] = 0
    P["g2"][0] = 2
    x = rng.standard_normal((T, C)).astype(np.float32)
    state = np.zeros((1 + C, C), np.float32)
    state[0] = rng.standard_normal(C)
    ns = [False, False, True, False]
    out, st, _ = O.time_mixing(P, x, state, np.zeros((T, C)), H, 3, 0, new_starts=ns)
    prev = np.vstack([state[0], x[:-1]])
    prev[2] = 0
    ref = ((prev * x).sum(-1))[:, None] * x        # (sum r k r_k) v with r = prev, k = v = x
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(st[0], x[2])


# -- the RWKV-7 LM (rwkv7.py:189-253) ------------------------------------------

def lm_params(rng, L, C, F, V, D=8, zero_out=False):
    P = {"emb": rng.standard_normal((V, C)).astype(np.float32),
         "head": (rng.standard_normal((V, C)) / np.sqrt(C)).astype(np.float32),
         "ln0_w": (1 + 0.1 * rng.standard_normal(C)).astype(np.float32),
         "ln0_b": (0.1 * rng.standard_normal(C)).astype(np.float32),
         "ln_out_w": (1 + 0.1 * rng.standard_normal(C)).astype(np.float32),
         "ln_out_b": (0.1 * rng.standard_normal(C)).astype(np.float32), "blocks": []}
    for _ in range(L):
        B = tm_zero(C, D)
        for n in O.TM_VECTORS + ("w0", "v0", "a0", "k_a", "r_k", "ln_b"):
            B[n] = (rng.random(C) * 0.5).astype(np.float32)
        B["k_k"] = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
        B["ln_w"] = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
        for n in O.TM_LINEAR:
            B[n] = (rng.standard_normal((C, C)) / np.sqrt(C)).astype(np.float32)
        for n in ("w1", "v1", "a1", "g1"):
            B[n] = (rng.standard_normal((C, D)) / np.sqrt(C)).astype(np.float32)
        for n in ("w2", "v2", "a2", "g2"):
            B[n] = (rng.standard_normal((D, C)) / np.sqrt(D)).astype(np.float32)
        B["ffn_x_k"] = rng.random(C).astype(np.float32)
        B["ffn_key"] = (rng.standard_normal((F, C)) / np.sqrt(C)).astype(np.float32)
        B["ffn_value"] = (rng.standard_normal((C, F)) / np.sqrt(F)).astype(np.float32)
        for n in ("ln1_w", "ln2_w"):
            B[n] = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
        for n in ("ln1_b", "ln2_b"):
            B[n] = (0.1 * rng.standard_normal(C)).astype(np.float32)
        if zero_out:
            B["output"][:] = 0
            B["ffn_value"][:] = 0
        P["blocks"].append(B)
    return P


def test_lm_with_silent_blocks_is_embedding_norm_head():
    # output = ffn value = 0: every block adds 0, so logits = ln_out(ln0(emb[tok])) head^T,
    # and each block's state rows 0 / 1 hold ln2 / ln1 of the last residual row.
    L, C, F, V, H, T = 2, 16, 32, 11, 2, 6
    rng = np.random.default_rng(6)
    P = lm_params(rng, L, C, F, V, zero_out=True)
    tok = rng.integers(0, V, T)
    logits, st = O.rwkv_lm_forward(P, tok, H)
    f = np.float64

    def ln(x, w, b):
        m = x.mean(-1, keepdims=True)
        return (x - m) / np.sqrt(x.var(-1, keepdims=True) + 1e-5) * w + b
    x = ln(P["emb"][tok].astype(f), P["ln0_w"], P["ln0_b"])
    ref = ln(x, P["ln_out_w"], P["ln_out_b"]) @ P["head"].T.astype(f)
    np.testing.assert_allclose(logits, ref, rtol=1e-4, atol=1e-4)
    for l, B in enumerate(P["blocks"]):
        np.testing.assert_allclose(st[l, 0], ln(x[-1], B["ln2_w"], B["ln2_b"]), rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(st[l, 1], ln(x[-1], B["ln1_w"], B["ln1_b"]), rtol=1e-4, atol=1e-5)


def test_lm_state_carry_equals_one_pass():
    # the model is recurrent: running tokens [0, T1) and then [T1, T) from the carried
    # state gives the one-pass logits and state, bit for bit (every op is per token
    # or in token order).
    L, C, F, V, H, T, T1 = 2, 16, 32, 13, 2, 9, 4
    rng = np.random.default_rng(7)
    P = lm_params(rng, L, C, F, V)
    tok = rng.integers(0, V, T)
    full, st_full = O.rwkv_lm_forward(P, tok, H)
    a, st_a = O.rwkv_lm_forward(P, tok[:T1], H)
    b, st_b = O.rwkv_lm_forward(P, tok[T1:], H, st_a)
    np.testing.assert_array_equal(np.vstack([a, b]), full)
    np.testing.assert_array_equal(st_b, st_full)


def test_lm_one_block_wiring():
    # one block from the pinned components: x0 = ln0(emb); x1 = x0 + att(ln1 x0);
    # x2 = x1 + ffn(ln2 x1); logits = ln_out(x2) head^T; state rows [ffn last, att state]
    L, C, F, V, H, T = 1, 16, 32, 7, 4, 5
    rng = np.random.default_rng(8)
    P = lm_params(rng, L, C, F, V)
    tok = rng.integers(0, V, T)
    st0 = (rng.standard_normal((1, 2 + C // H, C)) * 0.3).astype(np.float32)
    logits, st = O.rwkv_lm_forward(P, tok, H, st0)
    B = P["blocks"][0]
    x0 = O.layer_norm(P["emb"][tok], P["ln0_w"], P["ln0_b"])
    att, st_att, _ = O.time_mixing(B, O.layer_norm(x0, B["ln1_w"], B["ln1_b"]), st0[0, 1:],
                                   np.zeros((T, C)), H, T, 0)
    x1 = x0 + att
    h2 = O.layer_norm(x1, B["ln2_w"], B["ln2_b"])
    ffn, last = O.channel_mixing(h2, st0[0, 0], B["ffn_x_k"], B["ffn_key"], B["ffn_value"], T)
    x2 = x1 + ffn
    ref = O.layer_norm(x2, P["ln_out_w"], P["ln_out_b"]) @ P["head"].T
    np.testing.assert_allclose(logits, ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(st[0, 0], last)
    np.testing.assert_array_equal(st[0, 1:], st_att)
