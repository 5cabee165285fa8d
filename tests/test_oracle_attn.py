"""Pins of the C4 oracle (oracle/oracle_attn.c, the spiking self-attention
transformer of src/hyperscalees/models/snn_self_attention_heads.py).

The reference has no tests for this model (its Rust port,
snn_transformer.rs, replaces the LIF parts by continuous relaxations and tests
shapes only), so each function is pinned by closed forms a plausible
restatement mistake breaks: constant-current LIF counts, the inhibition's
effect traced by hand, degenerate attention rows, the per-row max
normalisation of lif_single, and the whole forward reducing to the position
embedding and readout when nothing fires.  CPU only.
"""
import math

import numpy as np
import pytest

from tests import oracle_lib as O


def lif_period(c, vth, tau):
    """First step k at which a LIF from v = 0 under constant current c reaches
    vth: c (1 - (1 - 1/tau)^k) >= vth (none when c <= vth)."""
    if c <= vth:
        return None
    return math.ceil(math.log(1.0 - vth / c) / math.log(1.0 - 1.0 / tau))


def test_softplus_values(oracle):
    for x in (-30.0, -3.0, -0.5, 0.0, 0.25, 2.0, 40.0):
        ref = math.log1p(math.exp(-abs(x))) + max(x, 0.0)
        assert oracle.or_sa_softplus(x) == pytest.approx(ref, rel=2e-7, abs=1e-30)
    # the initial raw threshold log(exp(v) - 1) maps back to v
    raw = np.float32(np.log(np.expm1(np.float32(0.05))))
    assert oracle.or_sa_softplus(float(raw)) == pytest.approx(0.05, rel=1e-5)


def test_row_softmax_lif_without_inhibition_is_constant_current_lif():
    # g_inh = 0: every key neuron is an independent LIF under constant current
    # h_j / max|h|, firing every k* steps (reset to 0): count = floor(n_iter / k*)
    h = np.array([1.0, 0.5, 0.2, -1.0], np.float32)
    p = np.zeros(4, np.float32)
    O.load().or_sa_row_softmax_lif(h, 4, 0.1, 0.0, 20.0, 8, p)
    counts = [0 if lif_period(c, 0.1, 20.0) is None else 8 // lif_period(c, 0.1, 20.0)
              for c in (h / np.abs(h).max()).tolist()]
    assert counts == [2, 1, 0, 0]
    np.testing.assert_allclose(p, np.array(counts) / (sum(counts) + 1e-6), rtol=1e-6)


@pytest.mark.parametrize("h,vth,g,counts", [
    # traced by hand: the first spikes (step 3) raise the inhibition of all
    # neurons by g per spike, so the weaker ones never reach the threshold again
    ([1.0, 0.9, 0.8, 0.3], 0.1, 0.2, [1, 1, 1, 0]),   # without inhibition 2, 2, 2, 1
    ([2.0, 1.0, 0.5], 0.08, 0.15, [3, 1, 0]),         # without inhibition 4, 2, 1
    ([1.0, 0.95], 0.1, 0.5, [1, 1]),                  # without inhibition 2, 2
])
def test_row_softmax_lif_inhibition(h, vth, g, counts):
    h = np.array(h, np.float32)
    p = np.zeros(h.size, np.float32)
    O.load().or_sa_row_softmax_lif(h, h.size, vth, g, 20.0, 8, p)
    np.testing.assert_allclose(p, np.array(counts) / (sum(counts) + 1e-6), rtol=1e-6)


def test_row_softmax_lif_silent_row_and_scale_invariance():
    p = np.zeros(5, np.float32)
    O.load().or_sa_row_softmax_lif(np.zeros(5, np.float32), 5, 0.1, 0.5, 20.0, 8, p)
    assert not p.any()                    # no spike: 0 / (0 + 1e-6)
    h = np.array([0.3, -0.2, 0.1, 0.25], np.float32)
    p1, p2 = np.zeros(4, np.float32), np.zeros(4, np.float32)
    O.load().or_sa_row_softmax_lif(h, 4, 0.05, 0.3, 20.0, 8, p1)
    O.load().or_sa_row_softmax_lif(h * np.float32(8.0), 4, 0.05, 0.3, 20.0, 8, p2)
    np.testing.assert_allclose(p1, p2, rtol=1e-6)   # rows are normalised by max |h|
    assert abs(p1.sum() - 1.0) < 1e-5 and p1[0] > 0


def test_attention_head_closed_forms():
    rng = np.random.default_rng(0)
    R, hd = 6, 4
    q = rng.standard_normal((R, hd)).astype(np.float32)
    v = rng.standard_normal((R, hd)).astype(np.float32)
    # identical keys: every key neuron sees the same current, so each row's
    # weights are uniform over the keys and every output row is mean(V)
    k = np.tile(np.abs(q[:1]), (R, 1)).astype(np.float32)
    q = np.abs(q)
    out = np.zeros((R, hd), np.float32)
    O.load().or_sa_attention_head(q.ctypes.data, k.ctypes.data, v.ctypes.data, R, hd, hd, 0.5,
                                  0.05, 0.5, 20.0, 8, out.ctypes.data)
    np.testing.assert_allclose(out, np.tile(v.mean(0), (R, 1)), rtol=1e-5, atol=1e-6)
    # a threshold no neuron reaches: all weights 0, output 0
    O.load().or_sa_attention_head(q.ctypes.data, k.ctypes.data, v.ctypes.data, R, hd, hd, 0.5,
                                  5.0, 0.5, 20.0, 8, out.ctypes.data)
    assert not out.any()
    # one key aligned with the query, the others orthogonal (h = 0): only it
    # fires, the row's output is that key's value
    q1 = np.eye(hd, dtype=np.float32)[:1].repeat(R, 0)
    k1 = np.zeros((R, hd), np.float32)
    k1[3, 0] = 1.0
    O.load().or_sa_attention_head(q1.ctypes.data, k1.ctypes.data, v.ctypes.data, R, hd, hd, 1.0,
                                  0.1, 0.5, 20.0, 8, out.ctypes.data)
    np.testing.assert_allclose(out, np.tile(v[3], (R, 1)), rtol=1e-5)


def test_ffn_spike_row_max_normalisation():
    c = np.array([[0.1, -0.4, 0.2, 0.4], [10.0, 5.0, -20.0, 9.9]], np.float32)
    act = np.zeros_like(c)
    O.load().or_sa_ffn_spike(c, 2, 4, 0.5, act)
    # per row: c / max|c| >= 0.5 (row 0: 0.25, -1, 0.5, 1; row 1: 0.5, 0.25, -1, 0.495)
    np.testing.assert_array_equal(act, [[0, 0, 1, 1], [1, 0, 0, 0]])
    # an all-zero row divides by 1e-6: 0 >= 0 gates every column open
    act0 = np.zeros((1, 4), np.float32)
    O.load().or_sa_ffn_spike(np.zeros((1, 4), np.float32), 1, 4, 0.0, act0)
    np.testing.assert_array_equal(act0, np.ones((1, 4)))


def test_encode_closed_form():
    T, R, d = 8, 2, 3
    cq = np.full((T, R, d), 1.0, np.float32)      # fires every 3rd step at threshold 0.1
    ck = np.zeros((T, R, d), np.float32)           # never fires
    cv = np.full((T, R, d), 100.0, np.float32)     # fires every step
    pos = np.arange(R * d, dtype=np.float32).reshape(R, d) * 0.01
    X = np.zeros((R, d), np.float32)
    O.load().or_sa_encode(cq, ck, cv, T, R, d, 0.1, 0.1, 0.1, 20.0, pos, X)
    k = lif_period(1.0, 0.1, 20.0)
    rq = (T // k) / T
    np.testing.assert_allclose(X, (rq + 0.0 + 1.0) / 3.0 + pos, rtol=1e-6)


def small_cfg():
    from hyperscalees_amd.snn_attention import SaConfig
    return SaConfig(tin=4, ntok=5, d_model=8, heads=2, blocks=2, classes=3, T=4, n=2, rank=2)


def test_forward_reduces_to_position_and_readout_when_silent():
    # thresholds no LIF reaches: rates 0, attention weights 0, ffn gates 0, so
    # X = pos_emb through both blocks and logits = (mean_tokens pos) W_out^T * gain
    from hyperscalees_amd import snn_attention as sa
    c = small_cfg()
    P = sa.init_params(c, seed=1)
    rng = np.random.default_rng(2)
    P["pos_emb"] = rng.standard_normal(P["pos_emb"].shape).astype(np.float32)
    for name in ("q_th", "k_th", "v_th", "attn_th", "b0_ff_th", "b1_ff_th"):
        P[name] = np.full((1, 1), 50.0, np.float32)
    P["out_gain"] = np.full((1, 1), 1.5, np.float32)
    x = (rng.random((c.T, c.ntok, c.tin)) < 0.5).astype(np.float32)
    got = O.sa_forward_member(c, P, x)
    ref = (P["pos_emb"].astype(np.float64).mean(0) @ P["out"].astype(np.float64).T) * 1.5
    np.testing.assert_allclose(got, ref, rtol=1e-5)


def test_forward_ffn_only_closed_form():
    # silent encoder and attention, an active ffn gate: per block
    # X += gate(X W_ff1^T) W_ff2^T with gate the row-max-normalised threshold
    from hyperscalees_amd import snn_attention as sa
    c = small_cfg()
    P = sa.init_params(c, seed=3)
    rng = np.random.default_rng(4)
    P["pos_emb"] = rng.standard_normal(P["pos_emb"].shape).astype(np.float32)
    for name in ("q_th", "k_th", "v_th", "attn_th"):
        P[name] = np.full((1, 1), 50.0, np.float32)
    P["b0_ff_th"] = np.full((1, 1), -1.0, np.float32)    # softplus: 0.313
    P["b1_ff_th"] = np.full((1, 1), 0.0, np.float32)     # softplus: 0.693
    x = np.zeros((c.T, c.ntok, c.tin), np.float32)
    X = P["pos_emb"].astype(np.float64)
    for b in range(c.blocks):
        th = math.log1p(math.exp(float(P[f"b{b}_ff_th"][0, 0])))
        cur = X @ P[f"b{b}_ff1"].astype(np.float64).T
        gate = (cur / np.maximum(np.abs(cur).max(1, keepdims=True), 1e-6) >= th).astype(np.float64)
        X = X + gate @ P[f"b{b}_ff2"].astype(np.float64).T
    ref = X.mean(0) @ P["out"].astype(np.float64).T
    got = O.sa_forward_member(c, P, x)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
