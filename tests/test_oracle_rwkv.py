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
