"""Pins of the CPU oracle (oracle/oracle.c) against the reference's own
known-answer tests, closed forms and invariants.  CPU only.

Each test names the reference test or property it follows (paths relative to
the reference root).  The reference ships no fixture files (its tests are
inline Rust), so the pins are its known answers plus properties a plausible
restatement mistake would break.
"""
import ctypes
import math

import numpy as np
import pytest

from tests import oracle_lib as O

M64 = 2**64 - 1
_libm = ctypes.CDLL("libm.so.6")
_libm.logf.restype = ctypes.c_float
_libm.logf.argtypes = [ctypes.c_float]
_libm.cosf.restype = ctypes.c_float
_libm.cosf.argtypes = [ctypes.c_float]
_libm.sqrtf.restype = ctypes.c_float
_libm.sqrtf.argtypes = [ctypes.c_float]


# ---- noise stream ----------------------------------------------------------

def py_noise_seed(key, te, tt):
    """noiser.rs:495-506 in Python integers (Rust i32 -> u64 sign-extends)."""
    h = (key ^ 0x9E3779B97F4A7C15) & M64
    h = (h * 0xBF58476D1CE4E5B9) & M64
    h ^= ((te & M64) * 0x94D049BB133111EB) & M64
    h = (((h << 17) | (h >> 47)) & M64) ^ (tt & M64)
    h ^= h >> 33
    h = (h * 0xBF58476D1CE4E5B9) & M64
    h ^= h >> 29
    h = (h * 0x94D049BB133111EB) & M64
    h ^= h >> 32
    return h


def py_xs64(x):
    x ^= (x << 13) & M64
    x ^= x >> 7
    x ^= (x << 17) & M64
    return x


def test_noise_seed_matches_python_restatement(oracle):
    rng = np.random.default_rng(0)
    cases = [(0, 0, 0), (42, 0, 0), (7, 3, 5), (M64, -1, -7), (0x9E3779B97F4A7C15, 2**31 - 1, 12)]
    cases += [(int(rng.integers(0, 2**63)) * 2 + 1, int(rng.integers(-2**31, 2**31)),
               int(rng.integers(0, 2**31))) for _ in range(200)]
    for k, e, t in cases:
        assert oracle.or_noise_seed(k, e, t) == py_noise_seed(k, e, t), (k, e, t)


def test_negative_epoch_sign_extends(oracle):
    # A zero-extending restatement would agree on non-negative inputs only.
    assert oracle.or_noise_seed(5, -1, 3) == py_noise_seed(5, -1, 3)
    assert oracle.or_noise_seed(5, -1, 3) != py_noise_seed(5, 2**32 - 1, 3)


def test_xorshift64_step_and_unit(oracle):
    x = 0x123456789ABCDEF1
    for _ in range(100):
        nx = py_xs64(x)
        assert oracle.or_xorshift64_step(x) == nx
        assert oracle.or_unit_from_u64(nx) == np.float32((nx >> 40) / 2**24)
        x = nx


def test_xorshift64_has_full_period_structure(oracle):
    # (13, 7, 17) is one of Marsaglia's full-period triples: no state returns to
    # itself within a short cycle and zero is a fixed point only of itself.
    assert oracle.or_xorshift64_step(0) == 0
    x = 1
    seen = set()
    for _ in range(10000):
        x = oracle.or_xorshift64_step(x)
        assert x not in seen and x != 0
        seen.add(x)


def py_normal_stream(seed, n):
    s = seed | 1
    out = []
    for _ in range(n):
        s = py_xs64(s)
        k1 = s >> 40
        s = py_xs64(s)
        k2 = s >> 40
        u1 = np.float32(k1) / np.float32(2**24)
        u1 = max(u1, np.float32(1e-9))
        r = _libm.sqrtf(np.float32(-2.0) * np.float32(_libm.logf(u1)))
        th = np.float32(np.float32(6.2831855) * (np.float32(k2) / np.float32(2**24)))
        out.append(np.float32(np.float32(r) * np.float32(_libm.cosf(th))))
    return np.array(out, np.float32)


def test_standard_normals_match_python_libm_restatement(oracle):
    for seed in [0, 1, 2, 1234, py_noise_seed(42, 0, 3)]:
        a = np.zeros(300, np.float32)
        oracle.or_standard_normals(seed, a, 300)
        np.testing.assert_array_equal(a, py_normal_stream(seed, 300))


def test_seed_or_one_rule(oracle):
    # noiser.rs:449: state = seed | 1, so seeds 0 and 1 give the same stream
    # and 2 and 3 do too (noiser.rs:686-700 uses new(1) vs new(2)).
    a, b, c = (np.zeros(16, np.float32) for _ in range(3))
    oracle.or_standard_normals(0, a, 16)
    oracle.or_standard_normals(1, b, 16)
    oracle.or_standard_normals(2, c, 16)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c)


def test_standard_normals_are_standard_normal(oracle):
    from scipy import stats
    x = np.zeros(400_000, np.float32)
    oracle.or_standard_normals(987654321, x, x.size)
    assert abs(x.mean()) < 0.01
    assert abs(x.var() - 1.0) < 0.01
    assert stats.kstest(x.astype(np.float64), "norm").pvalue > 1e-3
    # Box-Muller with the cos branch only: max |n| <= sqrt(-2 ln 1e-9) (u1 clamp).
    assert np.abs(x).max() <= math.sqrt(-2 * math.log(1e-9)) + 1e-3


def test_bm_halves_are_glibc(oracle):
    rng = np.random.default_rng(1)
    for k in list(rng.integers(0, 2**24, 2000)) + [0, 1, 2**23, 2**24 - 1]:
        k = int(k)
        u = np.float32(k) / np.float32(2**24)
        u1 = max(u, np.float32(1e-9))
        assert oracle.or_bm_radius(k) == _libm.sqrtf(np.float32(-2.0) * np.float32(_libm.logf(u1)))
        th = np.float32(np.float32(6.2831855) * u)
        assert oracle.or_bm_cos(k) == _libm.cosf(th)


# ---- factors (eggroll.rs:86-227) -------------------------------------------

def test_lora_params_shape_determinism_thread_variation(oracle):
    # eggroll.rs:1075-1096
    A1, B1 = O.lora_factors(0.5, 42, 2, 1, [0], 2, 3)
    A2, B2 = O.lora_factors(0.5, 42, 2, 1, [0], 2, 3)
    assert A1.shape == (1, 2, 2) and B1.shape == (1, 3, 2)
    np.testing.assert_array_equal(A1, A2)
    np.testing.assert_array_equal(B1, B2)
    A3, _ = O.lora_factors(0.5, 42, 2, 1, [4], 2, 3)
    assert np.any(A1 != A3)


def test_lora_params_layout_is_b_rows_then_a_rows(oracle):
    # eggroll.rs:98-102: one stream of (a+b)*r normals, B = rows [0,b), A = rows [b,a+b)*sc
    a, b, r, key = 3, 5, 4, 77
    A, B = O.lora_factors(1.0, key, r, 0, [0], a, b)
    s = np.zeros((a + b) * r, np.float32)
    oracle.or_standard_normals(py_noise_seed(key, 0, 0), s, s.size)
    np.testing.assert_array_equal(B[0], s[: b * r].reshape(b, r))
    np.testing.assert_array_equal(A[0], s[b * r:].reshape(a, r))


def test_antithetic_pairing(oracle):
    # eggroll.rs:60-65: threads 2i and 2i+1 share a stream, A negated for odd.
    A, B = O.lora_factors(0.3, 9, 3, 0, [0, 1, 6, 7], 4, 5)
    np.testing.assert_array_equal(B[0], B[1])
    np.testing.assert_array_equal(A[1], -A[0])
    np.testing.assert_array_equal(B[2], B[3])
    np.testing.assert_array_equal(A[3], -A[2])
    assert np.any(B[0] != B[2])


def test_epoch_mapping(oracle):
    # noise_reuse 0 -> epoch ignored; noise_reuse 2 -> epochs 0,1 share, 2 differs
    f = lambda e, nr: O.lora_factors(0.3, 9, 2, e, [3], 2, 2, noise_reuse=nr)[1]
    np.testing.assert_array_equal(f(0, 0), f(5, 0))
    np.testing.assert_array_equal(f(0, 2), f(1, 2))
    assert np.any(f(0, 2) != f(2, 2))


def test_batched_matches_per_thread(oracle):
    # eggroll.rs:1100-1129 (bit-exact)
    tids = np.array([0, 1, 2], np.int32)
    Ab, Bb = O.lora_factors(0.25, 1234, 2, 5, tids, 2, 3, noise_reuse=1)
    for i, t in enumerate(tids):
        A = np.zeros((2, 2), np.float32)
        B = np.zeros((3, 2), np.float32)
        oracle.or_get_lora_update_params(0.25, 1234, 2, 5, int(t), 2, 3, 1, A, B)
        np.testing.assert_array_equal(Ab[i], A)
        np.testing.assert_array_equal(Bb[i], B)


def test_base_sigma(oracle):
    assert oracle.or_base_sigma(0.02, 128) == np.float32(0.02) / np.float32(math.sqrt(128))
    assert oracle.or_base_sigma(0.5, 4) == np.float32(0.25)


# ---- do_mm (noiser.rs:553-620, eggroll.rs:1599-1612) -----------------------

def test_do_mm_known_answer():
    W = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    x = np.array([[1, 1, 1], [2, 2, 2]], np.float32)
    np.testing.assert_array_equal(O.do_mm(x, W).ravel(), [6, 15, 12, 30])


def test_do_tmm_known_answer(oracle):
    W = np.array([[1, 4], [2, 5], [3, 6]], np.float32)
    x = np.array([[1, 1, 1]], np.float32)
    y = np.zeros((1, 2), np.float32)
    oracle.or_do_Tmm(x, 1, W, 3, 2, None, None, 0, y)
    np.testing.assert_array_equal(y.ravel(), [6, 15])


def test_do_tmm_is_do_mm_transposed(oracle):
    # x W + (x A) B^T == do_mm(x; W^T, with B as the output-side and A as the
    # input-side factor): ties the LoRA term of do_Tmm to the pinned do_mm.
    # Integer-valued operands keep every product exact in f32.
    rng = np.random.default_rng(3)
    a, b, r, rows = 5, 4, 2, 3
    x = rng.integers(-3, 4, (rows, a)).astype(np.float32)
    W = rng.integers(-3, 4, (a, b)).astype(np.float32)
    A = rng.integers(-3, 4, (a, r)).astype(np.float32)
    B = rng.integers(-3, 4, (b, r)).astype(np.float32)
    y = np.zeros((rows, b), np.float32)
    oracle.or_do_Tmm(x, rows, W, a, b, A.ctypes.data, B.ctypes.data, r, y)
    np.testing.assert_array_equal(y, O.do_mm(x, np.ascontiguousarray(W.T), B, A))
    np.testing.assert_array_equal(y, x @ W + (x @ A) @ B.T)
    assert not np.array_equal(y, x @ W)  # the LoRA term is not zero here


def test_do_mm_noise_matches_brute_force():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 11)).astype(np.float32)
    W = rng.standard_normal((5, 11)).astype(np.float32)
    A, B = O.lora_factors(0.1, 5, 3, 0, [1], 5, 11)
    y = O.do_mm(x, W, A[0], B[0])
    ref = x.astype(np.float64) @ W.T.astype(np.float64) + (
        x.astype(np.float64) @ B[0].astype(np.float64)) @ A[0].T.astype(np.float64)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    assert not np.allclose(y, O.do_mm(x, W), atol=1e-6)


# ---- LIF (snn.rs:707-779) ---------------------------------------------------

def test_lif_known_answers():
    spk, v = O.lif(np.full((1, 1, 1), 10.0, np.float32), 20.0, 0.3)
    assert spk.ravel()[0] == 1.0 and v.ravel()[0] == 0.0   # charged 0.5 fires, reset
    spk, v = O.lif(np.full((1, 1, 1), 0.1, np.float32), 20.0, 0.3)
    assert spk.ravel()[0] == 0.0
    assert v.ravel()[0] == np.float32(np.float32(0.1) * np.float32(1 / np.float32(20.0)))
    spk, _ = O.lif(np.full((10, 1, 1), 6.0, np.float32), 20.0, 0.3)
    assert spk.max() == 1.0
    spk, _ = O.lif(np.full((4, 1, 2), -10.0, np.float32), 20.0, 0.3)
    assert spk.max() == 0.0


def test_lif_linear_regime_closed_form():
    # v_th far above: v_t = v_{t-1} + (c - v_{t-1})/tau exactly the f32 recurrence;
    # compare with the double closed form c*(1 - (1 - 1/tau)^t).
    T, c, tau = 16, 0.7, 10.0
    cur = np.full((T, 3, 4), c, np.float32)
    _, v = O.lif(cur, tau, 1e9)
    np.testing.assert_allclose(v, c * (1 - (1 - 1 / tau) ** T), rtol=1e-5)


def test_lif_reset_and_decay_sequence():
    # decay 0.9 (tau 10), v_th 1.0: constant current 2.0 -> v: 0.2,0.38,0.542,...
    T = 12
    spk, _ = O.lif(np.full((T, 1, 1), 2.0, np.float32), 10.0, 1.0)
    v, exp = 0.0, []
    for _ in range(T):
        v = v + (2.0 - v) * 0.1
        s = v >= 1.0
        exp.append(1.0 if s else 0.0)
        v = 0.0 if s else v
    np.testing.assert_array_equal(spk.ravel(), exp)


# ---- Poisson (poisson_encode_fused_oxide.rs:35-106, snn_mnist.rs:313-339) ---

def test_poisson_rate():
    p = np.full((10000, 1), 0.3, np.float32)
    s = O.poisson(p, 1, (1, 2, 3, 4))
    assert set(np.unique(s)) <= {0.0, 1.0}
    assert abs(s.mean() - 0.3) < 0.03


def test_poisson_ramp_rates():
    # noise_bench.rs:396-447: p ramp -> mean rates 0.5 / 0.25 / 0.75 within 0.01
    for pv in (0.25, 0.5, 0.75):
        s = O.poisson(np.full((4000, 25), pv, np.float32), 8, (7, 0, 0, 0))
        assert abs(s.mean() - pv) < 0.01


def test_poisson_extremes_and_prefix():
    p = np.array([[0.0, 1.0, -0.5, 2.0, 0.5]], np.float32)
    s = O.poisson(p, 16)
    assert s[:, 0, 0].max() == 0 and s[:, 0, 2].max() == 0
    assert s[:, 0, 1].min() == 1 and s[:, 0, 3].min() == 1
    p = np.random.default_rng(0).random((50, 30)).astype(np.float32)
    np.testing.assert_array_equal(O.poisson(p, 8)[:8], O.poisson(p, 16)[:8])


def test_poisson_seed_mix_is_xor():
    p = np.random.default_rng(1).random((20, 7)).astype(np.float32)
    np.testing.assert_array_equal(O.poisson(p, 4, (1, 2, 3, 4)), O.poisson(p, 4, (4, 3, 2, 1)))
    np.testing.assert_array_equal(O.poisson(p, 4, (5, 0, 0, 0)), O.poisson(p, 4, (1, 4, 0, 0)))


def test_poisson_first_value_closed_form():
    # element idx, step 0: x = xorshift32(1000000007*idx + mix + 0x9E3779B9)
    p = np.full((2, 3), 0.5, np.float32)
    s = O.poisson(p, 1, (0, 0, 0, 0))
    for idx in range(6):
        x = (1000000007 * idx + 0x9E3779B9) & 0xFFFFFFFF
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        u = np.float32(np.float32((x >> 9) + 1) / np.float32(8388609.0))
        assert s[0].ravel()[idx] == (1.0 if u < np.float32(0.5) else 0.0)


# ---- fitness (snn_mnist.rs:373-444) and z-score (eggroll.rs:1050-1071) ------

def test_loglik_matches_hand_computed():
    logits = np.array([[1.0, 2.0, 0.5], [3.0, 1.0, 2.0], [0.5, 0.5, 9.0]], np.float32)
    lab = np.array([1, 0, 2], np.int32)
    got = O.loglik(logits, lab)
    for i in range(3):
        row = logits[i].astype(np.float64)
        exp = row[lab[i]] - row.max() - math.log(np.exp(row - row.max()).sum())
        assert abs(got[i] - exp) < 1e-5
    tot = sum(np.exp(O.loglik(logits, np.full(3, c, np.int32))) for c in range(3))
    np.testing.assert_allclose(tot, 1.0, atol=1e-4)


def test_convert_fitnesses_global_and_group():
    out, m, s = O.convert_fitnesses(np.array([1, 2, 3, 4], np.float32))
    assert abs(out.mean()) < 1e-3 and abs((out**2).mean() - 1) < 1e-3
    assert m == 2.5 and abs(s - math.sqrt(1.25 + 1e-5)) < 1e-6
    out, _, _ = O.convert_fitnesses(np.array([1, 2, 3, 4], np.float32), 2)
    e = 0.5 / 1.11803399
    np.testing.assert_allclose(out, [-e, e, -e, e], atol=1e-4)


# ---- ES update (eggroll.rs:1172-1568) ---------------------------------------

def test_simple_lora_update_matches_hand_computed(oracle):
    # eggroll.rs:1172-1204: a=b=2, r=1, N=1, f=1 -> (sc*a_raw) outer b_raw
    s = np.zeros(4, np.float32)
    oracle.or_standard_normals(py_noise_seed(7, 0, 0), s, 4)
    sc = np.float32(0.5) / np.float32(1.0)
    exp = np.outer(sc * s[2:4], s[0:2])
    g = np.zeros((2, 2), np.float32)
    oracle.or_simple_lora_update(0.5, 7, 1, 0, np.array([1.0], np.float32),
                                 np.zeros(1, np.int32), np.zeros(1, np.int32), 1, 2, 2, g)
    np.testing.assert_allclose(g, exp, atol=1e-4)


def test_do_update_sign_is_minus_g_sqrt_n(oracle):
    # eggroll.rs:1208-1230 (dense, N=1): grad = -sign*sigma*noise
    s = np.zeros(2, np.float32)
    oracle.or_standard_normals(py_noise_seed(5, 0, 0), s, 2)
    g = np.zeros((2, 1), np.float32)
    oracle.or_do_update_full(0.3, 5, 0, 0, np.array([1.0], np.float32), np.zeros(1, np.int32),
                             np.zeros(1, np.int32), 1, 2, 1, g)
    np.testing.assert_allclose(g.ravel(), -(np.float32(0.3) * s), atol=1e-6)


def test_sgd_pipeline_matches_formula(oracle):
    # eggroll.rs:1234-1272: p + lr*g*sqrt(N) with g = mean f_i sign_i sigma u_i
    lr, sigma, key = 0.1, 0.5, 99
    fit = np.array([1.0, 2.0], np.float32)
    g = np.zeros(2)
    for i in range(2):
        u = np.zeros(2, np.float32)
        oracle.or_standard_normals(py_noise_seed(key, 0, 0), u, 2)
        sign = 1.0 if i % 2 == 0 else -1.0
        g += fit[i] * sign * sigma * u.astype(np.float64)
    g /= 2
    exp = np.array([1.0, -1.0]) + lr * g * math.sqrt(2)
    grad = np.zeros((1, 2), np.float32)
    oracle.or_do_update_full(sigma, key, 0, 0, fit, np.zeros(2, np.int32),
                             np.array([0, 1], np.int32), 2, 1, 2, grad)
    p = np.array([1.0, -1.0], np.float32)
    out = np.zeros(2, np.float32)
    z = np.zeros(2, np.float32)
    oracle.or_solver_step(0, lr, 0.9, 0.999, 1e-8, 0.0, 1, p, grad.ravel().copy(), z, z.copy(),
                          2, out)
    np.testing.assert_allclose(out, exp, atol=1e-4)


def test_accumulated_matches_full_batch(oracle):
    # eggroll.rs:1297-1369: K=3 chunks of 4 == one do_updates (grad level, 1e-5)
    conv = np.array([1.0, -0.5, 2.0, 0.5, -1.0, 1.5, 0.25, -0.75, 1.0, -0.25, 0.75, -1.5],
                    np.float32)
    tids = np.arange(12, dtype=np.int32)
    full = np.zeros((2, 3), np.float32)
    oracle.or_do_update_lora(0.5, 42, 2, 0, conv, np.full(12, 3, np.int32), tids, 12, 2, 3, full)
    acc = np.zeros((2, 3), np.float32)
    oracle.or_accumulated_lora_grad(0.5, 42, 2, 0, 3, conv, tids, 3, 4, 2, 3, acc)
    np.testing.assert_allclose(acc, full, atol=1e-5)


def test_lora_einsum_helpers_hand_computed(oracle):
    # eggroll.rs:1373-1405 with the reference's (n,r,*) example values
    a_t = np.array([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], np.float32)
    b_t = np.array([[[1, 2, 3], [4, 5, 6]], [[7, 8, 9], [10, 11, 12]]], np.float32)
    sc = np.array([0.5, -1.0], np.float32)
    raw = np.zeros((2, 3), np.float32)
    ones = np.zeros((2, 3), np.float32)
    oracle.or_lora_einsum_raw(a_t, b_t, sc, 2, 2, 2, 3, raw)
    oracle.or_lora_einsum_ones(a_t, b_t, 2, 2, 2, 3, ones)
    np.testing.assert_allclose(raw, np.einsum("nri,nrj,n->ij", a_t, b_t, sc), atol=1e-4)
    np.testing.assert_allclose(ones, np.einsum("nri,nrj->ij", a_t, b_t), atol=1e-4)
    # the hand values: ones[0,0] = 1*1+3*4+5*7+7*10 = 118
    assert ones[0, 0] == 118.0


def test_inline_affine_matches_two_phase(oracle):
    # eggroll.rs:1502-1568: sum einsum((raw-mean)/std) == (sum einsum(raw) - mean*ones)/std
    raw = np.array([1.0, -0.5, 2.0, 0.5, -1.0, 1.5, 0.25, -0.75], np.float32)
    conv, mean, std = O.convert_fitnesses(raw)
    tids = np.arange(8, dtype=np.int32)
    two_phase = np.zeros((2, 3), np.float32)
    oracle.or_accumulated_lora_grad(0.5, 42, 2, 0, 0, conv, tids, 2, 4, 2, 3, two_phase)
    bs = oracle.or_base_sigma(0.5, 2)
    g_raw = np.zeros((2, 3), np.float64)
    g_one = np.zeros((2, 3), np.float64)
    oracle.or_lora_einsum_f64(bs, 42, 2, 0, 0, raw, tids, 8, 2, 3, g_raw)
    oracle.or_lora_einsum_f64(bs, 42, 2, 0, 0, np.ones(8, np.float32), tids, 8, 2, 3, g_one)
    out = np.zeros((2, 3), np.float32)
    oracle.or_combine_affine(g_raw.astype(np.float32), g_one.astype(np.float32), 6, mean, std, 8,
                             out)
    np.testing.assert_allclose(out, two_phase, atol=1e-4)


def test_pairing_halves_the_einsum(oracle):
    # eggroll.rs:778-807: with antithetic pairs, sum_i f_i A_i B_i^T equals
    # sum_pairs (f_2i - f_2i+1) A_2i B_2i^T
    fit = np.random.default_rng(2).standard_normal(8).astype(np.float32)
    tids = np.arange(8, dtype=np.int32)
    g = np.zeros((3, 4), np.float64)
    oracle.or_lora_einsum_f64(0.1, 3, 2, 0, 0, fit, tids, 8, 3, 4, g)
    pair = np.zeros((3, 4), np.float64)
    fp = (fit[0::2] - fit[1::2]).astype(np.float32)
    oracle.or_lora_einsum_f64(0.1, 3, 2, 0, 0, fp, tids[0::2].copy(), 4, 3, 4, pair)
    np.testing.assert_allclose(g, pair, rtol=1e-6, atol=1e-7)


# ---- solver (noiser.rs:155-225) ----------------------------------------------

def test_adam_first_step_closed_form(oracle):
    g = np.array([0.5, -2.0, 1e-3], np.float32)
    p = np.array([1.0, 2.0, 3.0], np.float32)
    m = np.zeros(3, np.float32)
    v = np.zeros(3, np.float32)
    out = np.zeros(3, np.float32)
    oracle.or_solver_step(1, 0.01, 0.9, 0.999, 1e-8, 0.0, 1, p, g, m, v, 3, out)
    # t=1: m_hat = g, v_hat = g^2 -> p - lr*g/(|g|+eps)
    np.testing.assert_allclose(out, p - 0.01 * g / (np.abs(g) + 1e-8), rtol=1e-5)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
    out_w = np.zeros(3, np.float32)
    oracle.or_solver_step(2, 0.01, 0.9, 0.999, 1e-8, 1e-4, 1, p, g, np.zeros(3, np.float32),
                          np.zeros(3, np.float32), 3, out_w)
    # AdamW adds +wd*p with no lr factor (noiser.rs:208-212)
    np.testing.assert_allclose(out_w - out, 1e-4 * p, rtol=1e-3)


def test_clip_global_norm_hand_computed(oracle):
    # noiser.rs:231-244 (optax clip_by_global_norm): scale = max_norm / ||g||
    # over all tensors together when the norm exceeds max_norm, else 1.
    assert O.clip_scale([np.array([3.0, 4.0])], 1.0) == pytest.approx(0.2, rel=1e-7)
    # the norm is global: [3] and [4] in separate tensors give the same 5
    assert O.clip_scale([np.array([3.0]), np.array([[4.0]])], 1.0) == pytest.approx(0.2, rel=1e-7)
    assert O.clip_scale([np.array([3.0, 4.0])], 10.0) == 1.0      # below the threshold
    assert O.clip_scale([np.array([3.0, 4.0])], 5.0) == 1.0       # equal: strict '>'
    assert O.clip_scale([np.zeros(7)], 0.0) == 1.0                # all zero: no division
    assert O.clip_scale([np.zeros(3), np.zeros(2)], 1.0) == 1.0
    # squares, not absolute values: ||[1, -1, 1, -1]|| = 2
    assert O.clip_scale([np.array([1.0, -1.0, 1.0, -1.0])], 1.0) == pytest.approx(0.5, rel=1e-7)
    g = np.random.default_rng(5).standard_normal(1000)
    assert O.clip_scale([g[:300], g[300:]], 1.0) == pytest.approx(1.0 / np.linalg.norm(g),
                                                                   rel=1e-6)


# ---- the ES gradient checker (eggroll.rs:353-404) -----------------------------

def test_lora_grad_f64_is_scaled_einsum(oracle):
    # or_lora_grad_f64 = -(sqrt(N)/N) * sum_i f_i A_i B_i^T over tids 0..N-1
    # (simple_lora_update's sum, eggroll.rs:353-404, with the SGD scale -g*sqrt(N)),
    # split over threads; must equal the pinned single-thread einsum for any split.
    rng = np.random.default_rng(11)
    for n, a, b, r in ((2, 3, 4, 1), (7, 5, 3, 2), (16, 6, 9, 4)):
        fit = rng.standard_normal(n).astype(np.float32)
        sigma, key = 0.4, 0x1234567 + n
        bs = oracle.or_base_sigma(sigma, r)
        ein = np.zeros((a, b), np.float64)
        oracle.or_lora_einsum_f64(bs, key, r, 0, 3, fit, np.arange(n, dtype=np.int32), n, a, b,
                                  ein)
        want = (ein * (-math.sqrt(n) / n)).astype(np.float32)
        for nt in (1, 3, 8):
            g = O.lora_grad_f64(sigma, key, r, 3, fit, a, b, nthreads=nt)
            np.testing.assert_allclose(g, want, rtol=1e-6, atol=1e-9)


def test_lora_grad_f64_hand_computed_pair(oracle):
    # N = 2, r = 1: members 0 and 1 share B and have A_1 = -A_0 (antithetic pair,
    # eggroll.rs:60-65), so g = -(sqrt(2)/2) * (f_0 - f_1) * A_0 B_0^T.
    sigma, key, a, b = 0.5, 99, 2, 3
    A, B = O.lora_factors(oracle.or_base_sigma(sigma, 1), key, 1, 0, [0], a, b)
    f0, f1 = 1.25, -0.5
    g = O.lora_grad_f64(sigma, key, 1, 0, np.array([f0, f1], np.float32), a, b, nthreads=2)
    outer = [[float(A[0, p, 0]) * float(B[0, q, 0]) for q in range(b)] for p in range(a)]
    want = np.array([[-(math.sqrt(2) / 2) * (f0 - f1) * v for v in row] for row in outer])
    np.testing.assert_allclose(g, want, rtol=1e-6)
    # a fitness shared by both members cancels exactly
    g0 = O.lora_grad_f64(sigma, key, 1, 0, np.array([0.7, 0.7], np.float32), a, b)
    assert np.all(g0 == 0.0)


# ---- whole SNN member forward (snn.rs:253-282, snn_mnist.rs:180-201) ---------

def _snn_cfg(dims, T, rows, sigma, rank, tau_m=10.0, v_th=1.0, seeds=(1, 2, 3, 4), epoch=0):
    c = O.SnnCfg()
    d = np.array(dims, np.int32)
    c.n_layers = len(dims) - 1
    c.dims = d.ctypes.data_as(ctypes.POINTER(O.c_i32))
    c.T, c.rows, c.tau_m, c.v_th, c.sigma = T, rows, tau_m, v_th, sigma
    c.rank, c.noise_reuse, c.epoch = rank, 0, epoch
    for i in range(4):
        c.poisson_seed[i] = seeds[i]
    return c, d


def _snn_member_oracle(oracle, c, W, keys, probs_m, labels_m, m):
    Ws = [np.ascontiguousarray(w, np.float32) for w in W]
    Wp = (ctypes.c_void_p * len(Ws))(*[w.ctypes.data for w in Ws])
    kk = (O.c_u64 * len(keys))(*keys)
    out = np.zeros(1, np.float32)
    oracle.or_snn_forward_member(ctypes.byref(c), Wp, kk, np.ascontiguousarray(probs_m, np.float32),
                                 np.ascontiguousarray(labels_m, np.int32), m, out)
    return float(out[0])


def _snn_member_composed(dims, T, rows, sigma, rank, tau_m, v_th, seeds, W, keys, probs_m,
                         labels_m, m, bs):
    # The member's Poisson streams use the global (row, col) index: encode the
    # m+1 members' rows with this member's rows last and keep those.
    pad = np.zeros(((m + 1) * rows, dims[0]), np.float32)
    pad[m * rows:] = probs_m
    x = O.poisson(pad, T, seeds)[:, m * rows:]                 # (T, R, in)
    hidden = []
    for l in range(len(dims) - 2):
        a, b = dims[l + 1], dims[l]
        A, B = O.lora_factors(bs, keys[l], rank, 0, [m], a, b)
        cur = O.do_mm(x.reshape(T * rows, b), W[l], A[0], B[0]).reshape(T, rows, a)
        x, _ = O.lif(cur, tau_m, v_th)
        hidden.append(x)
    rate = x.sum(axis=0, dtype=np.float32) / np.float32(T)      # T a power of two: exact
    a, b = dims[-1], dims[-2]
    A, B = O.lora_factors(bs, keys[-1], rank, 0, [m], a, b)
    logits = O.do_mm(rate, W[-1], A[0], B[0])
    ll = O.loglik(logits, labels_m).astype(np.float64)
    return float(np.float32(ll.sum() / rows)), hidden


def test_snn_forward_member_is_composition_of_pinned_pieces(oracle):
    dims, T, rows, sigma, rank = (12, 6, 5, 3), 8, 3, 0.3, 2
    seeds = (5, 6, 7, 8)
    rng = np.random.default_rng(4)
    W = [rng.standard_normal((dims[l + 1], dims[l])).astype(np.float32) * g
         for l, g in zip(range(3), (4.0, 6.0, 1.0))]
    keys = [(i + 1) * 0x9E3779B97F4A7C15 & M64 for i in range(3)]
    c, _d = _snn_cfg(dims, T, rows, sigma, rank, seeds=seeds)
    bs = oracle.or_base_sigma(sigma, rank)
    fits = []
    for m in (0, 1, 6):
        probs = rng.random((rows, dims[0])).astype(np.float32)
        probs[rng.random(probs.shape) < 0.3] = 0.0
        labels = rng.integers(0, dims[-1], rows).astype(np.int32)
        got = _snn_member_oracle(oracle, c, W, keys, probs, labels, m)
        want, hidden = _snn_member_composed(dims, T, rows, sigma, rank, 10.0, 1.0, seeds, W, keys,
                                            probs, labels, m, bs)
        assert got == want, (m, got, want)
        # every hidden layer fires, so each piece of the wiring reaches the fitness
        assert all(h.sum() > 0 for h in hidden), m
        # the member index reaches the factors and the Poisson streams: member
        # m+1's composition on the same rows gives another fitness
        other, _ = _snn_member_composed(dims, T, rows, sigma, rank, 10.0, 1.0, seeds, W, keys,
                                        probs, labels, m + 1, bs)
        assert other != got
        fits.append(got)
    assert all(abs(f + math.log(3.0)) > 1e-3 for f in fits)  # not the silent-readout value


def test_snn_forward_members_equals_per_member(oracle):
    # or_snn_forward_members indexes member m's rows and labels and keeps the
    # global Poisson index, for any thread count.
    dims, T, rows, sigma, rank, n = (10, 7, 4), 4, 2, 0.2, 3, 6
    rng = np.random.default_rng(8)
    W = [rng.standard_normal((dims[l + 1], dims[l])).astype(np.float32) * 4.0 for l in range(2)]
    keys = [11, 22]
    c, _d = _snn_cfg(dims, T, rows, sigma, rank)
    probs = rng.random((n * rows, dims[0])).astype(np.float32)
    labels = rng.integers(0, dims[-1], n * rows).astype(np.int32)
    per = [_snn_member_oracle(oracle, c, W, keys, probs[m * rows:(m + 1) * rows],
                              labels[m * rows:(m + 1) * rows], m) for m in range(n)]
    assert len(set(per)) == n  # the hidden layer fires: members differ
    Ws = [np.ascontiguousarray(w) for w in W]
    Wp = (ctypes.c_void_p * 2)(*[w.ctypes.data for w in Ws])
    kk = (O.c_u64 * 2)(*keys)
    for nt in (1, 4):
        fit = np.zeros(n - 1, np.float32)
        oracle.or_snn_forward_members(ctypes.byref(c), Wp, kk, probs, labels, 1, n, nt, fit)
        np.testing.assert_array_equal(fit, np.array(per[1:], np.float32))


def test_snn_forward_member_silent_model_closed_form(oracle):
    # Hidden weights 0 and sigma 0: no current, no spike, rates 0, logits 0 for
    # any readout weights, so every row's log-likelihood is -ln(classes).
    dims, T, rows = (9, 5, 4, 10), 8, 3
    rng = np.random.default_rng(1)
    W = [np.zeros((5, 9), np.float32), np.zeros((4, 5), np.float32),
         rng.standard_normal((10, 4)).astype(np.float32)]
    c, _d = _snn_cfg(dims, T, rows, 0.0, 2)
    probs = rng.random((rows, 9)).astype(np.float32)
    labels = np.array([0, 3, 9], np.int32)
    got = _snn_member_oracle(oracle, c, W, [1, 2, 3], probs, labels, 2)
    assert got == pytest.approx(-math.log(10.0), rel=1e-6)
