"""GPU parity of the Poisson and LIF kernels (bit-exact) and of the fitness,
z-score and solver kernels (tolerance) against the oracle."""
import numpy as np
import pytest
import torch

from hyperscalees_amd._lib import (ADAM, ADAMW, FMT_BF16, FMT_BITS, FMT_F32, FMT_U8,
                                   REWARD_BINARY, REWARD_LOGLIK, SGD)
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu


def sparse_intensities(rng, rows, d, zero_frac=0.7):
    p = rng.random((rows, d)).astype(np.float32)
    p[rng.random((rows, d)) < zero_frac] = 0.0
    return p


def unpack_bits(words, width):
    w = words.cpu().numpy().view(np.uint64)
    bits = ((w[..., None] >> np.arange(64, dtype=np.uint64)) & np.uint64(1)).astype(np.float32)
    return bits.reshape(*w.shape[:-1], -1)[..., :width]


@pytest.mark.parametrize("rows,d,T", [(64, 784, 8), (37, 100, 16), (5, 1, 3), (256, 784, 16)])
def test_poisson_bit_exact_all_formats(hses_gpu, rows, d, T):
    rng = np.random.default_rng(rows * 7 + d)
    p = sparse_intensities(rng, rows, d)
    p[0, :min(d, 4)] = [0.0, 1.0, 0.5, 2.0][:min(d, 4)]
    seeds = (11, 22, 33, 44)
    ref = O.poisson(p, T, seeds)
    pt = torch.from_numpy(p).cuda()
    got = hses_gpu.poisson_encode(pt, T, seeds, FMT_F32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    bf = hses_gpu.poisson_encode(pt, T, seeds, FMT_BF16)
    np.testing.assert_array_equal(bf.float().cpu().numpy(), ref)
    u8 = hses_gpu.poisson_encode(pt, T, seeds, FMT_U8)
    np.testing.assert_array_equal(u8.cpu().numpy().astype(np.float32), ref)
    bits = hses_gpu.poisson_encode(pt, T, seeds, FMT_BITS)
    np.testing.assert_array_equal(unpack_bits(bits, d), ref)


@pytest.mark.parametrize("rows,d,T,zero_frac", [
    (9, 130, 1, 0.7), (6, 200, 2, 0.7), (11, 257, 4, 0.5), (7, 300, 32, 0.7),
    (5, 2048, 16, 0.7), (3, 2049, 16, 0.7),   # largest zero-skipping row, first fallback row
    (13, 784, 8, 0.0), (13, 784, 16, 1.0),     # every element active; every element zero
])
def test_poisson_bits_zero_skip(hses_gpu, rows, d, T, zero_frac):
    # Bit-packed rows: zero-skipping kernel for power-of-two T (rows of all
    # ones and all zeros included), streamed kernel beyond its row width.
    rng = np.random.default_rng(rows * 13 + d + T)
    p = sparse_intensities(rng, rows, d, zero_frac)
    p[1, :] = 1.0
    p[2, ::3] = 0.0
    seeds = (5, 6, 7, 8)
    ref = O.poisson(p, T, seeds)
    bits = hses_gpu.poisson_encode(torch.from_numpy(p).cuda(), T, seeds, FMT_BITS)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(unpack_bits(bits, d), ref)
    # gathered rows: output row i encodes p[idx[i]] seeded by its own flat index
    idx = rng.integers(0, rows, 2 * rows).astype(np.int32)
    got = hses_gpu.poisson_encode(torch.from_numpy(p).cuda(), T, seeds, FMT_BITS,
                                  rows_index=torch.from_numpy(idx).cuda())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(unpack_bits(got, d), O.poisson(p[idx], T, seeds))


@pytest.mark.parametrize("rows,d,T,fmt", [
    (37, 784, 16, FMT_BITS),   # zero-skipping kernel (the C3 input)
    (9, 300, 8, FMT_BITS),
    (5, 130, 40, FMT_BITS),    # T not a power of two: one wave per row
    (6, 70, 5, FMT_F32),       # element formats
    (4, 33, 3, FMT_U8),
])
def test_poisson_time_inner_layout(hses_gpu, rows, d, T, fmt):
    """hses_poisson_encode_planes with the time-inner layout (rows, T, width)
    stores the same spikes as the time-major layout, and the time-major call
    through it equals hses_poisson_encode."""
    rng = np.random.default_rng(rows * 3 + d)
    p = rng.random((rows, d)).astype(np.float32)
    p[rng.random(p.shape) < 0.5] = 0.0
    pt = torch.from_numpy(p).cuda()
    seeds = (7, 8, 9, 10)
    tm = hses_gpu.poisson_encode(pt, T, seeds, fmt)
    ti = hses_gpu.poisson_encode(pt, T, seeds, fmt, time_inner=True)
    torch.cuda.synchronize()
    assert torch.equal(ti.transpose(0, 1), tm)
    ref = O.poisson(p, T, seeds)
    got = tm.cpu().numpy()
    if fmt == FMT_BITS:
        w = got.view(np.uint64)
        got = ((w[..., None] >> np.arange(64, dtype=np.uint64)) & np.uint64(1)).reshape(T, rows, -1)[..., :d]
    np.testing.assert_array_equal(np.asarray(got, np.float32), ref)


def test_poisson_threshold_dense_p_sweep(hses_gpu):
    # Every representable neighbourhood of many thresholds: p on a fine grid
    # plus its f32 neighbours, checked against the f32-division formula.
    base = np.linspace(0, 1, 4001, dtype=np.float32)
    p = np.concatenate([base, np.nextafter(base, 2), np.nextafter(base, -1)]).astype(np.float32)
    p = np.tile(p, 4)[: (p.size * 4 // 100) * 100].reshape(-1, 100)
    ref = O.poisson(p, 12, (1, 2, 3, 5))
    got = hses_gpu.poisson_encode(torch.from_numpy(p).cuda(), 12, (1, 2, 3, 5))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


# Rows of a multiple of 64 columns take the 16-byte-load kernel (four
# (row, word) items per wave; 7 and 15 items leave a partial last wave), others
# the one-column-per-lane kernel; T = 37 and 20 scan several 16-step chunks.
@pytest.mark.parametrize("T,M,h,tau,vth", [(8, 64, 128, 10.0, 1.0), (16, 33, 100, 20.0, 0.3),
                                           (5, 3, 1, 10.0, -1e9), (16, 512, 128, 10.0, 1.0),
                                           (37, 5000, 128, 10.0, 1.0), (20, 3000, 200, 5.0, 0.5),
                                           (12, 7, 64, 4.0, 0.8), (9, 5, 192, 10.0, 1.0)])
def test_lif_bit_exact(hses_gpu, T, M, h, tau, vth):
    rng = np.random.default_rng(T * 1000 + h)
    cur = (rng.standard_normal((T, M, h)) * 1.5 + 0.4).astype(np.float32)
    v0 = (rng.standard_normal((M, h)) * 0.3).astype(np.float32)
    ref_s, ref_v = O.lif(cur, tau, vth, v0)
    ct = torch.from_numpy(cur).cuda()
    vt = torch.from_numpy(v0).cuda()
    s, v = hses_gpu.lif_scan(ct, tau, vth, v0=vt, fmt=FMT_F32, want_v=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), ref_s)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ref_v.view(np.uint32))
    bits = hses_gpu.lif_scan(ct, tau, vth, v0=vt, fmt=FMT_BITS)
    np.testing.assert_array_equal(unpack_bits(bits, h), ref_s)
    bf = hses_gpu.lif_scan(ct, tau, vth, v0=vt, fmt=FMT_BF16)
    np.testing.assert_array_equal(bf.float().cpu().numpy(), ref_s)
    u8 = hses_gpu.lif_scan(ct, tau, vth, v0=vt, fmt=FMT_U8)
    np.testing.assert_array_equal(u8.cpu().numpy().astype(np.float32), ref_s)


def test_lif_zero_v0_default(hses_gpu):
    cur = np.full((6, 2, 3), 2.0, np.float32)
    ref_s, _ = O.lif(cur, 10.0, 1.0)
    s = hses_gpu.lif_scan(torch.from_numpy(cur).cuda(), 10.0, 1.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), ref_s)


@pytest.mark.parametrize("n,rpm", [(40, 16), (9, 200), (5, 1), (6, 64)])
def test_member_loglik(hses_gpu, n, rpm):
    rng = np.random.default_rng(5 + rpm)
    c = 10
    logits = (rng.standard_normal((n * rpm, c)) * 3).astype(np.float32)
    labels = rng.integers(0, c, n * rpm).astype(np.int32)
    ref = O.loglik(logits, labels).reshape(n, rpm).astype(np.float64).mean(1)
    got = hses_gpu.member_loglik(torch.from_numpy(logits).cuda(), torch.from_numpy(labels).cuda(),
                                 n, rpm)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("reward", [REWARD_LOGLIK, REWARD_BINARY])
@pytest.mark.parametrize("c", [10, 256, 100])   # per-lane rows; wide rows (lanes over classes)
def test_member_fitness_rewards_and_correct_count(hses_gpu, reward, c):
    # fitness_from_logits_reward (snn_mnist.rs:180-201) per reward kind, member
    # means, and the argmax == label counter (first maximal class on ties).
    rng = np.random.default_rng(11 + reward + c)
    n, rpm = 37, 70
    logits = np.round(rng.standard_normal((n * rpm, c)) * 2).astype(np.float32)  # many ties
    labels = rng.integers(0, c, n * rpm).astype(np.int32)
    hit = (logits.argmax(1) == labels)
    if reward == REWARD_BINARY:
        ref = hit.astype(np.float64).reshape(n, rpm).mean(1)
    else:
        ref = O.loglik(logits, labels).reshape(n, rpm).astype(np.float64).mean(1)
    correct = torch.full((1,), 5, dtype=torch.int64, device="cuda")
    got = hses_gpu.member_fitness(torch.from_numpy(logits).cuda(), torch.from_numpy(labels).cuda(),
                                  n, rpm, reward, correct=correct)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    assert int(correct) == 5 + int(hit.sum())


def test_fitness_moments_and_combine_affine(hses_gpu):
    # accumulate_train.rs:843-846, 940-944 and combine_affine_grads
    # (eggroll.rs:902-915): sums over two chunks, then the affine combination
    # against the oracle's with the driver's f32 mean/std formulas.
    rng = np.random.default_rng(12)
    raw = (rng.standard_normal(3000) * 2 + 0.7).astype(np.float32)
    g = rng.standard_normal(4097).astype(np.float32)
    o = rng.standard_normal(4097).astype(np.float32)
    mom = torch.empty(2, dtype=torch.float64, device="cuda")
    hses_gpu.fitness_moments(torch.from_numpy(raw[:1234]).cuda(), mom)
    hses_gpu.fitness_moments(torch.from_numpy(raw[1234:]).cuda(), mom, accumulate=True)
    torch.cuda.synchronize()
    s1 = raw.astype(np.float64).sum()
    s2 = (raw * raw).astype(np.float64).sum()
    np.testing.assert_allclose(mom.cpu().numpy(), [s1, s2], rtol=1e-12)
    batch = raw.size
    mean = np.float32(np.float32(s1) / np.float32(batch))
    var = max(np.float32(np.float32(s2) / np.float32(batch)) - mean * mean, np.float32(0))
    std = np.float32(np.sqrt(np.float32(var + np.float32(1e-5))))
    for ones in (o, None):
        ref = np.zeros_like(g)
        O.load().or_combine_affine(g, o if ones is not None else np.zeros_like(g), g.size, mean,
                                   std, batch, ref)
        got = hses_gpu.combine_affine(torch.from_numpy(g).cuda(), mom, batch,
                                      ones_acc=None if ones is None else torch.from_numpy(o).cuda())
        torch.cuda.synchronize()
        np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("group", [0, 4])
def test_convert_fitnesses(hses_gpu, group):
    raw = np.random.default_rng(9).standard_normal(8192).astype(np.float32) * 3 + 1
    ref, m, s = O.convert_fitnesses(raw, group)
    out, stats = hses_gpu.convert_fitnesses(torch.from_numpy(raw).cuda(), group)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(stats.cpu().numpy(), [m, s], rtol=1e-6)


@pytest.mark.parametrize("kind", [SGD, ADAM, ADAMW])
def test_solver_step(hses_gpu, kind):
    rng = np.random.default_rng(kind)
    n = 1000
    p = rng.standard_normal(n).astype(np.float32)
    m = rng.standard_normal(n).astype(np.float32) * 0.1
    v = np.abs(rng.standard_normal(n).astype(np.float32)) * 0.01
    for step in (1, 2, 7):
        g = rng.standard_normal(n).astype(np.float32)
        ref = np.zeros_like(p)
        rm, rv = m.copy(), v.copy()
        O.load().or_solver_step(kind, 0.01, 0.9, 0.999, 1e-8, 1e-4, step, p, g, rm, rv, n, ref)
        pt, mt, vt = (torch.from_numpy(a.copy()).cuda() for a in (p, m, v))
        hses_gpu.solver_step(kind, 0.01, pt, torch.from_numpy(g).cuda(), mt, vt, step_t=step,
                             wd=1e-4)
        torch.cuda.synchronize()
        np.testing.assert_allclose(pt.cpu().numpy(), ref, rtol=1e-6, atol=1e-7)
        if kind != SGD:
            np.testing.assert_allclose(mt.cpu().numpy(), rm, rtol=1e-6, atol=1e-8)
        p, m, v = ref, rm, rv


def special_pool(rng, rows, d):
    """Sparse intensities with every class of element: exact zeros, negative,
    NaN, too small to fire, exact and over-one saturation, just below one."""
    p = sparse_intensities(rng, rows, d)
    specials = np.array([0.0, -0.5, np.nan, 1e-9, 1e-7, 1.0, 2.0, np.inf,
                         np.nextafter(np.float32(1.0), np.float32(0.0)), 0.5], np.float32)
    mask = rng.random((rows, d)) < 0.1
    p[mask] = rng.choice(specials, int(mask.sum()))
    p[0, :] = 1.0        # a fully saturated row
    if rows > 1:
        p[1, :] = 0.0    # a silent row
    return p


@pytest.mark.parametrize("pool_rows,d,T,time_inner", [
    (300, 784, 16, True),    # the C3 input: 784 = 12 words + 16 columns
    (300, 784, 16, False),
    (40, 100, 8, True),
    (17, 64, 32, False),     # one word per row, T = 32
    (9, 200, 1, True),
    (25, 2048, 4, False),    # widest prepared row
])
def test_poisson_pool_equals_encode(hses_gpu, pool_rows, d, T, time_inner):
    # the prepared pool's gathered encode == the direct gathered encode, bit
    # for bit, and == the oracle's spikes
    rng = np.random.default_rng(pool_rows + d + T)
    p = special_pool(rng, pool_rows, d)
    pt = torch.from_numpy(p).cuda()
    pool = hses_gpu.PoissonPool(pt)
    idx = rng.integers(0, pool_rows, 3 * pool_rows).astype(np.int32)
    idx[:3] = [0, 1, pool_rows - 1]
    idx[5] = -1             # outside the pool: all-zero rows
    idx[7] = pool_rows
    it = torch.from_numpy(idx).cuda()
    seeds = (11, 22, 33, 44)
    got = hses_gpu.poisson_encode_pool(pool, T, seeds, rows_index=it, time_inner=time_inner)
    ref = hses_gpu.poisson_encode(pt, T, seeds, FMT_BITS, rows_index=it, time_inner=time_inner)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    bits = unpack_bits(got.transpose(0, 1) if time_inner else got, d)
    safe = np.where((idx >= 0) & (idx < pool_rows), idx, 0)
    want = O.poisson(p[safe], T, seeds)
    want[:, (idx < 0) | (idx >= pool_rows), :] = 0.0
    np.testing.assert_array_equal(bits, want)
    # without a row index: output row i encodes pool row i
    got = hses_gpu.poisson_encode_pool(pool, T, seeds, time_inner=time_inner)
    ref = hses_gpu.poisson_encode(pt, T, seeds, FMT_BITS, time_inner=time_inner)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_poisson_pool_c3_batch(hses_gpu):
    # the C3 batch: 8192 members x 64 rows from a 60000 x 784 pool, both
    # encodes over all 524288 rows
    from hyperscalees_amd import snn
    pool, _ = snn.synthetic_pool(60000, 784, 10, seed=3)
    idx = snn.sample_index(0, 8192, 64, 60000)
    pt = torch.from_numpy(pool).cuda()
    it = torch.as_tensor(idx, dtype=torch.int32).cuda()
    pp = hses_gpu.PoissonPool(pt)
    got = hses_gpu.poisson_encode_pool(pp, 16, (1, 2, 3, 4), rows_index=it, time_inner=True)
    ref = hses_gpu.poisson_encode(pt, 16, (1, 2, 3, 4), FMT_BITS, rows_index=it, time_inner=True)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert int(ref.ne(0).sum()) > 0


def test_poisson_pool_rejects(hses_gpu):
    pt = torch.rand(4, 3000, device="cuda")
    with pytest.raises(ValueError, match="2048"):
        hses_gpu.PoissonPool(pt)
    pool = hses_gpu.PoissonPool(torch.rand(4, 100, device="cuda"))
    from hyperscalees_amd import _lib
    with pytest.raises(_lib.HsesError, match="power of two"):
        hses_gpu.poisson_encode_pool(pool, 12)
