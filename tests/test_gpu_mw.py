"""Member weights: hses_member_weights forms W_m = W + sign_m (sigma/sqrt(r))
A_m B_m^T of every member from the factor record, and the forwards run
y = x W_m^T on them (hses_perturbed_linear_mw, hses_perturbed_linear_lif_mw).

* the weights against float64 W + A_m B_m^T (A, B from or_batched_lora_noise):
  fp16 high + low parts of 1024 W_m within 2^-20 of each element's sum of
  |terms|, bf16 within half a bf16 step of the float64 value (plus that) and
  equal to its bf16 rounding but for near-ties; padding columns zero; nothing
  written past the range's members;
* currents against float64 evaluations of the reference product x W^T +
  (x B_m) A_m^T: split within 4e-6 of sum |terms|, bf16 within 2^-7 of it;
* spikes, rates and spike-count planes of the fused LIF equal the oracle's LIF
  scan (snn.rs:53-97) of the same kernel's currents, bit for bit;
* whole SNN steps on member weights against the factored split forward
  (same record, both fp32-accurate): fitness within 1e-5, spikes equal but for
  near-threshold flips.
"""
import numpy as np
import pytest
import torch

from hyperscalees_amd import kernels as K
from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAMW, FMT_BITS, MATH_BF16, MATH_F32X, HsesError
from tests import oracle_lib as O
from tests.test_gpu_linear import bf16_round, pack_bits
from tests.test_gpu_snn import unpack
from tests.test_gpu_split import decode_counts, reference_currents

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 13 % 2**64


def record(a, b, r, sigma, tid_lo, n):
    rec = K.factor_record(a, b, r, tid_lo, n)
    rec.fill_(float("nan"))
    K.pair_factors(KEY, r, sigma, 0, 0, tid_lo, n, a, b, rec, None)
    return rec


def reference_weights(W, a, b, r, sigma, tid_lo, n):
    bs = O.load().or_base_sigma(sigma, r)
    A, B = O.lora_factors(bs, KEY, r, 0, np.arange(tid_lo, tid_lo + n), a, b)
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    Wm = W.astype(np.float64)[None] + np.einsum("mar,mbr->mab", A64, B64)
    # sum of |terms| of each element, the scale of its fp32 rounding error
    S = np.abs(W.astype(np.float64))[None] + np.einsum("mar,mbr->mab", np.abs(A64), np.abs(B64))
    return Wm, S, A, B


@pytest.mark.parametrize("a,b,r,n,tid_lo", [
    (128, 784, 128, 4, 0),   # C3 fc1 shape
    (128, 128, 64, 5, 3),    # odd start and count: a half pair at both ends
    (50, 200, 48, 3, 1),     # ragged widths, rank 48
])
def test_member_weights(hses_gpu, a, b, r, n, tid_lo):
    rng = np.random.default_rng(a + b + r)
    sigma = 0.05
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    Wd = torch.from_numpy(W).cuda()
    rec = record(a, b, r, sigma, tid_lo, n)
    kp = (b + 63) // 64 * 64
    wx = K.member_weights(Wd, r, sigma, tid_lo, n, rec, math=MATH_F32X)
    wb = K.member_weights(Wd, r, sigma, tid_lo, n, rec, math=MATH_BF16)
    torch.cuda.synchronize()
    Wm, S, _, _ = reference_weights(W, a, b, r, sigma, tid_lo, n)
    # chunk-major storage: [part][input chunk of 64][a][64]
    hx = wx.view(n, 2, kp // 64, a, 64).permute(0, 1, 3, 2, 4).reshape(n, 2, a, kp)
    hx = hx.cpu().numpy().view(np.float16).astype(np.float64)
    got = (hx[:, 0] + hx[:, 1])[:, :, :b] / 1024.0
    assert not hx[:, :, :, b:].any(), "padding columns"
    # fp32 accumulation over r products and the split's 2^-22, within 2^-20
    # of the element's sum of |terms|
    err = np.abs(got - Wm)
    assert (err <= 2.0 ** -20 * S).all(), f"split weights err {(err / S).max():.3e} of sum|terms|"
    gb = wb.view(n, kp // 64, a, 64).permute(0, 2, 1, 3).reshape(n, a, kp).cpu().numpy()
    gbf = (gb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)[:, :, :b]
    assert not gb[:, :, b:].any(), "padding columns"
    # rounding to bf16 from an fp32-accurate value: within half a step plus
    # the value's own error
    errb = np.abs(gbf - Wm)
    # (half a bf16 step: at most 2^-8 of the value, 8 significant bits)
    assert (errb <= 2.0 ** -8 * np.abs(Wm) + 2.0 ** -20 * S).all(), f"bf16 weights err {errb.max():.3e}"
    exact = bf16_round(Wm.astype(np.float32)).astype(np.float64)
    assert np.mean(gbf == exact) > 0.999


def test_member_weights_half_pair_untouched(hses_gpu):
    # tid_lo odd: the first pair's even member (tid_lo - 1) is not in the
    # range and has no slot; n odd: the last pair's odd member likewise
    a, b, r, n, tid_lo = 64, 128, 32, 3, 1
    rec = record(a, b, r, 0.05, tid_lo, n)
    W = torch.randn(a, b, device="cuda") * 0.1
    out = torch.full((K._lib.load().hses_member_weights_bytes(a, b, n + 1, MATH_F32X) // 2,),
                     -1, dtype=torch.int16, device="cuda")
    K.member_weights(W, r, 0.05, tid_lo, n, rec, math=MATH_F32X, out=out)
    torch.cuda.synchronize()
    kp = 128
    per = 2 * a * kp
    assert (out[: n * per] != -1).all(), "every member of the range is written"
    assert (out[n * per:] == -1).all(), "nothing past the range"


MW_CASES = [
    # a, b, r, n, tid_lo, rows, T
    (128, 784, 128, 8, 0, 16, 16),     # C3 fc1 shape
    (128, 128, 64, 5, 3, 64, 4),       # odd start and count
    (10, 128, 128, 6, 1, 32, 8),       # narrow output (one output tile)
    (128, 784, 128, 128, 0, 32, 16),   # pairs split over 4 workgroups (512 rows each)
    (64, 800, 32, 4, 0, 64, 4),        # last chunk 32 inputs: its first half streams alone
    (64, 801, 32, 4, 0, 64, 4),        # last chunk 33 inputs: both halves
]


@pytest.mark.parametrize("a,b,r,n,tid_lo,rows,T", MW_CASES)
def test_mw_currents(hses_gpu, a, b, r, n, tid_lo, rows, T):
    rng = np.random.default_rng(a * 3 + b + r + n)
    sigma = 0.05
    xf = (rng.random((T, n * rows, b)) < 0.3).astype(np.float32)
    x = pack_bits(xf)
    W = (3.0 * rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    Wd = torch.from_numpy(W).cuda()
    rec = record(a, b, r, sigma, tid_lo, n)
    wx = K.member_weights(Wd, r, sigma, tid_lo, n, rec, math=MATH_F32X)
    wb = K.member_weights(Wd, r, sigma, tid_lo, n, rec, math=MATH_BF16)
    yx = K.perturbed_linear_mw(x, wx, a, b, tid_lo, n, rows, n_time=T, math=MATH_F32X)
    yb = K.perturbed_linear_mw(x, wb, a, b, tid_lo, n, rows, n_time=T, math=MATH_BF16)
    torch.cuda.synchronize()
    _, _, A, B = reference_weights(W, a, b, r, sigma, tid_lo, n)
    ref, scale = reference_currents(xf, W, A, B, rows)
    gx = yx.cpu().numpy().reshape(T, n * rows, a).astype(np.float64)
    gb = yb.cpu().numpy().reshape(T, n * rows, a).astype(np.float64)
    ex = (np.abs(gx - ref) / np.maximum(scale, 1e-30)).max()
    eb = (np.abs(gb - ref) / np.maximum(scale, 1e-30)).max()
    print(f"member weights: split max err {ex:.2e} of sum|terms|, bf16 {eb:.2e}")
    assert np.isfinite(gx).all() and np.isfinite(gb).all()
    assert ex <= 4e-6, f"split currents err {ex:.2e}"
    assert eb <= 2.0 ** -7, f"bf16 currents err {eb:.2e}"


LIF_CASES = [
    # a, b, r, n, tid_lo, rows, T, time_inner, math
    (128, 784, 128, 6, 0, 16, 16, True, MATH_F32X),
    (128, 784, 128, 6, 0, 16, 16, True, MATH_BF16),
    (128, 128, 64, 5, 3, 64, 4, False, MATH_F32X),
    (128, 784, 128, 128, 0, 32, 16, True, MATH_F32X),  # split over 4 workgroups
    (32, 20, 32, 4, 0, 64, 4, True, MATH_F32X),        # one chunk of 20 inputs: two tiles
]


@pytest.mark.parametrize("a,b,r,n,tid_lo,rows,T,time_inner,math", LIF_CASES)
def test_lif_mw_equals_lif_of_its_currents(hses_gpu, a, b, r, n, tid_lo, rows, T, time_inner,
                                           math):
    rng = np.random.default_rng(a + b + r + n + T)
    sigma, tau, vth = 0.05, 10.0, 1.0
    xf = (rng.random((T, n * rows, b)) < 0.3).astype(np.float32)
    x_tm = pack_bits(xf)
    W = (12.0 * rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    Wd = torch.from_numpy(W).cuda()
    rec = record(a, b, r, sigma, tid_lo, n)
    wm = K.member_weights(Wd, r, sigma, tid_lo, n, rec, math=math)
    y = K.perturbed_linear_mw(x_tm, wm, a, b, tid_lo, n, rows, n_time=T, math=math)
    x = x_tm.transpose(0, 1).contiguous() if time_inner else x_tm
    spk, rate, _ = K.perturbed_linear_lif_mw(x, wm, a, b, tid_lo, n, rows, T, tau, vth, math=math,
                                             spikes=True, rate=True, time_inner=time_inner)
    _, _, counts = K.perturbed_linear_lif_mw(x, wm, a, b, tid_lo, n, rows, T, tau, vth,
                                             math=math, counts=True, time_inner=time_inner)
    torch.cuda.synchronize()
    cur = y.cpu().numpy().reshape(T, n * rows, a)
    ref_s, _ = O.lif(cur, tau, vth)
    assert ref_s.sum() > 0.02 * ref_s.size, "the layer is nearly silent"
    got = unpack(spk.transpose(0, 1) if time_inner else spk, a)
    np.testing.assert_array_equal(got, ref_s)
    np.testing.assert_array_equal(rate.cpu().numpy(), ref_s.mean(0).astype(np.float32))
    np.testing.assert_array_equal(decode_counts(counts, a), ref_s.sum(0))


def test_mw_validation(hses_gpu):
    a, b, r, n, rows, T = 64, 128, 32, 2, 64, 4
    rec = record(a, b, r, 0.05, 0, n)
    W = torch.zeros((a, b), dtype=torch.float32, device="cuda")
    wm = K.member_weights(W, r, 0.05, 0, n, rec, math=MATH_F32X)
    x = pack_bits(np.zeros((T, n * rows, b), np.float32))
    x24 = pack_bits(np.zeros((T, n * 24, b), np.float32))
    with pytest.raises(HsesError, match="multiple of 256"):
        K.perturbed_linear_mw(x24, wm, a, b, 0, n, 24, n_time=T, math=MATH_F32X)
    with pytest.raises(HsesError, match="hses_member_weights_bytes"):
        K.perturbed_linear_mw(x, wm[: wm.numel() // 2], a, b, 0, n, rows, n_time=T,
                              math=MATH_F32X)
    with pytest.raises((HsesError, ValueError), match="math"):
        K.member_weights(W, r, 0.05, 0, n, rec, math=0)
    x64 = pack_bits(np.zeros((T, n * rows, 64), np.float32))
    w64 = torch.zeros((a, 64), dtype=torch.float32, device="cuda")
    rec64 = record(a, 64, r, 0.05, 0, n)
    wb64 = K.member_weights(w64, r, 0.05, 0, n, rec64, math=MATH_BF16)
    with pytest.raises(HsesError, match="b > 64"):
        K.perturbed_linear_mw(x64, wb64, a, 64, 0, n, rows, n_time=T, math=MATH_BF16)
    torch.cuda.synchronize()


C3S = dict(dims=(784, 128, 128, 128, 10), T=16, rows=64, n=16, rank=128, sigma=0.02,
           tau_m=10.0, v_th=1.0, math=MATH_F32X, solver=ADAMW, lr=0.01, poisson_seed=(5, 6, 7, 8))


def make_weights(cfg, seed=0):
    return [torch.from_numpy(w).cuda() for w in snn.init_weights(cfg.dims, seed, gain=snn.ACTIVE_GAIN)]


def make(cfg, member_weights, seed=0, pool_size=3000):
    pool, labels = snn.synthetic_pool(pool_size, cfg.dims[0], cfg.dims[-1], seed)
    idx = snn.sample_index(seed, cfg.n, cfg.rows, pool_size)
    W = snn.init_weights(cfg.dims, seed, gain=snn.ACTIVE_GAIN)
    return snn.SnnEs(cfg, W, pool, labels, idx, member_weights=member_weights)


@pytest.mark.parametrize("extra", [dict(), dict(accumulate=2, solver=snn.SGD, lr=0.05),
                                   dict(n=9)])
def test_snn_steps_on_member_weights(hses_gpu, extra):
    # both forwards are fp32-accurate and differ only in rounding order, so a
    # spike flips only where a membrane potential lies within rounding of the
    # threshold: most members' fitness agrees to fp32 rounding, a flip moves
    # a member's by ~1e-4; gradients (same records, z-scores of the two
    # fitness vectors) follow.  One step each from the same parameters (a
    # second step would start from AdamW updates that amplify those
    # differences).
    cfg = snn.SnnConfig(**dict(C3S, **extra))
    es_f = make(cfg, member_weights=False)
    es_m = make(cfg, member_weights=True)
    assert es_m.mw and not es_f.mw
    for epoch in (0, 3):
        for es in (es_f, es_m):  # parameters reset between the two checks
            for w, w0 in zip(es.W, make_weights(cfg)):
                w.copy_(w0)
        f_f = es_f.step(epoch).clone()
        f_m = es_m.step(epoch).clone()
        torch.cuda.synchronize()
        rel = ((f_m - f_f).abs() / f_f.abs()).cpu().numpy()
        print(f"epoch {epoch}: fitness rel max {rel.max():.2e}, median {np.median(rel):.2e}")
        assert rel.max() <= 3e-3 and np.median(rel) <= 1e-5, f"epoch {epoch}: fitness"
        for l in range(1, es_f.L - 1):
            s_f, s_m = es_f.spikes_tm(l), es_m.spikes_tm(l)
            flips = int((s_f != s_m).sum())  # words that differ (each >= 1 flip)
            assert flips <= 1e-4 * s_f.numel() * 64, f"layer {l}: {flips} differing words"
        for l in range(es_f.L):
            err = (es_m.grads[l] - es_f.grads[l]).abs().max().item()
            assert err <= 5e-2 * es_f.grads[l].abs().max().item(), f"layer {l} gradient"


def pack_planes(counts, P, b, spare=0):
    """(M, b) counts -> (M, P + spare, words) uint64 bit planes (bit n of plane p =
    bit p of count n); spare plane rows filled with ones (must be ignored)."""
    M, wb = counts.shape[0], (b + 63) // 64
    out = np.zeros((M, P + spare, wb), np.uint64)
    out[:, P:] = np.uint64(2**64 - 1)
    for p in range(P):
        bits = ((counts >> p) & 1).astype(np.uint64)
        for c in range(b):
            out[:, p, c // 64] |= bits[:, c] << np.uint64(c % 64)
    return out


@pytest.mark.parametrize("a,b,r,n,tid_lo,rows,T", [
    (10, 128, 128, 6, 1, 64, 16),   # the C3 readout shape; half pairs at both ends
    (10, 128, 128, 8, 0, 64, 16),
    (32, 100, 48, 5, 2, 20, 8),     # ragged input width, odd count, rank 48
    (3, 64, 32, 2, 0, 128, 1),      # one plane, the most rows per member
])
def test_readout_counts(hses_gpu, a, b, r, n, tid_lo, rows, T):
    # hses_perturbed_readout_counts against float64: rate (W + A_m B_m^T)^T
    # with rate = count / T decoded from the planes
    rng = np.random.default_rng(a + b + r + n + rows)
    sigma = 0.05
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    Wd = torch.from_numpy(W).cuda()
    rec = record(a, b, r, sigma, tid_lo, n)
    M, P = n * rows, K.count_planes(T)
    counts = rng.integers(0, T + 1, (M, b))
    cpl = torch.from_numpy(pack_planes(counts, P, b, spare=1).view(np.int64)).cuda()
    got = K.readout_counts(cpl, Wd, r, sigma, tid_lo, n, rows, T, rec).cpu().numpy()
    Wm, S, _, _ = reference_weights(W, a, b, r, sigma, tid_lo, n)
    rate = counts.astype(np.float64) / T
    for m in range(n):
        sl = slice(m * rows, (m + 1) * rows)
        ref = rate[sl] @ Wm[m].T
        scale = rate[sl] @ S[m].T + 1e-30
        err = np.abs(got[sl] - ref) / scale
        assert err.max() <= 4e-6, f"member {m}: err {err.max():.2e} of sum|terms|"


def test_readout_counts_rejects(hses_gpu):
    a, b, r, n = 40, 128, 32, 2  # a > 32
    rec = record(a, b, r, 0.05, 0, n)
    W = torch.zeros(a, b, device="cuda")
    cpl = torch.zeros((n * 4, 5, 2), dtype=torch.int64, device="cuda")
    with pytest.raises(HsesError, match="a <= 32"):
        K.readout_counts(cpl, W, r, 0.05, 0, n, 4, 16, rec)
