"""The split (fp32-accurate) forwards, HSES_MATH_F32X: every fp32 operand as an
fp16 high part plus the fp16 rounding of its remainder, fp16 MFMA products
accumulated in fp32.

* the split operand image (hses_pair_image_x) is the high/low split of the
  record's B rows and bs-scaled A rows in the kernel layout, zero padded;
* currents (hses_perturbed_linear_pre_x) against float64 evaluations of the
  reference product x W^T + (x B_m) A_m^T (or_batched_lora_noise's factors):
  within 4e-6 of sum |terms| per element, and at least 50x closer than the
  bf16 path on the same inputs (so the bound tells the two apart);
* spikes and rates (hses_perturbed_linear_lif_pre_x), and the spike-count
  bit planes (hses_perturbed_linear_lif_counts_pre_x), equal the oracle's LIF
  scan (snn.rs:53-97) of the split path's own currents, bit for bit (the
  kernels share the accumulators; the LIF is fp32 in both);
* the whole C3 step at N = 8192 in split mode: spike mismatches against the
  fp32 oracle (or_do_mm currents, or_lif_scan) per hidden layer, member
  fitness against the oracle on the GPU's own spikes, and the whole member
  forward (or_snn_forward_member, fp32 throughout) end to end.
"""
import numpy as np
import pytest
import torch

from hyperscalees_amd import kernels as K
from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAMW, FMT_BITS, MATH_BF16, MATH_F32X
from tests import oracle_lib as O
from tests.test_gpu_linear import pack_bits
from tests.test_gpu_record import pairs_of
from tests.test_gpu_snn import unpack

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 11 % 2**64
XSCALE = 1024.0


def swap23(c):
    return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1)


def split16(v):
    """float32 -> (fp16 high part, fp16 low part) as numpy float16 (RNE)."""
    v = np.asarray(v, np.float32)
    hi = v.astype(np.float16)
    lo = (v - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


def draw_split(a, b, r, sigma, tid_lo, n, epoch=0, nreuse=0):
    rec = K.factor_record(a, b, r, tid_lo, n)
    img = K.pair_image(a, b, r, tid_lo, n)
    K.pair_factors(KEY, r, sigma, epoch, nreuse, tid_lo, n, a, b, rec, img)
    imx = K.pair_image_x(a, b, r, tid_lo, n)
    imx.fill_(-1)  # 0xffff: a NaN pattern where the split must write
    K.split_pair_image(a, b, r, sigma, tid_lo, n, rec, imx)
    return rec, img, imx


@pytest.mark.parametrize("a,b,r,n,tid_lo", [
    (128, 784, 128, 4, 0),   # C3 fc1 shape
    (10, 128, 128, 5, 3),    # C3 readout shape, odd start and count
    (50, 200, 48, 2, 1),     # ragged widths, rank padded to 64 columns
])
def test_split_image_layout(hses_gpu, a, b, r, n, tid_lo):
    sigma = 0.02
    rec, _, imx = draw_split(a, b, r, sigma, tid_lo, n)
    torch.cuda.synchronize()
    P = pairs_of(tid_lo, n)
    kp = (b + 63) // 64 * 64
    be, ae = r * kp, a * 136
    stride = 2 * be + 2 * ae
    assert imx.numel() == P * stride
    recv = rec[: P * r * (a + b)].view(P, r, a + b).cpu().numpy()
    im = imx.view(P, stride).cpu().numpy().view(np.float16)
    bs = np.float32(sigma) / np.sqrt(np.float32(r))
    pos = np.array([swap23(c) for c in range(r)])
    rp32 = (r + 31) // 32 * 32
    for p in range(P):
        bh, bl = split16(recv[p, :, :b])
        np.testing.assert_array_equal(im[p, :be].reshape(r, kp)[:, :b], bh)
        np.testing.assert_array_equal(im[p, be:2 * be].reshape(r, kp)[:, :b], bl)
        assert not im[p, :2 * be].reshape(2, r, kp)[:, :, b:].any(), "padding columns"
        A = (recv[p, :, b:].T * bs).astype(np.float32) * np.float32(XSCALE)
        ah, al = split16(A)
        at = im[p, 2 * be:].reshape(2, a, 136)
        np.testing.assert_array_equal(at[0][:, pos], ah)
        np.testing.assert_array_equal(at[1][:, pos], al)
        assert not at[:, :, r:rp32].any(), "rank padding"
        # the split reproduces the fp32 value to ~2^-22
        full = recv[p, :, :b].astype(np.float64)
        back = bh.astype(np.float64) + bl.astype(np.float64)
        assert np.abs(back - full).max() <= 2.0 ** -21 * max(np.abs(full).max(), 1e-30)


@pytest.mark.parametrize("a,b,r,n,tid_lo", [
    (128, 784, 128, 6, 0),   # C3 fc1 shape
    (10, 128, 128, 5, 3),    # readout shape, half pairs at both ends
    (96, 200, 48, 4, 1),     # rank padding, ragged K
])
def test_pair_factors_x_draws_the_split_image(hses_gpu, a, b, r, n, tid_lo):
    # the draw into the split image keeps the same record and writes the
    # image hses_pair_image_x derives from that record, bit for bit
    sigma = 0.02
    rec, _, imx = draw_split(a, b, r, sigma, tid_lo, n)
    rec2 = K.factor_record(a, b, r, tid_lo, n)
    imx2 = K.pair_image_x(a, b, r, tid_lo, n)
    rec2.fill_(float("nan"))
    imx2.fill_(-1)
    K.pair_factors(KEY, r, sigma, 0, 0, tid_lo, n, a, b, rec2, imx2, split=True)
    torch.cuda.synchronize()
    assert torch.equal(rec2, rec)
    P = pairs_of(tid_lo, n)
    kp = (b + 63) // 64 * 64
    be, ae = r * kp, a * 136
    rp32 = (r + 31) // 32 * 32
    # every element the kernels read: B parts whole, A rows' first rp32 columns
    v1 = imx.view(P, 2 * be + 2 * ae)
    v2 = imx2.view(P, 2 * be + 2 * ae)
    assert torch.equal(v1[:, :2 * be], v2[:, :2 * be])
    assert torch.equal(v1[:, 2 * be:].reshape(P, 2 * a, 136)[:, :, :rp32],
                       v2[:, 2 * be:].reshape(P, 2 * a, 136)[:, :, :rp32])


def reference_currents(x, W, A, B, rows):
    """float64 currents (T, M, a) and sum |terms| for time-major x (T, M, b) of
    members with `rows` rows each; A (n, a, r) scaled and signed, B (n, b, r)."""
    T, M, b = x.shape
    n = M // rows
    xs = x.reshape(T, n, rows, b).astype(np.float64)
    W64 = W.astype(np.float64)
    y = xs @ W64.T
    scale = np.abs(xs) @ np.abs(W64).T
    for m in range(n):
        xb = xs[:, m] @ B[m].astype(np.float64)
        y[:, m] += xb @ A[m].astype(np.float64).T
        scale[:, m] += (np.abs(xs[:, m]) @ np.abs(B[m]).astype(np.float64)) @ np.abs(A[m]).astype(np.float64).T
    return y.reshape(T, M, -1), scale.reshape(T, M, -1)


CUR_CASES = [
    # a, b, r, n, tid_lo, rows, T
    (128, 784, 128, 8, 0, 4, 16),     # C3 fc1 shape
    (10, 128, 128, 7, 3, 3, 1),       # readout shape; odd start and count
    (50, 64, 32, 6, 1, 5, 2),         # one K tile
    (128, 200, 48, 130, 0, 2, 4),     # 65 pairs, ragged K
    (128, 784, 128, 128, 0, 32, 16),  # pairs split over 4 workgroups (64 pairs, 512 rows each)
]


@pytest.mark.parametrize("a,b,r,n,tid_lo,rows,T", CUR_CASES)
def test_pre_x_currents_fp32_accurate(hses_gpu, a, b, r, n, tid_lo, rows, T):
    rng = np.random.default_rng(a * 7 + b + r + n)
    sigma = 0.05
    xf = (rng.random((T, n * rows, b)) < 0.3).astype(np.float32)
    x = pack_bits(xf)
    W = (3.0 * rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    Wd = torch.from_numpy(W).cuda()
    rec, img, imx = draw_split(a, b, r, sigma, tid_lo, n)
    y = K.perturbed_linear(x, Wd, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_BITS,
                           n_time=T, math=MATH_F32X, rec=rec, img=imx)
    ybf = K.perturbed_linear(x, Wd, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_BITS,
                             n_time=T, math=MATH_BF16, rec=rec, img=img)
    torch.cuda.synchronize()
    bs = O.load().or_base_sigma(sigma, r)
    A, B = O.lora_factors(bs, KEY, r, 0, np.arange(tid_lo, tid_lo + n), a, b)
    ref, scale = reference_currents(xf, W, A, B, rows)
    got = y.cpu().numpy().reshape(T, n * rows, a).astype(np.float64)
    gbf = ybf.cpu().numpy().reshape(T, n * rows, a).astype(np.float64)
    err = (np.abs(got - ref) / np.maximum(scale, 1e-30)).max()
    err_bf = (np.abs(gbf - ref) / np.maximum(scale, 1e-30)).max()
    print(f"split max err {err:.2e} of sum|terms|, bf16 {err_bf:.2e}")
    assert np.isfinite(got).all()
    assert err <= 4e-6, f"split currents err {err:.2e}"
    assert err_bf >= 50 * err, f"bf16 {err_bf:.2e} vs split {err:.2e}: the bound does not discriminate"


LIF_CASES = [
    # a, b, r, n, tid_lo, rows, T, time_inner
    (128, 784, 128, 6, 0, 8, 16, True),     # C3 fc1 shape, time-inner
    (128, 128, 64, 5, 3, 8, 4, False),      # odd start and count, time-major
    (128, 784, 128, 128, 0, 32, 16, True),  # split over 4 workgroups
]


@pytest.mark.parametrize("a,b,r,n,tid_lo,rows,T,time_inner", LIF_CASES)
def test_lif_pre_x_equals_lif_of_its_currents(hses_gpu, a, b, r, n, tid_lo, rows, T, time_inner):
    rng = np.random.default_rng(a + b + r + n + T)
    sigma, tau, vth = 0.05, 10.0, 1.0
    xf = (rng.random((T, n * rows, b)) < 0.3).astype(np.float32)
    x_tm = pack_bits(xf)
    W = (12.0 * rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    Wd = torch.from_numpy(W).cuda()
    rec, _, imx = draw_split(a, b, r, sigma, tid_lo, n)
    y = K.perturbed_linear(x_tm, Wd, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_BITS,
                           n_time=T, math=MATH_F32X, rec=rec, img=imx)
    x = x_tm.transpose(0, 1).contiguous() if time_inner else x_tm
    spk, rate = K.perturbed_linear_lif(x, Wd, KEY, r, sigma, 0, 0, tid_lo, n, rows, T, tau, vth,
                                       want_spikes=True, want_rate=True, rec=rec, img=imx,
                                       time_inner=time_inner, math=MATH_F32X)
    torch.cuda.synchronize()
    cur = y.cpu().numpy().reshape(T, n * rows, a)
    ref_s, _ = O.lif(cur, tau, vth)
    s_tm = spk.transpose(0, 1) if time_inner else spk
    got = unpack(s_tm, a)
    assert ref_s.sum() > 0.02 * ref_s.size, "the layer is nearly silent"
    np.testing.assert_array_equal(got, ref_s)
    np.testing.assert_array_equal(rate.cpu().numpy(), ref_s.mean(0).astype(np.float32))
    counts = K.perturbed_linear_lif_counts_x(x, Wd, r, sigma, tid_lo, n, rows, T, tau, vth, rec,
                                             imx, time_inner=time_inner)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(decode_counts(counts, a), ref_s.sum(0))


def decode_counts(counts, a):
    """(M, P, words) count planes -> (M, a) counts."""
    planes = unpack(counts, a)  # (M, P, a)
    return sum(planes[:, p] * 2.0 ** p for p in range(planes.shape[1]))


def test_split_rejects_unsupported(hses_gpu):
    a, b, r, n, rows, T = 64, 1000, 32, 2, 4, 1  # b > 896: the split layout does not fit LDS
    rec = K.factor_record(a, b, r, 0, n)
    img = K.pair_image(a, b, r, 0, n)
    K.pair_factors(KEY, r, 0.05, 0, 0, 0, n, a, b, rec, img)
    imx = K.pair_image_x(a, b, r, 0, n)
    K.split_pair_image(a, b, r, 0.05, 0, n, rec, imx)
    x = pack_bits(np.zeros((T, n * rows, b), np.float32))
    W = torch.zeros((a, b), dtype=torch.float32, device="cuda")
    with pytest.raises(Exception, match="896"):
        K.perturbed_linear(x, W, KEY, r, 0.05, 0, 0, 0, n, rows, x_fmt=FMT_BITS, n_time=T,
                           math=MATH_F32X, rec=rec, img=imx)
    small = imx[: imx.numel() // 2]
    with pytest.raises(Exception, match="hses_pair_image_x_bytes"):
        K.perturbed_linear(x, W, KEY, r, 0.05, 0, 0, 0, n, rows, x_fmt=FMT_BITS, n_time=T,
                           math=MATH_F32X, rec=rec, img=small)
    torch.cuda.synchronize()


# ---- the C3 step in split mode ------------------------------------------------

C3X = dict(dims=(784, 128, 128, 128, 10), T=16, rows=64, n=8192, rank=128, sigma=0.02,
           tau_m=10.0, v_th=1.0, math=MATH_F32X, solver=ADAMW, lr=0.01,
           poisson_seed=(5, 6, 7, 8))
MEMBERS = (0, 1, 511, 512, 2047, 4095, 8190, 8191)
POOL = 60000


@pytest.fixture(scope="module")
def c3x_run(hses_gpu):
    cfg = snn.SnnConfig(**C3X)
    pool, labels = snn.synthetic_pool(POOL, cfg.dims[0], cfg.dims[-1], 0)
    idx = snn.sample_index(0, cfg.n, cfg.rows, POOL)
    W = snn.init_weights(cfg.dims, 0, gain=snn.ACTIVE_GAIN)
    es = snn.SnnEs(cfg, W, pool, labels, idx)
    assert es.fused and es.ahead and es.split
    assert es.mw and es.ro_counts and es.ppool is not None, "the benched C3 path"
    fit = es.forward(0)
    torch.cuda.synchronize()
    R = cfg.rows
    rows = np.concatenate([np.arange(m * R, (m + 1) * R) for m in MEMBERS])
    rows_t = torch.as_tensor(rows, device="cuda")
    spk = [unpack(es.spikes_tm(l).index_select(1, rows_t), cfg.dims[l]) for l in range(es.L - 1)]
    counts = decode_counts(es.cpl.index_select(0, rows_t), cfg.dims[-2])
    return dict(cfg=cfg, pool=pool, labels=labels, idx=idx, W=W, spk=spk, counts=counts,
                fit=fit.cpu().numpy().copy())


def test_c3_split_spikes_against_fp32_oracle(c3x_run):
    cfg, W, R = c3x_run["cfg"], c3x_run["W"], c3x_run["cfg"].rows
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    L = len(cfg.dims) - 1
    for l in range(L - 1):
        a, b = cfg.dims[l + 1], cfg.dims[l]
        A, B = O.lora_factors(bs, cfg.keys[l], cfg.rank, 0, np.array(MEMBERS), a, b)
        n_ref = mism = 0
        for j, m in enumerate(MEMBERS):
            x = c3x_run["spk"][l][:, j * R:(j + 1) * R]
            cur = O.do_mm(x.reshape(-1, b), W[l], A[j], B[j]).reshape(cfg.T, R, a)
            ref, _ = O.lif(cur, cfg.tau_m, cfg.v_th)
            if l < L - 2:
                got = c3x_run["spk"][l + 1][:, j * R:(j + 1) * R]
                mism += int((got != ref).sum())
            else:
                # the last hidden layer leaves spike counts: |count difference|
                # counts the flips that do not cancel within a (row, column)
                got = c3x_run["counts"][j * R:(j + 1) * R]
                mism += int(np.abs(got - ref.sum(0)).sum())
            n_ref += int(ref.sum())
        print(f"split layer {l}: {n_ref} reference spikes, {mism} mismatches against the "
              f"fp32 oracle ({mism / max(n_ref, 1):.2e})")
        assert n_ref > 0.03 * cfg.T * R * len(MEMBERS) * a, f"layer {l} is nearly silent"
        assert mism <= 1e-4 * n_ref, f"layer {l}: {mism} of {n_ref} against fp32"


def test_c3_split_fitness(c3x_run):
    # readout on the GPU's own last-layer spikes (their rate), fp32 oracle logits
    cfg, W, R = c3x_run["cfg"], c3x_run["W"], c3x_run["cfg"].rows
    bs = O.load().or_base_sigma(cfg.sigma, cfg.rank)
    a, b = cfg.dims[-1], cfg.dims[-2]
    A, B = O.lora_factors(bs, cfg.keys[-1], cfg.rank, 0, np.array(MEMBERS), a, b)
    worst = 0.0
    for j, m in enumerate(MEMBERS):
        rate = np.ascontiguousarray(c3x_run["counts"][j * R:(j + 1) * R] / cfg.T, np.float32)
        logits = O.do_mm(rate, W[-1], A[j], B[j])
        lab = c3x_run["labels"][c3x_run["idx"][m * R:(m + 1) * R]]
        ref = float(O.loglik(logits, lab).astype(np.float64).mean())
        rel = abs(float(c3x_run["fit"][m]) - ref) / abs(ref)
        worst = max(worst, rel)
        assert rel <= 1e-5, f"member {m}: fitness {c3x_run['fit'][m]} vs {ref}"
    print(f"split fitness on own spikes: worst rel difference {worst:.2e}")


def test_c3_split_member_forward_end_to_end(c3x_run):
    from tests.test_gpu_c3_full import oracle_cfg
    cfg, R = c3x_run["cfg"], c3x_run["cfg"].rows
    c, _dims = oracle_cfg(cfg)
    Ws = [np.ascontiguousarray(w) for w in c3x_run["W"]]
    Wp = (O.ctypes.c_void_p * len(Ws))(*[w.ctypes.data for w in Ws])
    keys = (O.c_u64 * len(cfg.keys))(*cfg.keys)
    worst = 0.0
    for m in MEMBERS:
        rows = c3x_run["idx"][m * R:(m + 1) * R]
        probs = np.ascontiguousarray(c3x_run["pool"][rows], np.float32)
        lab = np.ascontiguousarray(c3x_run["labels"][rows], np.int32)
        out = np.zeros(1, np.float32)
        O.load().or_snn_forward_member(O.ctypes.byref(c), Wp, keys, probs, lab, m, out)
        rel = abs(float(c3x_run["fit"][m]) - float(out[0])) / abs(float(out[0]))
        worst = max(worst, rel)
        assert rel <= 5e-3, f"member {m}: {c3x_run['fit'][m]} vs oracle {out[0]}"
    print(f"split end-to-end member fitness: worst rel difference {worst:.2e}")
