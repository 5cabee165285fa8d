"""Factors drawn ahead: hses_pair_factors draws every pair's factors into the
factor record and the bf16 B operand image, and the *_pre forwards read them
instead of drawing.

Pinned against the generating forwards, which the oracle pins elsewhere
(test_gpu_linear, test_gpu_snn, test_gpu_c3_full): the record hses_pair_factors
writes equals the one the *_rec forwards keep, the image is the bf16 rounding
of the record's B rows and scaled A rows in their kernel layouts with zero
padding, and the *_pre forwards' spikes,
rates and currents equal the *_rec forwards' bit for bit (same operands,
products and order), also inside whole SNN steps."""
import numpy as np
import pytest
import torch

from hyperscalees_amd import kernels as K
from hyperscalees_amd import snn
from hyperscalees_amd._lib import FMT_BITS, FMT_F32, MATH_BF16, SGD, HsesError
from tests.test_gpu_linear import pack_bits
from tests.test_gpu_record import C3_SMALL, pairs_of

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15 * 7 % 2**64


def draw(a, b, r, sigma, epoch, nreuse, tid_lo, n):
    rec = K.factor_record(a, b, r, tid_lo, n)
    img = K.pair_image(a, b, r, tid_lo, n)
    rec.fill_(float("nan"))
    img.fill_(-1)  # 0xffff: a NaN pattern where the draw must write
    K.pair_factors(KEY, r, sigma, epoch, nreuse, tid_lo, n, a, b, rec, img)
    return rec, img


def swap23(c):
    return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1)


def check_image(rec, img, a, b, r, sigma, tid_lo, n):
    """Per pair: B^T as [c][kp] (bf16 of the raw normal, zero for k >= b), then
    A as [o][swap23(c)] rows of 136 (bf16 of normal * sigma / sqrt(r), zero
    for rank columns [r, r rounded up to 32))."""
    P = pairs_of(tid_lo, n)
    kp = (b + 63) // 64 * 64
    stride = r * kp + a * 136
    assert img.numel() == P * stride
    recv = rec[: P * r * (a + b)].view(P, r, a + b)
    im = img.view(P, stride)
    bt = im[:, : r * kp].view(P, r, kp)
    want = recv[:, :, :b].to(torch.bfloat16).view(torch.int16)  # do_mm: B unscaled, RNE
    assert torch.equal(bt[:, :, :b], want)
    assert not bt[:, :, b:].any(), "padding columns must be zero"
    bs = torch.tensor(np.float32(sigma) / np.sqrt(np.float32(r)), device=rec.device)
    at = im[:, r * kp:].view(P, a, 136)
    pos = torch.tensor([swap23(c) for c in range(r)], device=rec.device)
    wantA = (recv[:, :, b:].transpose(1, 2) * bs).to(torch.bfloat16).view(torch.int16)
    assert torch.equal(at[:, :, pos], wantA)
    rp32 = (r + 31) // 32 * 32
    assert not at[:, :, r:rp32].any(), "rank padding must be zero"


@pytest.mark.parametrize("a,b,r,n,tid_lo,T,epoch,nreuse", [
    (128, 784, 128, 6, 0, 16, 0, 0),    # C3 fc1 shape, three pairs, 48 padding columns
    (128, 128, 64, 5, 3, 4, 2, 0),      # odd start and count: half pairs at both ends
    (96, 200, 48, 4, 1, 2, 1, 3),       # rank 48 (A padded to 64 columns), noise reuse
    (128, 128, 128, 9, 0, 16, 1, 1),    # C3 fc2 shape, odd count
])
def test_lif_pre_equals_rec(hses_gpu, a, b, r, n, tid_lo, T, epoch, nreuse):
    rng = np.random.default_rng(a + b + r + n)
    rows, sigma = 8, 0.05
    x = pack_bits((rng.random((T, n * rows, b)) < 0.3).astype(np.float32))
    gain = 3.0 if T >= 4 else 12.0  # short series need larger currents to fire
    W = torch.from_numpy((gain * rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)).cuda()
    rec0 = K.factor_record(a, b, r, tid_lo, n)
    s0, q0 = K.perturbed_linear_lif(x, W, KEY, r, sigma, epoch, nreuse, tid_lo, n, rows, T, 10.0,
                                    1.0, want_spikes=True, want_rate=True, rec=rec0)
    s0, q0 = s0.clone(), q0.clone()
    rec, img = draw(a, b, r, sigma, epoch, nreuse, tid_lo, n)
    torch.cuda.synchronize()
    assert torch.equal(rec, rec0), "record of the draw differs from the forward's"
    check_image(rec, img, a, b, r, sigma, tid_lo, n)
    s1, q1 = K.perturbed_linear_lif(x, W, KEY, r, sigma, epoch, nreuse, tid_lo, n, rows, T, 10.0,
                                    1.0, want_spikes=True, want_rate=True, rec=rec, img=img)
    torch.cuda.synchronize()
    assert s0.any(), "no spikes: the case checks nothing"
    assert torch.equal(s0, s1) and torch.equal(q0, q1)


@pytest.mark.parametrize("a,b,r,n,tid_lo,T", [
    (128, 784, 128, 4, 0, 16),     # k_pair_bits storing currents
    (64, 300, 32, 5, 1, 1),
])
def test_bits_currents_pre_equal_rec(hses_gpu, a, b, r, n, tid_lo, T):
    rng = np.random.default_rng(a * 3 + b + n)
    rows, sigma = 16, 0.05
    x = pack_bits((rng.random((T, n * rows, b)) < 0.3).astype(np.float32))
    W = torch.from_numpy((rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)).cuda()
    rec0 = K.factor_record(a, b, r, tid_lo, n)
    y0 = K.perturbed_linear(x, W, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_BITS,
                            n_time=T, math=MATH_BF16, rec=rec0).clone()
    rec, img = draw(a, b, r, sigma, 0, 0, tid_lo, n)
    y1 = K.perturbed_linear(x, W, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_BITS,
                            n_time=T, math=MATH_BF16, rec=rec, img=img)
    torch.cuda.synchronize()
    assert torch.equal(rec, rec0)
    assert torch.equal(y0, y1)


@pytest.mark.parametrize("a,b,r,n,tid_lo", [
    (10, 128, 128, 6, 0),     # C3 readout on rates (pairs in groups of 12)
    (40, 96, 32, 7, 2),       # several pairs per group, four W column tiles
    (10, 128, 128, 27, 1),    # a group split over the grid, odd ends
    (12, 256, 32, 5, 1),      # four K tiles of fp32 x loaded a sub-step ahead
])
def test_dense_pre_equals_rec(hses_gpu, a, b, r, n, tid_lo):
    rng = np.random.default_rng(a * b + n)
    rows, sigma = 16, 0.02
    x = torch.from_numpy(rng.random((n * rows, b)).astype(np.float32)).cuda()
    W = torch.from_numpy((rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)).cuda()
    rec0 = K.factor_record(a, b, r, tid_lo, n)
    y0 = K.perturbed_linear(x, W, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_F32,
                            math=MATH_BF16, rec=rec0).clone()
    rec, img = draw(a, b, r, sigma, 0, 0, tid_lo, n)
    y1 = K.perturbed_linear(x, W, KEY, r, sigma, 0, 0, tid_lo, n, rows, x_fmt=FMT_F32,
                            math=MATH_BF16, rec=rec, img=img)
    torch.cuda.synchronize()
    assert torch.equal(rec, rec0)
    check_image(rec, img, a, b, r, sigma, tid_lo, n)
    assert torch.equal(y0, y1)


def make(cfg, ahead, seed=0, pool_size=3000):
    pool, labels = snn.synthetic_pool(pool_size, cfg.dims[0], cfg.dims[-1], seed)
    idx = snn.sample_index(seed, cfg.n, cfg.rows, pool_size)
    W = snn.init_weights(cfg.dims, seed, gain=snn.ACTIVE_GAIN)
    # the factored forward (member weights would change the arithmetic)
    return snn.SnnEs(cfg, W, pool, labels, idx, fused=True, record=True, ahead=ahead,
                     member_weights=False)


@pytest.mark.parametrize("extra,epochs", [
    (dict(), (0, 1, 2)),
    (dict(accumulate=2, solver=SGD, lr=0.05), (0, 1, 2)),             # two chunks per step
    (dict(n=9, solver=SGD, lr=0.05), (0, 1, 2)),
    (dict(noise_reuse=1, solver=SGD, lr=0.05), (0, 1, 2, 3)),          # fresh noise every epoch
    (dict(noise_reuse=1), (0, 1, 5, 6, 6)),                           # skipped / repeated epochs
    (dict(n=130, solver=SGD, lr=0.05), (0, 1)),    # 65 pairs: each pair split over 4 workgroups
])
def test_snn_steps_drawn_ahead_equal_drawn_inline(hses_gpu, extra, epochs):
    cfg = dict(C3_SMALL, **extra)
    es_i = make(snn.SnnConfig(**cfg), ahead=False)
    es_a = make(snn.SnnConfig(**cfg), ahead=True)
    assert es_a.img is not None and es_i.img is None
    for epoch in epochs:
        f_i = es_i.step(epoch).clone()
        f_a = es_a.step(epoch).clone()
        torch.cuda.synchronize()
        assert torch.equal(f_i, f_a), f"fitness, epoch {epoch}"
        for l in range(es_i.L):
            assert torch.equal(es_i.grads[l], es_a.grads[l]), f"layer {l} gradient, epoch {epoch}"
            assert torch.equal(es_i.W[l], es_a.W[l])
    assert any(g.abs().max() > 0 for g in es_a.grads)


def test_pre_entry_point_validation(hses_gpu):
    a, b, r, n = 128, 784, 128, 4
    rec = K.factor_record(a, b, r, 0, n)
    img = K.pair_image(a, b, r, 0, n)
    with pytest.raises(HsesError, match="image"):
        K.pair_factors(KEY, r, 0.02, 0, 0, 0, n, a, b, rec, img[: img.numel() // 2])
    with pytest.raises(HsesError, match="record"):
        K.pair_factors(KEY, r, 0.02, 0, 0, 0, n, a, b, rec[:100], img)
    with pytest.raises(HsesError, match="rank"):
        K.pair_factors(KEY, 8, 0.02, 0, 0, 0, n, a, b, rec, img)
