"""GPU parity of the batched perturbed forward (do_mm / lora_linear_batched).

Reference: y_m = x_m W^T + (x_m B_m) A_m^T with the oracle's bit-exact factors,
evaluated in float64 by brute force (eggroll.rs:419-446, snn.rs:665-685).
Tolerances: fp32 math rel 1e-5 of the output scale; bf16 math compared with
the same product on bf16-rounded W/B (rel 2e-3), and with the fp32 result
within rel 2e-2 (the bf16-path bar)."""
import numpy as np
import pytest
import torch

from hyperscalees_amd._lib import FMT_BF16, FMT_BITS, FMT_F32, MATH_BF16, MATH_F32
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu
KEY = 0x9E3779B97F4A7C15


def bf16_round(a):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)
    return t.to(torch.float32).numpy()


def ref_forward(x3, W, A, B, rpm):
    """x3 (T, n*rpm, b) -> (T, n*rpm, a) in float64."""
    x3 = x3.astype(np.float64)
    y = x3 @ W.astype(np.float64).T
    n = A.shape[0]
    for m in range(n):
        xs = x3[:, m * rpm:(m + 1) * rpm, :]
        y[:, m * rpm:(m + 1) * rpm, :] += (xs @ B[m].astype(np.float64)) @ A[m].astype(np.float64).T
    return y


def pack_bits(x3):
    T, M, b = x3.shape
    words = (b + 63) // 64
    padded = np.zeros((T, M, words * 64), np.uint64)
    padded[..., :b] = x3.astype(np.uint64)
    w = (padded.reshape(T, M, words, 64) << np.arange(64, dtype=np.uint64)).sum(-1, dtype=np.uint64)
    return torch.from_numpy(w.view(np.int64)).cuda()


def run(hses_gpu, x3, W, r, sigma, n, rpm, tid_lo=0, fmt=FMT_F32, math=MATH_F32, epoch=0, nreuse=0):
    T, M, b = x3.shape
    if fmt == FMT_F32:
        xt = torch.from_numpy(np.ascontiguousarray(x3, np.float32)).cuda()
    elif fmt == FMT_BF16:
        xt = torch.from_numpy(np.ascontiguousarray(x3, np.float32)).to(torch.bfloat16).cuda()
    else:
        xt = pack_bits(x3)
    y = hses_gpu.perturbed_linear(xt, torch.from_numpy(W).cuda(), KEY, r, sigma, epoch, nreuse,
                                  tid_lo, n, rpm, x_fmt=fmt, n_time=T, math=math)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(T, M, -1)


def factors(sigma, r, n, tid_lo, a, b, epoch=0, nreuse=0):
    bs = O.load().or_base_sigma(sigma, r)
    return O.lora_factors(bs, KEY, r, epoch, np.arange(tid_lo, tid_lo + n), a, b, noise_reuse=nreuse)


def assert_close(y, ref, rel):
    scale = np.abs(ref).max()
    err = np.abs(y - ref).max()
    assert err <= rel * scale, f"max err {err:.3e} > {rel:.1e} * {scale:.3e}"


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo", [
    (16, 16, 1, 1024, 1024, 1, 0),      # C2 layer shape, 16 members
    (3, 64, 8, 128, 784, 4, 0),         # C1 fc1, time-major, 3 members
    (5, 5, 3, 10, 100, 4, 3),           # members straddle tiles, odd tid_lo, ragged a/b
    (7, 9, 1, 70, 33, 2, 1),
    (4, 64, 1, 10, 128, 4, 6),          # C1 readout
])
def test_perturbed_linear_f32(hses_gpu, n, rpm, T, a, b, r, tid_lo):
    rng = np.random.default_rng(n * 100 + b)
    x3 = rng.standard_normal((T, n * rpm, b)).astype(np.float32)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(0.02 * 10, r, n, tid_lo, a, b)
    y = run(hses_gpu, x3, W, r, 0.2, n, rpm, tid_lo)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 1e-5)


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,fmt", [
    (4, 48, 1, 300, 100, 16, 5, FMT_F32),    # rank 16, four members per tile, three column tiles
    (6, 40, 2, 96, 300, 3, 2, FMT_BITS),     # rank 3 (padded to 4), bit-packed, time-major
    (5, 64, 1, 64, 77, 5, 1, FMT_BF16),      # rank 5 (padded to 8), unaligned bf16 rows
    (9, 16, 1, 40, 1000, 1, 0, FMT_F32),     # rank 1, 64-column tile, eight members per tile
    (3, 200, 1, 130, 64, 8, 7, FMT_F32),     # members straddle tiles, 128 + 2 columns
])
def test_fp32_gemm_kernel(hses_gpu, n, rpm, T, a, b, r, tid_lo, fmt):
    # the fp32 MFMA GEMM with x B_m fused and the members' factors drawn up front
    rng = np.random.default_rng(n * 31 + a + b + r)
    if fmt == FMT_BITS:
        x3 = (rng.random((T, n * rpm, b)) < 0.3).astype(np.float32)
    else:
        x3 = rng.standard_normal((T, n * rpm, b)).astype(np.float32)
        if fmt == FMT_BF16:
            x3 = bf16_round(x3)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(0.2, r, n, tid_lo, a, b)
    y = run(hses_gpu, x3, W, r, 0.2, n, rpm, tid_lo, fmt=fmt, math=MATH_F32)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 1e-5)


def test_perturbed_linear_spike_formats_agree(hses_gpu):
    # Binary inputs are exact in every format: F32, BF16 and packed bits give
    # the same bits for the same math mode.
    rng = np.random.default_rng(7)
    n, rpm, T, a, b, r = 4, 16, 4, 128, 784, 4
    x3 = (rng.random((T, n * rpm, b)) < 0.2).astype(np.float32)
    W = (rng.standard_normal((a, b)) / 28).astype(np.float32)
    A, B = factors(0.02, r, n, 0, a, b)
    ref = ref_forward(x3, W, A, B, rpm)
    for math in (MATH_F32, MATH_BF16):
        ys = [run(hses_gpu, x3, W, r, 0.02, n, rpm, fmt=f, math=math)
              for f in (FMT_F32, FMT_BF16, FMT_BITS)]
        np.testing.assert_array_equal(ys[0], ys[1])
        np.testing.assert_array_equal(ys[0], ys[2])
        if math == MATH_F32:
            assert_close(ys[0], ref, 1e-5)
        else:
            refb = ref_forward(x3, bf16_round(W), A, bf16_round(B), rpm)
            assert_close(ys[0], refb, 2e-3)
            assert_close(ys[0], ref, 2e-2)


def test_clean_path_is_plain_product(hses_gpu):
    rng = np.random.default_rng(3)
    x3 = rng.standard_normal((1, 40, 50)).astype(np.float32)
    W = rng.standard_normal((30, 50)).astype(np.float32)
    y = run(hses_gpu, x3, W, 4, 0.0, 8, 5)
    assert_close(y, x3.astype(np.float64) @ W.T.astype(np.float64), 1e-5)


def test_noise_reuse_epoch(hses_gpu):
    rng = np.random.default_rng(4)
    n, rpm, a, b, r = 6, 8, 16, 24, 2
    x3 = rng.standard_normal((1, n * rpm, b)).astype(np.float32)
    W = rng.standard_normal((a, b)).astype(np.float32)
    A, B = factors(0.5, r, n, 0, a, b, epoch=5, nreuse=2)
    y = run(hses_gpu, x3, W, r, 0.5, n, rpm, epoch=5, nreuse=2)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 1e-5)


def ref_forward_bf16(x3, W, A, B, rpm):
    """The bf16 pair kernel's arithmetic: bf16 W, B, A and a bf16 rounding of
    (sign * x B) before the second product; float64 accumulation otherwise."""
    Wb, Bb, Ab = bf16_round(W), bf16_round(B), bf16_round(A)
    x64 = x3.astype(np.float64)
    y = x64 @ Wb.astype(np.float64).T
    n = A.shape[0]
    for m in range(n):
        xs = x64[:, m * rpm:(m + 1) * rpm, :]
        xb = (xs @ Bb[m].astype(np.float64)).astype(np.float32)
        y[:, m * rpm:(m + 1) * rpm, :] += bf16_round(xb).astype(np.float64) @ Ab[m].astype(np.float64).T
    return y


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,fmt", [
    (4, 64, 16, 128, 784, 128, 0, FMT_BITS),   # C3 fc1 (two pairs)
    (3, 64, 16, 128, 128, 128, 1, FMT_BITS),   # C3 fc2, partial pairs at both ends
    (4, 64, 1, 10, 128, 128, 0, FMT_F32),      # C3 readout on rates
    (2, 40, 3, 96, 200, 64, 0, FMT_BF16),      # rows not a multiple of the block
    (5, 7, 2, 33, 50, 16, 2, FMT_F32),
    (3, 20, 2, 16, 96, 32, 1, FMT_BF16),       # a = 16: one W column tile per wave
    (3, 20, 2, 16, 128, 32, 1, FMT_BF16),      # a = 16, b % 64 == 0: x loaded a sub-step ahead
    (5, 7, 2, 12, 256, 16, 2, FMT_F32),        # same, four K tiles, rows not a multiple of the block
])
def test_perturbed_linear_pair_kernel(hses_gpu, n, rpm, T, a, b, r, tid_lo, fmt):
    rng = np.random.default_rng(n * 1000 + a + r)
    if fmt == FMT_BITS:
        x3 = (rng.random((T, n * rpm, b)) < 0.2).astype(np.float32)
    else:
        x3 = (rng.integers(0, 17, (T, n * rpm, b)) / 16.0).astype(np.float32)  # rates, exact in bf16
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(0.2, r, n, tid_lo, a, b)
    y = run(hses_gpu, x3, W, r, 0.2, n, rpm, tid_lo, fmt=fmt, math=MATH_BF16)
    assert_close(y, ref_forward_bf16(x3, W, A, B, rpm), 2e-3)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 2e-2)


def test_pair_kernel_many_pairs_per_workgroup(hses_gpu):
    """More pairs than workgroups: each persistent workgroup reuses its B
    staging slot and LDS for several pairs in a row."""
    n, rpm, T, a, b, r = 600, 2, 1, 32, 96, 32
    rng = np.random.default_rng(5)
    x3 = (rng.random((T, n * rpm, b)) < 0.3).astype(np.float32)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(0.2, r, n, 0, a, b)
    y = run(hses_gpu, x3, W, r, 0.2, n, rpm, 0, fmt=FMT_BITS, math=MATH_BF16)
    assert_close(y, ref_forward_bf16(x3, W, A, B, rpm), 2e-3)


def test_device_properties(hses_gpu):
    p = torch.cuda.get_device_properties(0)
    print("device", p.name, "CUs", p.multi_processor_count,
          "smem/block", getattr(p, "shared_memory_per_block", None),
          "smem/mp", getattr(p, "shared_memory_per_multiprocessor", None))


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo", [
    (4, 64, 16, 128, 784, 128, 0),   # C3 fc1
    (3, 64, 16, 128, 128, 128, 1),   # C3 fc2/fc3 shape, partial pairs at both ends
    (5, 12, 8, 100, 200, 64, 0),     # partial spike word (a = 100), r = 64
    (4, 3, 1, 64, 96, 16, 0),        # T = 1
    (2, 5, 32, 70, 130, 48, 1),      # T = 32, r % 32 == 16
    (600, 1, 4, 32, 64, 32, 0),      # more pairs than workgroups
])
def test_fused_lif_matches_unfused(hses_gpu, n, rpm, T, a, b, r, tid_lo):
    """hses_perturbed_linear_lif == hses_lif_scan(hses_perturbed_linear(...))
    bit for bit (spikes), and its rates == hses_spike_rate of those spikes.
    The unfused currents are pinned against the oracle by the tests above."""
    rng = np.random.default_rng(n * 7 + T)
    x3 = (rng.random((T, n * rpm, b)) < 0.3).astype(np.float32)
    W = (rng.standard_normal((a, b)) * (6.0 / np.sqrt(b))).astype(np.float32)
    xb = pack_bits(x3)
    Wt = torch.from_numpy(W).cuda()
    tau, vth = 10.0, (1.0 if T > 4 else 0.25)  # short series need a lower threshold to spike
    y = hses_gpu.perturbed_linear(xb, Wt, KEY, r, 0.2, 3, 0, tid_lo, n, rpm, x_fmt=FMT_BITS,
                                  n_time=T, math=MATH_BF16)
    spk_ref = hses_gpu.lif_scan(y.view(T, n * rpm, a), tau, vth, fmt=FMT_BITS)
    rate_ref = hses_gpu.spike_rate(spk_ref, FMT_BITS, a)
    spk, rate = hses_gpu.perturbed_linear_lif(xb, Wt, KEY, r, 0.2, 3, 0, tid_lo, n, rpm, T, tau,
                                              vth, want_rate=True)
    torch.cuda.synchronize()
    assert torch.equal(spk, spk_ref)
    assert torch.equal(rate, rate_ref)
    mean = float(rate.mean())
    assert 0.005 < mean < 0.95, mean
    # spikes only: same words
    spk2, none = hses_gpu.perturbed_linear_lif(xb, Wt, KEY, r, 0.2, 3, 0, tid_lo, n, rpm, T, tau,
                                               vth)
    assert none is None and torch.equal(spk2, spk_ref)


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,pre", [
    (4, 64, 16, 128, 784, 128, 0, True),    # C3 fc1, factors drawn ahead (the step's form)
    (3, 64, 16, 128, 128, 128, 1, True),    # C3 fc2/fc3 shape (resident tiles), partial pairs
    (5, 12, 8, 100, 200, 64, 0, False),     # partial spike word, generating form
    (2, 5, 32, 70, 130, 48, 1, False),      # T = 32
])
def test_fused_lif_time_inner_layout(hses_gpu, n, rpm, T, a, b, r, tid_lo, pre):
    """The time-inner layout (each row's T words adjacent, (M, T, words)) gives
    the spikes and rates of the time-major layout, bit for bit."""
    rng = np.random.default_rng(n * 11 + T + b)
    M = n * rpm
    x3 = (rng.random((T, M, b)) < 0.3).astype(np.float32)
    W = (rng.standard_normal((a, b)) * (6.0 / np.sqrt(b))).astype(np.float32)
    xb = pack_bits(x3)
    Wt = torch.from_numpy(W).cuda()
    tau, vth = 10.0, 1.0
    kw = {}
    if pre:
        rec = hses_gpu.factor_record(a, b, r, tid_lo, n)
        img = hses_gpu.pair_image(a, b, r, tid_lo, n)
        hses_gpu.pair_factors(KEY, r, 0.2, 3, 0, tid_lo, n, a, b, rec, img)
        kw = dict(rec=rec, img=img)
    spk_tm, rate_tm = hses_gpu.perturbed_linear_lif(xb, Wt, KEY, r, 0.2, 3, 0, tid_lo, n, rpm, T,
                                                    tau, vth, want_rate=True, **kw)
    x_ti = xb.transpose(0, 1).contiguous()
    spk_ti, rate_ti = hses_gpu.perturbed_linear_lif(x_ti, Wt, KEY, r, 0.2, 3, 0, tid_lo, n, rpm, T,
                                                    tau, vth, want_rate=True, time_inner=True, **kw)
    torch.cuda.synchronize()
    assert tuple(spk_ti.shape) == (M, T, spk_tm.shape[2])
    assert torch.equal(spk_ti.transpose(0, 1), spk_tm)
    assert torch.equal(rate_ti, rate_tm)
    assert 0.005 < float(rate_tm.mean()) < 0.95


def ref_forward_t(x3, W, A, B, rpm):
    """do_Tmm: x3 (T, n*rpm, a) -> (T, n*rpm, b), x W + (x A_m) B_m^T in float64."""
    x3 = x3.astype(np.float64)
    y = x3 @ W.astype(np.float64)
    for m in range(A.shape[0]):
        xs = x3[:, m * rpm:(m + 1) * rpm, :]
        y[:, m * rpm:(m + 1) * rpm, :] += (xs @ A[m].astype(np.float64)) @ B[m].astype(np.float64).T
    return y


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,math", [
    (16, 16, 1, 512, 512, 1, 0, MATH_F32),     # C5-like square layer, r = 1
    (6, 8, 1, 512, 256, 1, 3, MATH_BF16),      # C5 precision, odd first thread id
    (5, 5, 3, 100, 10, 4, 3, MATH_F32),        # time-major, members straddle tiles, ragged
    (7, 9, 1, 33, 70, 2, 1, MATH_F32),
    (4, 32, 1, 96, 128, 16, 0, MATH_BF16),     # pair kernel, rank 16
    (3, 64, 2, 784, 128, 128, 1, MATH_BF16),   # pair kernel at the C3 rank, half pairs
    (5, 8, 1, 64, 12, 16, 1, MATH_BF16),       # pair kernel, output width <= 16
])
def test_perturbed_linear_t(hses_gpu, n, rpm, T, a, b, r, tid_lo, math):
    # do_Tmm_impl (eggroll.rs:450-477): the same (a, b) parameter stream as
    # do_mm, with A (scaled) on the input side and B on the output side.
    rng = np.random.default_rng(n * 31 + a + b + r)
    x3 = rng.standard_normal((T, n * rpm, a)).astype(np.float32)
    W = (rng.standard_normal((a, b)) / np.sqrt(a)).astype(np.float32)
    sigma = 0.2
    A, B = factors(sigma, r, n, tid_lo, a, b)
    ref = ref_forward_t(x3, W, A, B, rpm)
    y = hses_gpu.perturbed_linear_t(torch.from_numpy(x3).cuda(), torch.from_numpy(W).cuda(), KEY,
                                    r, sigma, 0, 0, tid_lo, n, rpm, n_time=T, math=math)
    torch.cuda.synchronize()
    y = y.cpu().numpy().reshape(T, n * rpm, b)
    assert_close(y, ref, 1e-5 if math == MATH_F32 else 2e-2)
    if math == MATH_F32:
        # the oracle's restatement of do_Tmm_impl on member 0's rows at t = 0
        y0 = np.zeros((rpm, b), np.float32)
        O.load().or_do_Tmm(np.ascontiguousarray(x3[0, :rpm]), rpm, W, a, b,
                           np.ascontiguousarray(A[0]).ctypes.data,
                           np.ascontiguousarray(B[0]).ctypes.data, r, y0)
        assert_close(y[0, :rpm], y0.astype(np.float64), 1e-5)


def test_perturbed_linear_t_clean(hses_gpu):
    # sigma = 0: the clean x W (do_Tmm_impl without iterinfo)
    rng = np.random.default_rng(77)
    x = rng.standard_normal((40, 65)).astype(np.float32)
    W = rng.standard_normal((65, 33)).astype(np.float32)
    y = hses_gpu.perturbed_linear_t(torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda(), KEY,
                                    4, 0.0, 0, 0, 0, 40, 1)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), x.astype(np.float64) @ W.astype(np.float64), 1e-5)


# -- the wide-output small-rank kernel (bf16 math, members x rank <= 16 per 128-row tile) --

@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,fmt", [
    (4, 128, 1, 512, 512, 1, 0, FMT_F32),      # C5 square layer, one member per tile
    (3, 128, 1, 2048, 512, 1, 1, FMT_F32),     # C5 ChannelMixing key, odd first member
    (2, 128, 1, 512, 2048, 1, 0, FMT_BF16),    # C5 ChannelMixing value, bf16 activations
    (6, 64, 1, 300, 256, 2, 3, FMT_F32),       # two members per tile, ragged output width
    (5, 100, 1, 130, 96, 1, 0, FMT_F32),       # members straddle tiles (three per tile)
    (4, 32, 2, 256, 200, 4, 2, FMT_F32),       # time-major planes, four members per tile
    (3, 64, 1, 192, 300, 2, 0, FMT_BITS),      # bit-packed input, K not a multiple of 64
    (3, 128, 1, 100, 512, 1, 0, FMT_F32),      # output width in (64, 128]: 128-column passes
    (2, 128, 1, 100, 256, 1, 1, FMT_BF16),
    (4, 64, 1, 64, 200, 2, 0, FMT_BF16),       # exactly 64 columns: 64-column passes
])
def test_wide_kernel(hses_gpu, n, rpm, T, a, b, r, tid_lo, fmt):
    rng = np.random.default_rng(n * 7 + a + b + r)
    if fmt == FMT_BITS:
        x3 = (rng.random((T, n * rpm, b)) < 0.3).astype(np.float32)
    else:
        x3 = rng.standard_normal((T, n * rpm, b)).astype(np.float32)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    sigma = 0.2
    A, B = factors(sigma, r, n, tid_lo, a, b)
    y = run(hses_gpu, x3, W, r, sigma, n, rpm, tid_lo, fmt=fmt, math=MATH_BF16)
    xb = bf16_round(x3)
    assert_close(y, ref_forward(xb, bf16_round(W), A, bf16_round(B), rpm), 2e-3)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 2e-2)


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,fmt,sigma", [
    (4, 128, 1, 512, 512, 1, 0, FMT_BF16, 0.2),    # C5 square layer: two members per tile
    (3, 100, 1, 300, 200, 3, 1, FMT_F32, 0.2),     # ragged output tile, K % 64 != 0, 4 members per tile
    (2, 64, 4, 256, 128, 4, 2, FMT_F32, 0.2),      # time-major planes, rank 4
    (2, 128, 1, 2048, 512, 1, 0, FMT_BF16, 0.2),   # ChannelMixing key width: 8 column tiles
    (2, 128, 1, 512, 256, 1, 0, FMT_F32, 0.0),     # sigma 0: the plain product
])
def test_bf16_gemm_kernel(hses_gpu, n, rpm, T, a, b, r, tid_lo, fmt, sigma):
    # outputs >= 256 wide at bf16 math: the bf16 MFMA GEMM with x B_m fused
    rng = np.random.default_rng(n * 13 + a + b + r)
    x3 = rng.standard_normal((T, n * rpm, b)).astype(np.float32)
    if fmt == FMT_BF16:
        x3 = bf16_round(x3)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(max(sigma, 1e-30), r, n, tid_lo, a, b)
    if sigma == 0.0:
        A = np.zeros_like(A)
    y = run(hses_gpu, x3, W, r, sigma, n, rpm, tid_lo, fmt=fmt, math=MATH_BF16)
    assert_close(y, ref_forward(bf16_round(x3), bf16_round(W), A, bf16_round(B), rpm), 2e-3)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 2e-2)


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,sigma", [
    (4, 128, 1, 512, 512, 1, 0, 0.2),     # C5 square layer
    (2, 128, 1, 2048, 512, 1, 0, 0.2),    # ChannelMixing key width
    (2, 128, 1, 512, 2048, 1, 0, 0.2),    # ChannelMixing value: 64 K steps
    (3, 128, 1, 512, 32, 1, 1, 0.2),      # one K step (w2 / a2 / v2)
    (3, 128, 1, 512, 96, 1, 0, 0.2),      # three K steps (g2)
    (3, 100, 1, 300, 64, 1, 2, 0.2),      # ragged rows and output width
    (2, 64, 4, 256, 128, 4, 2, 0.2),      # time-major planes, rank 4
    (6, 64, 1, 256, 160, 4, 0, 0.2),      # rank 4, four members per tile (register path)
    (2, 128, 1, 512, 256, 1, 0, 0.0),     # sigma 0
])
def test_bf16_gemm_bf16_x_equals_f32_x(hses_gpu, n, rpm, T, a, b, r, tid_lo, sigma):
    # bf16 x takes the direct-to-LDS pipeline where it applies, fp32 x holding
    # the same (bf16-representable) values the register pipeline: the same
    # operands, products and accumulation order, so the outputs are equal
    rng = np.random.default_rng(n * 17 + a + b + r)
    x3 = bf16_round(rng.standard_normal((T, n * rpm, b)).astype(np.float32))
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    y32 = run(hses_gpu, x3, W, r, sigma, n, rpm, tid_lo, fmt=FMT_F32, math=MATH_BF16)
    y16 = run(hses_gpu, x3, W, r, sigma, n, rpm, tid_lo, fmt=FMT_BF16, math=MATH_BF16)
    np.testing.assert_array_equal(y16, y32)


@pytest.mark.parametrize("act", [1, 2, 3])
def test_bf16_gemm_activation_bf16_out(hses_gpu, act):
    from hyperscalees_amd._lib import ACT_RELU_SQ, ACT_SIGMOID, ACT_TANH
    n, rpm, a, b, r, sigma = 3, 128, 512, 256, 1, 0.2
    rng = np.random.default_rng(act)
    x = bf16_round(rng.standard_normal((n * rpm, b)).astype(np.float32))
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(sigma, r, n, 0, a, b)
    y = hses_gpu.perturbed_linear(torch.from_numpy(x).cuda().to(torch.bfloat16),
                                  torch.from_numpy(W).cuda(), KEY, r, sigma, 0, 0, 0, n, rpm,
                                  x_fmt=FMT_BF16, math=MATH_BF16, act=act, out_bf16=True)
    torch.cuda.synchronize()
    ref = ref_forward(x[None], bf16_round(W), A, bf16_round(B), rpm)[0]
    f = {ACT_TANH: np.tanh, ACT_SIGMOID: lambda v: 1 / (1 + np.exp(-v)),
         ACT_RELU_SQ: lambda v: np.maximum(v, 0) ** 2}[act]
    assert_close(y.float().cpu().numpy(), f(ref), 6e-3)   # plus the bf16 rounding of y


@pytest.mark.parametrize("a,b,act", [(512, 32, 1), (96, 512, 2), (512, 512, 3), (256, 64, 0),
                                     (512, 96, 2), (512, 120, 0)])  # C5 g1: width 96
def test_wide_kernel_transposed_and_activations(hses_gpu, a, b, act):
    # do_Tmm on a parameter W (a, b): y = act(x W + (x A_m) B_m^T), bf16 math
    from hyperscalees_amd._lib import ACT_RELU_SQ, ACT_SIGMOID, ACT_TANH
    n, rpm, r, tid_lo, sigma = 4, 128, 1, 1, 0.3
    rng = np.random.default_rng(a + b + act)
    x = rng.standard_normal((n * rpm, a)).astype(np.float32)
    W = (rng.standard_normal((a, b)) / np.sqrt(a)).astype(np.float32)
    A, B = factors(sigma, r, n, tid_lo, a, b)
    y = hses_gpu.perturbed_linear_t(torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda(), KEY, r,
                                    sigma, 0, 0, tid_lo, n, rpm, math=MATH_BF16, act=act)
    torch.cuda.synchronize()
    ref = ref_forward_t(bf16_round(x)[None], bf16_round(W), bf16_round(A), B, rpm)[0]
    f = {0: lambda v: v, ACT_TANH: np.tanh, ACT_SIGMOID: lambda v: 1 / (1 + np.exp(-v)),
         ACT_RELU_SQ: lambda v: np.maximum(v, 0) ** 2}[act]
    assert_close(y.cpu().numpy(), f(ref), 2e-3)


def test_linear_activation_unfused_path_matches(hses_gpu):
    # fp32 math runs k_linear_small and applies the activation afterwards
    from hyperscalees_amd._lib import ACT_RELU_SQ
    n, rpm, a, b, r = 3, 16, 40, 24, 2
    rng = np.random.default_rng(9)
    x = rng.standard_normal((n * rpm, b)).astype(np.float32)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(0.2, r, n, 0, a, b)
    y = hses_gpu.perturbed_linear(torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda(), KEY, r,
                                  0.2, 0, 0, 0, n, rpm, act=ACT_RELU_SQ)
    torch.cuda.synchronize()
    ref = np.maximum(ref_forward(x[None], W, A, B, rpm)[0], 0) ** 2
    assert_close(y.cpu().numpy(), ref, 1e-5)


@pytest.mark.parametrize("n,rpm,T,a,b,r,tid_lo,fmt", [
    (1024, 1, 1, 10, 64, 8, 0, FMT_F32),     # C4 readout on pooled rows
    (300, 2, 1, 70, 33, 8, 3, FMT_F32),      # output wider than a wave, odd first member
    (130, 1, 2, 20, 100, 12, 0, FMT_BF16),   # time planes, bf16 activations
])
def test_rows_kernel_few_rows_per_member(hses_gpu, n, rpm, T, a, b, r, tid_lo, fmt):
    # more members per 64-row tile than the small-rank kernel stages: one wave per member
    rng = np.random.default_rng(n + a)
    x3 = rng.standard_normal((T, n * rpm, b)).astype(np.float32)
    if fmt == FMT_BF16:
        x3 = bf16_round(x3)
    W = (rng.standard_normal((a, b)) / np.sqrt(b)).astype(np.float32)
    A, B = factors(0.2, r, n, tid_lo, a, b)
    y = run(hses_gpu, x3, W, r, 0.2, n, rpm, tid_lo, fmt=fmt, math=MATH_F32)
    assert_close(y, ref_forward(x3, W, A, B, rpm), 1e-5)
