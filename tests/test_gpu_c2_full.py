"""configs[1] (C2) at its full size: one EggRoll layer W 1024x1024 fp32,
N = 4096 members, r = 1, 16 rows per member, x ~ N(0, 1), through the product
path the bench times (hses_perturbed_linear with fp32 math, then the z-score and
hses_es_update).

* Sampled members (both ends of the population, either side of the 128-row
  GEMM tiles' member boundaries and of the workgroup wrap points, the middle)
  against float64 brute force on the oracle's factors and against the oracle's
  own fp32 do_mm, rel 1e-5 of the output scale (eggroll.rs:419-446).
* Every member against a PyTorch fp32 reference: the shared product x W^T from
  torch's GEMM (TF32 off) plus each member's rank-1 term from the factors that
  hses_lora_factors materialises (those equal the oracle's bit for bit, checked
  here on the sampled members), rel 1e-5 of the output scale.
* The ES gradient over all 4096 members against the oracle's double-accumulated
  gradient on the same z-scored fitness, rel 1e-5 (eggroll.rs:353-404).
"""
import math

import numpy as np
import pytest
import torch

from hyperscalees_amd._lib import MATH_F32
from tests import oracle_lib as O

pytestmark = pytest.mark.gpu

N, RPM, A_OUT, B_IN, RANK, SIGMA = 4096, 16, 1024, 1024, 1, 0.02
KEY = 0x9E3779B97F4A7C15
MEMBERS = (0, 1, 7, 8, 9, 15, 16, 255, 256, 511, 512, 1023, 1024, 2047, 2048, 3001, 4094, 4095)


@pytest.fixture(scope="module")
def c2_run(hses_gpu):
    K = hses_gpu
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((A_OUT, B_IN)) / 32.0).astype(np.float32)
    x = rng.standard_normal((N * RPM, B_IN)).astype(np.float32)
    fit = rng.standard_normal(N).astype(np.float32)
    Wd, xd, fd = (torch.from_numpy(v).cuda() for v in (W, x, fit))
    y = K.perturbed_linear(xd, Wd, KEY, RANK, SIGMA, 0, 0, 0, N, RPM, math=MATH_F32)
    z, _ = K.convert_fitnesses(fd)
    grad = K.es_update(z, 0, KEY, RANK, SIGMA, 0, 0, A_OUT, B_IN,
                       float(np.float32(-math.sqrt(N) / N)))
    bs = O.load().or_base_sigma(SIGMA, RANK)
    Af, Bf = K.lora_factors(bs, KEY, RANK, 0, 0, (0, N), A_OUT, B_IN)
    torch.cuda.synchronize()
    return dict(W=W, x=x, fit=fit, Wd=Wd, xd=xd, y=y, z=z.cpu().numpy(),
                grad=grad.cpu().numpy(), Af=Af, Bf=Bf)


def test_c2_full_sampled_members_vs_oracle(c2_run):
    W, x = c2_run["W"], c2_run["x"]
    bs = O.load().or_base_sigma(SIGMA, RANK)
    A, B = O.lora_factors(bs, KEY, RANK, 0, np.array(MEMBERS), A_OUT, B_IN)
    rows = np.concatenate([np.arange(m * RPM, (m + 1) * RPM) for m in MEMBERS])
    y = c2_run["y"].index_select(0, torch.as_tensor(rows, device="cuda")).cpu().numpy()
    Wd64 = W.astype(np.float64)
    for j, m in enumerate(MEMBERS):
        xs = x[m * RPM:(m + 1) * RPM]
        got = y[j * RPM:(j + 1) * RPM]
        ref = xs.astype(np.float64) @ Wd64.T
        ref += (xs.astype(np.float64) @ B[j].astype(np.float64)) @ A[j].astype(np.float64).T
        scale = np.abs(ref).max()
        assert np.abs(got - ref).max() <= 1e-5 * scale, f"member {m} vs float64"
        ora = O.do_mm(xs, W, A[j], B[j])
        assert np.abs(got - ora).max() <= 1e-5 * scale, f"member {m} vs the oracle's do_mm"
        # the materialised factors the whole-population check uses are the oracle's
        np.testing.assert_array_equal(c2_run["Af"][m].cpu().numpy(), A[j])
        np.testing.assert_array_equal(c2_run["Bf"][m].cpu().numpy(), B[j])


def test_c2_full_every_member_vs_torch_fp32(c2_run):
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        base = c2_run["xd"] @ c2_run["Wd"].t()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    xm = c2_run["xd"].view(N, RPM, B_IN)
    xb = torch.bmm(xm, c2_run["Bf"])                                  # (N, RPM, 1)
    corr = torch.bmm(xb, c2_run["Af"].transpose(1, 2).contiguous())   # (N, RPM, A_OUT)
    ref = base + corr.view(N * RPM, A_OUT)
    scale = ref.abs().max().item()
    err = (c2_run["y"] - ref).abs()
    per_member = err.view(N, RPM * A_OUT).max(dim=1).values
    worst = int(per_member.argmax().item())
    assert per_member.max().item() <= 1e-5 * scale, \
        f"member {worst}: err {per_member[worst].item():.3e} of scale {scale:.3e}"
    # the perturbation is present in every member (not silently dropped)
    assert (corr.view(N, -1).abs().max(dim=1).values > 0).all()


def test_c2_full_es_gradient(c2_run):
    g = O.lora_grad_f64(SIGMA, KEY, RANK, 0, c2_run["z"], A_OUT, B_IN, nthreads=16)
    err = np.abs(c2_run["grad"] - g).max()
    assert err <= 1e-5 * np.abs(g).max(), f"gradient err {err:.3e} of {np.abs(g).max():.3e}"
