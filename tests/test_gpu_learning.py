"""End-to-end training: repeated ES steps on the GPU learn a task.

The reference trains the SNN-MLP on MNIST with this loop (accumulate_train.rs:770-944,
snn_mnist.rs:180-201) and reports best_val ~0.91; no dataset is available here, so the
task is synthetic: 64 sparse intensity vectors labelled by a fixed random linear teacher
(argmax of x T over 10 classes, learnable by the model), every member evaluating all 64.
The per-step parity tests pin each step against the oracle; these check that the steps
compose into learning: the population's mean log-likelihood fitness rises and the share of
rows whose logits' argmax is the label climbs well above its start (chance is 0.1).
Everything is seeded and the kernels are deterministic, so the curves repeat exactly."""
import numpy as np
import pytest

from hyperscalees_amd import snn
from hyperscalees_amd._lib import ADAMW, MATH_BF16, MATH_F32, MATH_F32X, SGD

pytestmark = pytest.mark.gpu


def teacher_task(n_samples=64, seed=5):
    pool, _ = snn.synthetic_pool(n_samples, 784, 10, seed=seed)
    teacher = np.random.default_rng(seed + 1).standard_normal((784, 10)).astype(np.float32)
    return pool, np.argmax(pool @ teacher, axis=1).astype(np.int32)


def train(cfg, steps):
    pool, labels = teacher_task(cfg.rows)
    idx = np.tile(np.arange(cfg.rows, dtype=np.int32), cfg.n)
    W = snn.init_weights(cfg.dims, 0, gain=snn.ACTIVE_GAIN)
    es = snn.SnnEs(cfg, W, pool, labels, idx)
    fit, acc = [], []
    for i in range(steps):
        f = es.step(epoch=i)
        fit.append(float(f.mean()))
        acc.append(int(es.correct.item()) / (cfg.n * cfg.rows))
    return np.array(fit), np.array(acc)


@pytest.mark.parametrize("math", [MATH_F32X, MATH_BF16])
def test_member_weight_step_learns(hses_gpu, math):
    # the C3 path (factors drawn ahead, member weights, fused LIF, count-plane
    # readout, record-fed update, AdamW) at a small population
    cfg = snn.SnnConfig(T=16, rows=64, n=512, rank=32, sigma=0.02, math=math, solver=ADAMW,
                        lr=0.01, poisson_seed=(1, 2, 3, 4))
    fit, acc = train(cfg, 60)
    print(f"math {math}: fitness {fit[0]:.3f} -> {fit[-10:].mean():.3f}, "
          f"accuracy {acc[0]:.3f} -> {acc[-10:].mean():.3f}")
    assert fit[-10:].mean() > fit[0] + 0.6
    assert acc[-10:].mean() > max(0.25, acc[0] + 0.1)


def test_small_rank_step_learns(hses_gpu):
    # the C1 path (fp32 small-rank forward and update, SGD)
    cfg = snn.SnnConfig(T=8, rows=64, n=256, rank=4, sigma=0.02, math=MATH_F32, solver=SGD,
                        lr=0.2, poisson_seed=(1, 2, 3, 4))
    fit, acc = train(cfg, 100)
    print(f"C1: fitness {fit[0]:.3f} -> {fit[-10:].mean():.3f}, "
          f"accuracy {acc[0]:.3f} -> {acc[-10:].mean():.3f}")
    assert fit[-10:].mean() > fit[0] + 0.2
    assert acc[-10:].mean() > acc[0] + 0.01
