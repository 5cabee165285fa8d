"""SNN-MLP EggRoll ES step on the GPU, composed from the libhses kernels.

One step (the per-chunk body of accumulate_train.rs:770-938 and the
deterministic noiser stream):
  1. Poisson-encode each member's samples into bit-packed spike trains
     (poisson_encode_fused_oxide.rs:61-106);
  2. hidden layers: perturbed linear (eggroll.rs:419-446, snn.rs:665-685)
     then the LIF scan (snn.rs:53-97), spikes kept bit-packed;
  3. readout on the mean rate (snn.rs:274-280), log-likelihood fitness
     averaged over the member's samples (snn_mnist.rs:180-201);
  4. z-score (eggroll.rs:967-992), ES gradient per layer
     (eggroll.rs:353-404) and one solver step (noiser.rs:155-225).
With `accumulate` K > 1 the population runs as K chunks of N/K members with
frozen parameters, as the reference's K-chunk driver does
(accumulate_train.rs:719-944): each chunk's raw fitness weights an ES
gradient accumulated over the chunks, the raw-fitness sums accumulate on the
device, and combine_affine_grads (eggroll.rs:902-915) turns the sums into the
z-scored gradient before the one solver step.  Nothing is copied to the host.
The model is the reference SnnModel generalised to any number of hidden LIF
layers (the JAX model is depth-generic); every layer is an MM parameter with
its own base key (i+1)*0x9E3779B97F4A7C15 (accumulate_train.rs:603-608).
"""
import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import kernels as K
from ._lib import ADAMW, FMT_BITS, FMT_F32, MATH_BF16, MATH_F32X, REWARD_LOGLIK, SGD

KEY_MUL = 0x9E3779B97F4A7C15


def layer_keys(n_layers):
    return [((i + 1) * KEY_MUL) % 2**64 for i in range(n_layers)]


@dataclass
class SnnConfig:
    dims: tuple = (784, 128, 128, 128, 10)
    T: int = 16
    rows: int = 64                 # samples per member
    n: int = 8192                  # population size N
    rank: int = 128
    sigma: float = 0.02
    tau_m: float = 10.0            # leak 1/tau = 0.1, i.e. decay 0.9
    v_th: float = 1.0
    noise_reuse: int = 0
    # MATH_F32X: fp32-accurate forward (split fp16 operands; the reference's
    # fp32 arithmetic), on the fused path with factors drawn ahead (rank a
    # multiple of 16 in [32, 128], hidden widths <= 128, T <= 16).  MATH_BF16:
    # the faster bf16 forward (spikes differ from fp32 near the threshold).
    # MATH_F32: the generic fp32 kernels (small ranks).
    math: int = MATH_F32X
    solver: int = ADAMW
    lr: float = 0.01
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 1e-4
    poisson_seed: tuple = (0, 0, 0, 0)
    reward: int = REWARD_LOGLIK    # fitness_from_logits_reward kind (snn_mnist.rs:175-201)
    accumulate: int = 1            # K chunks of n / K members (accumulate_train.rs:770)
    max_norm: float = 0.0          # > 0: Solver::TrustRegion, clip by global norm (noiser.rs:215-244)
    keys: list = field(default_factory=list)

    def __post_init__(self):
        if not self.keys:
            self.keys = layer_keys(len(self.dims) - 1)
        if self.accumulate < 1 or self.n % self.accumulate:
            raise ValueError(f"n={self.n} is not a multiple of accumulate={self.accumulate}")

    @property
    def chunk(self):
        return self.n // self.accumulate


def sample_index(seed, n, rows, pool_size):
    """Per-(member, slot) pool index: splitmix64(seed, member*rows+slot) mod pool."""
    c = (np.arange(n * rows, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15))
    z = c + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    z = z ^ (z >> np.uint64(31))
    return (z % np.uint64(pool_size)).astype(np.int32)


def synthetic_pool(pool_size, in_dim, classes, seed=0, zero_frac=0.7):
    """Sparse intensity vectors (70% exact zeros, rest U(0,1)) and uniform labels."""
    rng = np.random.default_rng(seed)
    x = rng.random((pool_size, in_dim), dtype=np.float32)
    x[rng.random((pool_size, in_dim)) < zero_frac] = 0.0
    y = rng.integers(0, classes, pool_size).astype(np.int32)
    return x, y


# With W ~ N(0, 1/fan_in), v_th = 1 and leak 0.1 the hidden layers fire at
# ~1e-6.  Per-layer gains (12, 18, 20 for the hidden layers, 10 for the
# readout) keep every hidden layer of the 784-128-128-128-10 model at 7-9%
# firing so the spikes carry information.  The gains change no arithmetic cost.
ACTIVE_GAIN = (12.0, 18.0, 20.0, 10.0)


def init_weights(dims, seed=0, gain=1.0):
    """W_l ~ N(0, gain_l^2/fan_in) (Mm::new, common.rs:113-121, has gain 1), from
    a seeded fixture RNG.  `gain` is a scalar or one value per layer."""
    rng = np.random.default_rng(seed + 1)
    L = len(dims) - 1
    gains = list(gain) if isinstance(gain, (tuple, list)) else [gain] * L
    if len(gains) != L:
        gains = (gains + [gains[-1]] * L)[:L]
    return [(gains[i] * rng.standard_normal((dims[i + 1], dims[i])) / np.sqrt(dims[i])).astype(np.float32)
            for i in range(L)]


class SnnEs:
    """Device-resident SNN-MLP population evaluation and ES update."""

    def __init__(self, cfg, weights, pool, pool_labels, index, device="cuda", fused=None,
                 record=None, ahead=None, member_weights=None, overlap=None, prepared_pool=None,
                 noise_cache=False):
        self.cfg = cfg
        c = cfg
        self.dev = device
        self.W = [torch.as_tensor(w, dtype=torch.float32).to(device).contiguous() for w in weights]
        self.pool = torch.as_tensor(pool, dtype=torch.float32).to(device).contiguous()
        # The pool stays fixed across steps: the thresholds of its elements
        # that can fire are prepared once (hses_poisson_pool_prepare), and each
        # batch's encode reads those instead of classifying the gathered
        # probabilities again (the same spikes).
        can_pp = (str(device).startswith("cuda") and 1 <= c.T <= 32 and c.T & (c.T - 1) == 0
                  and self.pool.shape[1] <= 2048)
        use_pp = can_pp if prepared_pool is None else (bool(prepared_pool) and can_pp)
        self.ppool = K.PoissonPool(self.pool) if use_pp else None
        idx = torch.as_tensor(index, dtype=torch.int32).to(device).contiguous()
        self.index = idx
        self.labels = torch.as_tensor(pool_labels, dtype=torch.int32).to(device)[idx.long()].contiguous()
        M = c.chunk * c.rows  # activation rows of one chunk
        self.M = M
        L = len(c.dims) - 1
        self.L = L
        hmax = max(c.dims[1:-1]) if L > 1 else 1
        # Hidden layers run as one fused forward+LIF kernel when the
        # large-rank kernel applies; the fp32 currents then never exist.
        can_fuse = (c.math in (MATH_BF16, MATH_F32X) and c.sigma != 0.0 and c.rank % 16 == 0
                    and 16 <= c.rank <= 128 and hmax <= 128 and c.T <= 64
                    and (c.T & (c.T - 1)) == 0)
        self.fused = can_fuse if fused is None else (bool(fused) and can_fuse)
        # Bit-packed spikes of the input and of every hidden layer.  The fused
        # path keeps them time-inner, (M, T, words): a member's rows, in the
        # kernels' slot-major row order, are then contiguous, so a 256-row
        # block of the next layer is one contiguous read.  The unfused path
        # (LIF scan, spike rates) keeps the time-major (T, M, words) layout.
        self.time_inner = self.fused
        self.spk = [torch.empty((M, c.T, K.fmt_width(FMT_BITS, d)) if self.time_inner else
                                (c.T, M, K.fmt_width(FMT_BITS, d)), dtype=torch.int64, device=device)
                    for d in c.dims[:-1]]
        self.cur = None if self.fused else \
            torch.empty((c.T, M, hmax), dtype=torch.float32, device=device)
        self.rate = torch.empty((M, c.dims[-2]), dtype=torch.float32, device=device)
        self.logits = torch.empty((M, c.dims[-1]), dtype=torch.float32, device=device)
        self.raw = torch.empty(c.n, dtype=torch.float32, device=device)
        self.moments = torch.zeros(2, dtype=torch.float64, device=device)
        self.correct = torch.zeros(1, dtype=torch.int64, device=device)
        self.grads = [torch.zeros_like(w) for w in self.W]
        self.m = [torch.zeros_like(w) for w in self.W]
        self.v = [torch.zeros_like(w) for w in self.W]
        self.step_t = 0
        # Factor records: the fused forward keeps every pair's normals so the
        # ES update reads them instead of drawing them again (rank >= 32; the
        # readout runs on the same pair kernels).  Sized for a chunk starting
        # at an even or an odd member.
        can_record = self.fused and c.rank >= 32 and c.dims[-1] <= 128
        self.record = can_record if record is None else (bool(record) and can_record)
        self.rec = None
        if self.record:
            self.rec = []
            for w in self.W:
                a, b = w.shape
                n_odd = c.chunk if c.accumulate > 1 and c.chunk % 2 else 0
                nbytes = max(K._lib.load().hses_factor_record_bytes(a, b, c.rank, t, c.chunk)
                             for t in (0, n_odd))
                self.rec.append(torch.empty(nbytes // 4, dtype=torch.float32, device=device))
        self._rec_at = [None] * L  # per layer: (epoch, lo) of the forward its record holds
        # Factors drawn ahead (with a record): each layer's draw is a launch of
        # its own (hses_pair_factors, full occupancy) and the forward reads the
        # record and the bf16 B operand image instead of drawing.
        self.ahead = self.record if ahead is None else (bool(ahead) and self.record)
        self.split = c.math == MATH_F32X
        # Member weights (factors drawn ahead, rows per member = samples x T a
        # multiple of 256): each hidden layer's draw writes the record alone,
        # hses_member_weights forms every member's W + sign (sigma/sqrt(r)) A B^T
        # from it, and the forward is x W_m^T (half the matrix work of the
        # factored product at 1024 rows per member); the readout, with fewer
        # rows per member, stays on the factored product.
        can_mw = (self.ahead and L > 1 and (c.rows * c.T) % 256 == 0
                  and (self.split or min(c.dims[:-2]) > 64))
        self.mw = can_mw if member_weights is None else (bool(member_weights) and can_mw)
        self.ro_counts = False  # set with the split buffers
        self.wm = None
        if self.mw:
            n_odd = c.chunk if c.accumulate > 1 and c.chunk % 2 else 0
            nbytes = max(K._lib.load().hses_member_weights_bytes(w.shape[0], w.shape[1],
                                                                 c.chunk + (n_odd > 0), c.math)
                         for w in self.W[:-1])
            self.wm = torch.empty(nbytes // 2, dtype=torch.int16, device=device)
        # The draws (VALU-bound, independent of the activations) run on a
        # second stream at the default priority: the first layer's as the
        # chunk's forward starts (beside the Poisson encode), the others once
        # the first layer's GEMM is issued, so that they share the CUs with
        # that matrix-core-bound kernel (one draw wave per SIMD fits beside
        # it); each layer's forward waits for its draw.
        # The noise cache (LoraNoiseCache, eggroll.rs:229-309; the hot path of
        # accumulated_update_cached, eggroll.rs:627): with noise_reuse = 0 a
        # member's factors depend on the layer key and its thread id only
        # (true_epoch is 0, eggroll.rs:60-65), so the records drawn for the
        # population stay valid across epochs and later steps skip the draws.
        # Off by default: the reference's training binary regenerates the
        # noise every step (accumulated_update passes no cache).
        self.noise_cache = bool(noise_cache)
        if self.noise_cache and not (self.ahead and c.noise_reuse == 0 and c.accumulate == 1):
            raise ValueError("the noise cache needs factors drawn ahead, noise_reuse = 0 and "
                             "accumulate = 1 (one record per layer for the whole population)")
        can_overlap = self.ahead and str(device).startswith("cuda") and not self.noise_cache
        self.overlap = can_overlap if overlap is None else (bool(overlap) and can_overlap)
        self.side = torch.cuda.Stream(device=device) if self.overlap else None
        self._drawn = {}  # layer -> (epoch, lo, event) of a draw issued on the side stream
        # The next forward's first-layer draw, prefetched on the side stream
        # during this one (its (epoch, lo) predicted: the next chunk, or the
        # next epoch's first) into a second record buffer, so that a step
        # starts with the Poisson encode alone; a forward for anything else
        # draws inline as before.
        self.rec0_next = torch.empty_like(self.rec[0]) if self.overlap else None
        self._prefetched = None  # (epoch, lo, event) of the draw in rec0_next
        self.img = None
        if self.ahead and not self.split:
            self.img = []
            n_odd = c.chunk if c.accumulate > 1 and c.chunk % 2 else 0
            for l, w in enumerate(self.W):
                if self.mw and l < L - 1:
                    self.img.append(None)  # member weights instead
                    continue
                a, b = w.shape
                nbytes = max(K._lib.load().hses_pair_image_bytes(a, b, c.rank, t, c.chunk)
                             for t in (0, n_odd))
                self.img.append(torch.empty(nbytes // 2, dtype=torch.int16, device=device))
        # The split (fp32-accurate) mode: every layer's draw writes the record
        # and a split operand image (hses_pair_factors_x), which the forward
        # reads in place of the bf16 image.  The last hidden layer leaves its
        # spike counts as P = log2(T) + 1 bit planes, and the readout runs on
        # the planes as P bit-packed rows per sample (rows_per_member =
        # rows * P), its outputs combined with the weights 2^p / T: by
        # linearity that is the readout of the spike rate (snn.rs:274-280),
        # sum_p 2^p plane_p / T, which the split kernels take exactly.
        self.img_x = None
        if self.split:
            if not (self.ahead and self.time_inner and c.T <= 16):
                raise ValueError("MATH_F32X needs the fused path with factors drawn ahead "
                                 "(rank a multiple of 16 in [32, 128], widths <= 128, T <= 16)")
            self.img_x = []
            n_odd = c.chunk if c.accumulate > 1 and c.chunk % 2 else 0
            for l, w in enumerate(self.W):
                if self.mw and l < L - 1:
                    self.img_x.append(None)  # member weights instead
                    continue
                a, b = w.shape
                nbytes = max(K._lib.load().hses_pair_image_x_bytes(a, b, c.rank, t, c.chunk)
                             for t in (0, n_odd))
                self.img_x.append(torch.empty(nbytes // 2, dtype=torch.int16, device=device))
            self.npl = K.count_planes(c.T)
            self.cpl = torch.empty((M, self.npl, K.fmt_width(FMT_BITS, c.dims[-2])),
                                   dtype=torch.int64, device=device)
            # a narrow readout reads the count planes directly, its member
            # weights formed per pair in LDS (hses_perturbed_readout_counts);
            # otherwise the factored split product on the planes' bit rows
            self.ro_counts = c.dims[-1] <= 32 and c.dims[-2] <= 128 and c.rows <= 128
            if self.ro_counts:
                self.img_x[-1] = None  # the readout's draw is the record alone
            else:
                self.ylog = torch.empty((1, M * self.npl, c.dims[-1]), dtype=torch.float32,
                                        device=device)
                self.plane_w = torch.tensor([2.0 ** p / c.T for p in range(self.npl)],
                                            dtype=torch.float32, device=device).view(1, -1, 1)

    # -- forward -------------------------------------------------------------
    def spikes_tm(self, l):
        """Layer l's input spikes as a time-major (T, M, words) view."""
        return self.spk[l].transpose(0, 1) if self.time_inner else self.spk[l]

    def chunk_seeds(self, lo):
        """Poisson seeds of the chunk starting at member lo.  The kernel seeds
        element (row, col) of a call with 1000000007*(row*in + col) + (s0^s1^s2^s3);
        adding 1000000007 * (first row * in) to the mixed seed makes a chunk's
        encode equal to rows lo*rows.. of a whole-population encode."""
        c = self.cfg
        s0, s1, s2, s3 = (int(v) & 0xFFFFFFFF for v in c.poisson_seed)
        mix = (s0 ^ s1 ^ s2 ^ s3) + 1000000007 * lo * c.rows * c.dims[0]
        return (mix & 0xFFFFFFFF, 0, 0, 0)

    def poisson(self, lo=0):
        c = self.cfg
        rows = slice(lo * c.rows, (lo + c.chunk) * c.rows)
        if self.ppool is not None:
            K.poisson_encode_pool(self.ppool, c.T, self.chunk_seeds(lo), out=self.spk[0],
                                  rows_index=self.index[rows], time_inner=self.time_inner)
            return
        K.poisson_encode(self.pool, c.T, self.chunk_seeds(lo), FMT_BITS, out=self.spk[0],
                         rows_index=self.index[rows], time_inner=self.time_inner)

    def hidden_layer(self, l, epoch, lo=0):
        c = self.cfg
        a = c.dims[l + 1]
        if self.fused:
            # feeds the readout: only its spike rates (split mode: spike-count
            # planes) are used
            last = l == self.L - 2
            img = self._draw(l, epoch, lo)
            if self.mw:
                # img: the member weights of this layer
                counts = self.cpl if last and self.split else None
                K.perturbed_linear_lif_mw(self.spk[l], img, a, c.dims[l], lo, c.chunk, c.rows, c.T,
                                          c.tau_m, c.v_th, math=c.math,
                                          spikes=None if last else self.spk[l + 1],
                                          rate=self.rate if last and not self.split else None,
                                          counts=counts, time_inner=self.time_inner)
                self._rec_at[l] = self._rec_key(epoch, lo)
                return
            if last and self.split:
                K.perturbed_linear_lif_counts_x(self.spk[l], self.W[l], c.rank, c.sigma, lo,
                                                c.chunk, c.rows, c.T, c.tau_m, c.v_th,
                                                self.rec[l], img, counts=self.cpl,
                                                time_inner=self.time_inner)
                self._rec_at[l] = self._rec_key(epoch, lo)
                return
            K.perturbed_linear_lif(self.spk[l], self.W[l], c.keys[l], c.rank, c.sigma, epoch,
                                   c.noise_reuse, lo, c.chunk, c.rows, c.T, c.tau_m, c.v_th,
                                   spikes=None if last else self.spk[l + 1],
                                   rate=self.rate if last else None,
                                   want_spikes=not last, want_rate=last,
                                   rec=self.rec[l] if self.rec else None, img=img,
                                   time_inner=self.time_inner, math=c.math)
            if self.rec:
                self._rec_at[l] = self._rec_key(epoch, lo)
            return
        cur = self.cur[:, :, :a] if a == self.cur.shape[2] else \
            self.cur.view(-1)[: c.T * self.M * a].view(c.T, self.M, a)
        K.perturbed_linear(self.spk[l], self.W[l], c.keys[l], c.rank, c.sigma, epoch,
                           c.noise_reuse, lo, c.chunk, c.rows, x_fmt=FMT_BITS, n_time=c.T,
                           math=c.math, out=cur)
        K.lif_scan(cur, c.tau_m, c.v_th, fmt=FMT_BITS, out=self.spk[l + 1])

    def readout(self, epoch, lo=0):
        c = self.cfg
        if self.split:
            img = self._draw(self.L - 1, epoch, lo)
            if self.ro_counts:
                K.readout_counts(self.cpl, self.W[-1], c.rank, c.sigma, lo, c.chunk, c.rows, c.T,
                                 self.rec[-1], out=self.logits)
            else:
                x = self.cpl.view(1, self.M * self.npl, -1)
                K.perturbed_linear(x, self.W[-1], c.keys[-1], c.rank, c.sigma, epoch,
                                   c.noise_reuse, lo, c.chunk, c.rows * self.npl, x_fmt=FMT_BITS,
                                   n_time=1, math=MATH_F32X, out=self.ylog, rec=self.rec[-1],
                                   img=img)
                torch.sum(self.ylog.view(self.M, self.npl, -1) * self.plane_w, 1,
                          out=self.logits)
            self._rec_at[-1] = self._rec_key(epoch, lo)
            labels = self.labels[lo * c.rows:(lo + c.chunk) * c.rows]
            return K.member_fitness(self.logits, labels, c.chunk, c.rows, c.reward,
                                    out=self.raw[lo:lo + c.chunk], correct=self.correct)
        if not self.fused:
            K.spike_rate(self.spk[self.L - 1], FMT_BITS, c.dims[-2], out=self.rate)
        img = self._draw(self.L - 1, epoch, lo)
        K.perturbed_linear(self.rate, self.W[-1], c.keys[-1], c.rank, c.sigma, epoch,
                           c.noise_reuse, lo, c.chunk, c.rows, x_fmt=FMT_F32, n_time=1,
                           math=c.math, out=self.logits.view(1, self.M, -1),
                           rec=self.rec[-1] if self.rec else None, img=img)
        if self.rec:
            self._rec_at[-1] = self._rec_key(epoch, lo)
        labels = self.labels[lo * c.rows:(lo + c.chunk) * c.rows]
        return K.member_fitness(self.logits, labels, c.chunk, c.rows, c.reward,
                                out=self.raw[lo:lo + c.chunk], correct=self.correct)

    def _draw_factors(self, l, epoch, lo, rec=None):
        """Layer l's factors of the chunk into its record (or `rec`) and,
        without member weights, its operand image, on the current stream."""
        c = self.cfg
        a, b = self.W[l].shape
        img = self.img_x if self.split else self.img
        # the record alone: member weights, or the readout on count planes
        bare = (self.mw and l < self.L - 1) or (self.ro_counts and l == self.L - 1)
        K.pair_factors(c.keys[l], c.rank, c.sigma, epoch, c.noise_reuse, lo, c.chunk, a, b,
                       self.rec[l] if rec is None else rec, None if bare else img[l],
                       split=self.split and not bare)

    def _next_forward(self, epoch, lo):
        """The (epoch, lo) a training loop runs after this forward."""
        c = self.cfg
        return (epoch, lo + c.chunk) if lo + c.chunk < c.n else (epoch + 1, 0)

    def _issue_draws(self, epoch, lo, layers):
        """Layers' draws of the chunk on the side stream, after the work
        issued so far on the current stream (the previous update still reads
        the records)."""
        start = torch.cuda.Event()
        start.record()
        with torch.cuda.stream(self.side):
            self.side.wait_event(start)
            for l in layers:
                self._draw_factors(l, epoch, lo)
                done = torch.cuda.Event()
                done.record(self.side)
                self._drawn[l] = (epoch, lo, done)

    def _rec_key(self, epoch, lo):
        """What a record holds: the (epoch, lo) of its draw, or with the noise
        cache (lo) alone (the factors do not depend on the epoch)."""
        return (0 if self.noise_cache else epoch, lo)

    def _draw(self, l, epoch, lo):
        """Layer l's operand of the chunk: with member weights every member's
        W_m formed from the record, else the operand image; None when the
        forward draws its factors itself.  The draw itself was issued on the
        side stream (waited for here) or runs now; with the noise cache a
        record that already holds the chunk is not drawn again."""
        img = self.img_x if self.split else self.img
        if not img:
            return None
        drawn = self._drawn.pop(l, None)
        if self.noise_cache and self._rec_at[l] == self._rec_key(epoch, lo):
            pass  # the record (and operand image) of an earlier step still hold these factors
        elif drawn is not None and drawn[:2] == (epoch, lo):
            torch.cuda.current_stream().wait_event(drawn[2])
        else:
            self._draw_factors(l, epoch, lo)
        c = self.cfg
        a, b = self.W[l].shape
        out = img[l]
        if self.mw and l < self.L - 1:
            n_wm = K._lib.load().hses_member_weights_bytes(a, b, c.chunk, c.math) // 2
            out = K.member_weights(self.W[l], c.rank, c.sigma, lo, c.chunk, self.rec[l],
                                   math=c.math, out=self.wm[:n_wm])
        if self.overlap and l == 0 and drawn is not None:
            # the other layers' draws, beside the first layer's GEMM
            self._issue_draws(epoch, lo, range(1, self.L))
        if self.overlap and self.mw and l == min(1, self.L - 2) and drawn is not None:
            # the next forward's first-layer draw, beside the later layers'
            # GEMMs (its buffer was last read by the previous step, which the
            # side stream has waited for; with an operand image layer 0 has
            # one image only, so only the record-only draw is prefetched)
            ne, nl = self._next_forward(epoch, lo)
            issued = torch.cuda.Event()
            issued.record()
            with torch.cuda.stream(self.side):
                self.side.wait_event(issued)
                self._draw_factors(0, ne, nl, rec=self.rec0_next)
                done = torch.cuda.Event()
                done.record(self.side)
            self._prefetched = (ne, nl, done)
        return out

    def forward(self, epoch=0, lo=0, mark=None):
        """Raw fitness of the chunk of members [lo, lo + chunk) (a view of self.raw).
        mark(name), when given, is called after each stage is issued (e.g. to
        record an event on the current stream)."""
        mark = mark or (lambda name: None)
        if self.overlap:
            pre, self._prefetched = self._prefetched, None
            if pre is not None and pre[:2] == (epoch, lo):
                # the prefetched draw: its buffer becomes layer 0's record
                self.rec[0], self.rec0_next = self.rec0_next, self.rec[0]
                self._drawn[0] = pre
            else:
                self._issue_draws(epoch, lo, [0])
        self.poisson(lo)
        mark("poisson")
        for l in range(self.L - 1):
            self.hidden_layer(l, epoch, lo)
            mark(f"hidden{l}")
        fit = self.readout(epoch, lo)
        mark("readout")
        return fit

    def _grad(self, l, fit, lo, epoch, scale, accumulate=False):
        """grads[l] (+)= scale * sum_m fit[m] A_m B_m^T over members [lo, lo + len(fit)),
        from the factor records when they hold this epoch's chunk."""
        c = self.cfg
        a, b = self.W[l].shape
        if (self.rec is not None and self._rec_at[l] == self._rec_key(epoch, lo)
                and fit.numel() == c.chunk):
            K.es_update_rec(fit, lo, self.rec[l], c.rank, c.sigma, a, b, scale,
                            out=self.grads[l], accumulate=accumulate)
        else:
            K.es_update(fit, lo, c.keys[l], c.rank, c.sigma, epoch, c.noise_reuse, a, b, scale,
                        out=self.grads[l], accumulate=accumulate)

    # -- update --------------------------------------------------------------
    def _solve(self, l, gscale):
        c = self.cfg
        K.solver_step(c.solver, c.lr, self.W[l], self.grads[l], self.m[l], self.v[l],
                      step_t=self.step_t, beta1=c.beta1, beta2=c.beta2, eps=c.eps,
                      wd=c.weight_decay if c.solver == ADAMW else 0.0, gscale=gscale)

    def _clip(self):
        """TrustRegion's clip factor over all layers' gradients, or None."""
        if self.cfg.max_norm <= 0.0:
            return None
        return K.clip_global_norm(self.grads, self.cfg.max_norm)

    def update(self, raw_fit, epoch=0):
        c = self.cfg
        z, _ = K.convert_fitnesses(raw_fit)
        scale = np.float32(-math.sqrt(c.n) / c.n)   # -g * sqrt(N) with g = (1/N) sum (eggroll.rs:403)
        self.step_t += 1
        clip = c.max_norm > 0.0  # the global norm needs every gradient before any step
        for l in range(self.L):
            self._grad(l, z, 0, epoch, scale)
            if not clip:
                self._solve(l, None)
        if clip:
            gscale = self._clip()
            for l in range(self.L):
                self._solve(l, gscale)
        return z

    def step(self, epoch=0, mark=None):
        """One ES step; returns the raw fitness (N,).  self.correct counts the
        step's rows whose argmax is the label.  mark: see forward (plus "update")."""
        self.correct.zero_()
        if self.cfg.accumulate == 1:
            fit = self.forward(epoch, mark=mark)
            self.update(fit, epoch)
            if mark:
                mark("update")
            return fit
        return self.step_accumulate(epoch)

    def step_accumulate(self, epoch=0):
        """The K-chunk step (accumulate_train.rs:770-944) with the parameters
        frozen over the chunks.  Per chunk: forward, raw-fitness sums, and
        grad_acc += sum_i raw_i A_i B_i^T.  The ones sum sum_i A_i B_i^T of
        combine_affine_grads vanishes over the noiser stream's antithetic pairs
        (A negated for odd thread ids, B shared), also across chunk boundaries,
        so it is only formed for an unpaired last member (odd N)."""
        c = self.cfg
        for k in range(c.accumulate):
            lo = k * c.chunk
            raw = self.forward(epoch, lo)
            K.fitness_moments(raw, self.moments, accumulate=k > 0)
            for l in range(self.L):
                self._grad(l, raw, lo, epoch, np.float32(1.0), accumulate=k > 0)
        one = torch.ones(1, dtype=torch.float32, device=self.dev) if c.n % 2 else None
        self.step_t += 1
        for l in range(self.L):
            a, b = self.W[l].shape
            ones = None
            if one is not None:
                ones = K.es_update(one, c.n - 1, c.keys[l], c.rank, c.sigma, epoch, c.noise_reuse,
                                   a, b, np.float32(1.0))
            K.combine_affine(self.grads[l], self.moments, c.n, ones_acc=ones, out=self.grads[l])
        gscale = self._clip()
        for l in range(self.L):
            self._solve(l, gscale)
        return self.raw
