"""Torch-tensor wrappers over the libhses entry points.

PyTorch supplies device memory and the current stream; every computation runs
in libhses.so.  Each wrapper validates that its tensors are contiguous device
tensors of the expected dtype before calling the C ABI.
"""
import ctypes

import torch

from . import _lib
from ._lib import (FMT_BF16, FMT_BITS, FMT_F32, FMT_U8, MATH_BF16, MATH_F32, MATH_F32X,  # noqa: F401
                   REWARD_BINARY, REWARD_LOGLIK)

_FMT_DTYPE = {FMT_F32: torch.float32, FMT_BF16: torch.bfloat16, FMT_U8: torch.uint8,
              FMT_BITS: torch.int64}


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t, dtype, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


_WORK = {}


def _workspace(nbytes, device):
    """A cached device workspace of at least nbytes (one per device and stream)."""
    key = (str(device), torch.cuda.current_stream().cuda_stream)
    buf = _WORK.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORK[key] = buf
    return buf


def fmt_width(fmt, width):
    """Storage units per row of `width` activations in format `fmt`."""
    return (width + 63) // 64 if fmt == FMT_BITS else width


def init(device=0):
    _lib.call("hses_init", device)


def bm_stats():
    out = (ctypes.c_uint32 * 2)()
    _lib.call("hses_bm_stats", out)
    return int(out[0]), int(out[1])


def noise_seed(key, true_epoch, true_thread):
    return int(_lib.load().hses_noise_seed(key & (2**64 - 1), true_epoch, true_thread))


def bm_eval(k_lo, n, device="cuda"):
    """Device Box-Muller halves for unit indices [k_lo, k_lo+n)."""
    lg = torch.empty(n, dtype=torch.float32, device=device)
    rad = torch.empty_like(lg)
    cs = torch.empty_like(lg)
    _lib.call("hses_bm_eval", k_lo, n, _p(lg), _p(rad), _p(cs), _stream())
    return lg, rad, cs


def lora_factors(base_sigma, key, rank, epoch, noise_reuse, tids, a, b, device="cuda"):
    """batched_lora_noise: tids is an int tensor/sequence or (tid_lo, n)."""
    if isinstance(tids, tuple):
        tid_lo, n = tids
        d_tids = None
    else:
        d_tids = torch.as_tensor(tids, dtype=torch.int32, device=device).contiguous()
        tid_lo, n = 0, d_tids.numel()
    A = torch.empty((n, a, rank), dtype=torch.float32, device=device)
    B = torch.empty((n, b, rank), dtype=torch.float32, device=device)
    _lib.call("hses_lora_factors", base_sigma, key & (2**64 - 1), rank, epoch, noise_reuse,
              tid_lo, _p(d_tids), n, a, b, _p(A), _p(B), _stream())
    return A, B


def nonlora_noise(base_sigma, key, epoch, noise_reuse, tids, a, b, device="cuda"):
    if isinstance(tids, tuple):
        tid_lo, n = tids
        d_tids = None
    else:
        d_tids = torch.as_tensor(tids, dtype=torch.int32, device=device).contiguous()
        tid_lo, n = 0, d_tids.numel()
    out = torch.empty((n, a, b), dtype=torch.float32, device=device)
    _lib.call("hses_nonlora_noise", base_sigma, key & (2**64 - 1), epoch, noise_reuse, tid_lo,
              _p(d_tids), n, a, b, _p(out), _stream())
    return out


def poisson_encode(p, T, seeds=(0, 0, 0, 0), fmt=FMT_F32, out=None, rows_index=None,
                   time_inner=False):
    """(rows, in_dim) probabilities -> (T, rows, width) spikes in `fmt`, or
    (rows, T, width) with time_inner (each row's T words adjacent).  With
    rows_index (int32, length R) output row i encodes p[rows_index[i]]."""
    _dev(p, torch.float32, "p")
    prow, in_dim = p.shape
    rows = prow
    if rows_index is not None:
        _dev(rows_index, torch.int32, "rows_index")
        rows = rows_index.numel()
    units = fmt_width(fmt, in_dim)
    shape = (rows, T, units) if time_inner else (T, rows, units)
    if out is None:
        out = torch.empty(shape, dtype=_FMT_DTYPE[fmt], device=p.device)
    _dev(out, _FMT_DTYPE[fmt], "out")
    if tuple(out.shape) != shape:
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {shape}")
    stride, plane = (T * units, units) if time_inner else (units, rows * units)
    s0, s1, s2, s3 = (int(s) & 0xFFFFFFFF for s in seeds)
    _lib.call("hses_poisson_encode_planes", _p(p), prow, _p(rows_index), rows, in_dim, in_dim, T,
              s0, s1, s2, s3, _p(out), fmt, stride, plane, _stream())
    return out


class PoissonPool:
    """A pool of probability rows (pool_rows, in_dim) prepared once for
    repeated bit-packed encodes of gathered rows (hses_poisson_pool_prepare):
    per row the exact thresholds of the elements that can fire."""

    def __init__(self, p):
        _dev(p, torch.float32, "p")
        self.rows, self.in_dim = p.shape
        self.nbytes = int(_lib.load().hses_poisson_pool_bytes(self.rows, self.in_dim))
        if self.nbytes == 0:
            raise ValueError(f"no prepared pool for in_dim {self.in_dim} (at most 2048)")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=p.device)
        _lib.call("hses_poisson_pool_prepare", _p(p), self.rows, self.in_dim, p.stride(0),
                  _p(self.buf), self.nbytes, _stream())


def poisson_encode_pool(pool, T, seeds=(0, 0, 0, 0), out=None, rows_index=None,
                        time_inner=False):
    """poisson_encode(p, T, seeds, FMT_BITS, out, rows_index, time_inner) on
    the PoissonPool prepared from p: the same spikes."""
    rows = pool.rows
    if rows_index is not None:
        _dev(rows_index, torch.int32, "rows_index")
        rows = rows_index.numel()
    units = fmt_width(FMT_BITS, pool.in_dim)
    shape = (rows, T, units) if time_inner else (T, rows, units)
    if out is None:
        out = torch.empty(shape, dtype=_FMT_DTYPE[FMT_BITS], device=pool.buf.device)
    _dev(out, _FMT_DTYPE[FMT_BITS], "out")
    if tuple(out.shape) != shape:
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {shape}")
    stride, plane = (T * units, units) if time_inner else (units, rows * units)
    s0, s1, s2, s3 = (int(s) & 0xFFFFFFFF for s in seeds)
    _lib.call("hses_poisson_encode_pool", _p(pool.buf), pool.nbytes, pool.rows, pool.in_dim,
              _p(rows_index), rows, T, s0, s1, s2, s3, _p(out), stride, plane, _stream())
    return out


def spike_rate(spikes, fmt, h, out=None):
    """(T, rows, units) spikes in `fmt` -> (rows, h) fp32 mean over T."""
    _dev(spikes, _FMT_DTYPE[fmt], "spikes")
    T, rows, units = spikes.shape
    if out is None:
        out = torch.empty((rows, h), dtype=torch.float32, device=spikes.device)
    _lib.call("hses_spike_rate", _p(spikes), fmt, units, T, rows, h, _p(out), _stream())
    return out


def lif_scan(cur, tau_m, v_th, v0=None, fmt=FMT_F32, want_v=False, out=None):
    """cur (T, rows, h) fp32 -> spikes (T, rows, width) in `fmt` [, v_final (rows, h)]."""
    _dev(cur, torch.float32, "cur")
    T, rows, h = cur.shape
    if v0 is not None:
        _dev(v0, torch.float32, "v0")
    units = fmt_width(fmt, h)
    spk = out if out is not None else torch.empty((T, rows, units), dtype=_FMT_DTYPE[fmt],
                                                  device=cur.device)
    _dev(spk, _FMT_DTYPE[fmt], "spikes")
    v_out = torch.empty((rows, h), dtype=torch.float32, device=cur.device) if want_v else None
    _lib.call("hses_lif_scan", _p(cur), _p(v0), T, rows, h, h, tau_m, v_th, _p(spk), fmt, units,
              _p(v_out), _stream())
    return (spk, v_out) if want_v else spk


def factor_record(a, b, rank, tid_lo, n, device="cuda"):
    """A factor record buffer for the members [tid_lo, tid_lo + n) of an (a, b)
    parameter (hses_factor_record_bytes)."""
    nbytes = int(_lib.load().hses_factor_record_bytes(a, b, rank, tid_lo, n))
    if nbytes == 0:
        raise ValueError("no factor record for this shape")
    return torch.empty(nbytes // 4, dtype=torch.float32, device=device)


def _rec_arg(rec):
    _dev(rec, torch.float32, "rec")
    return _p(rec), rec.numel() * 4


def pair_image(a, b, rank, tid_lo, n, device="cuda"):
    """A bf16 operand image buffer (stored as int16) for the factors of members
    [tid_lo, tid_lo + n) of an (a, b) parameter (hses_pair_image_bytes)."""
    nbytes = int(_lib.load().hses_pair_image_bytes(a, b, rank, tid_lo, n))
    if nbytes == 0:
        raise ValueError("no operand image for this shape")
    return torch.empty(nbytes // 2, dtype=torch.int16, device=device)


def _img_arg(img):
    _dev(img, torch.int16, "img")
    return _p(img), img.numel() * 2


def pair_image_x(a, b, rank, tid_lo, n, device="cuda"):
    """A split (fp16 high + low parts, stored as int16) operand image buffer for
    the fp32-accurate forwards (hses_pair_image_x_bytes)."""
    nbytes = int(_lib.load().hses_pair_image_x_bytes(a, b, rank, tid_lo, n))
    if nbytes == 0:
        raise ValueError("no operand image for this shape")
    return torch.empty(nbytes // 2, dtype=torch.int16, device=device)


def split_pair_image(a, b, rank, sigma, tid_lo, n, rec, img):
    """Fill the split operand image `img` (pair_image_x) from the factor record
    `rec` of the same members (hses_pair_image_x)."""
    _lib.call("hses_pair_image_x", a, b, rank, sigma, tid_lo, n, *_rec_arg(rec), *_img_arg(img),
              _stream())


def pair_factors(key, rank, sigma, epoch, noise_reuse, tid_lo, n, a, b, rec, img, split=False):
    """Draw every pair's factors of members [tid_lo, tid_lo + n) into the factor
    record `rec` and the operand image `img` (hses_pair_factors); the forwards
    given rec= and img= then read them instead of drawing.  split: `img` is the
    split image (pair_image_x) for the fp32-accurate forwards
    (hses_pair_factors_x).  img=None: the record alone (member_weights'
    input)."""
    img_args = (None, 0) if img is None else _img_arg(img)
    _lib.call("hses_pair_factors_x" if split else "hses_pair_factors", key & (2**64 - 1), rank,
              sigma, epoch, noise_reuse, tid_lo, n, a, b, *_rec_arg(rec), *img_args, _stream())


def member_weights(W, rank, sigma, tid_lo, n, rec, math=MATH_F32X, out=None):
    """Every member's perturbed weights W + sign_m (sigma/sqrt(r)) A_m B_m^T from
    the factor record (hses_member_weights): int16 storage of bf16 (math BF16)
    or of fp16 high and low parts of 1024 W_m (math F32X), chunk-major
    ([part][input chunk of 64][a][64]) per member."""
    a, b = W.shape
    _dev(W, torch.float32, "W")
    nbytes = int(_lib.load().hses_member_weights_bytes(a, b, n, math))
    if nbytes == 0:
        raise ValueError("no member weights for this shape / math")
    if out is None:
        out = torch.empty(nbytes // 2, dtype=torch.int16, device=W.device)
    _dev(out, torch.int16, "out")
    _lib.call("hses_member_weights", _p(W), a, b, rank, sigma, tid_lo, n, *_rec_arg(rec), math,
              _p(out), out.numel() * 2, _stream())
    return out


def perturbed_linear_mw(x, wm, a, b, tid_lo, n, rows_per_member, n_time=1, math=MATH_F32X,
                        out=None):
    """y = x W_m^T on member weights (hses_perturbed_linear_mw); x bit-packed
    (n_time, M, words(b)) or 2-D; returns y (n_time, M, a) fp32."""
    _dev(x, _FMT_DTYPE[FMT_BITS], "x")
    _dev(wm, torch.int16, "wm")
    units = fmt_width(FMT_BITS, b)
    M = n * rows_per_member
    if x.shape[-1] != units or x.numel() != n_time * M * units:
        raise ValueError(f"x has shape {tuple(x.shape)}, expected ({n_time}, {M}, {units})")
    if out is None:
        out = torch.empty((n_time, M, a), dtype=torch.float32, device=x.device)
    _dev(out, torch.float32, "out")
    if out.numel() != n_time * M * a:
        raise ValueError("out has the wrong size")
    _lib.call("hses_perturbed_linear_mw", _p(x), FMT_BITS, units, M * units, n_time, a, b, tid_lo,
              n, rows_per_member, math, _p(wm), wm.numel() * 2, _p(out), a, M * a, _stream())
    return out if n_time > 1 or x.dim() == 3 else out[0]


def perturbed_linear_lif_mw(x, wm, a, b, tid_lo, n, rows_per_member, n_time, tau_m, v_th,
                            math=MATH_F32X, spikes=None, rate=None, counts=None,
                            time_inner=False):
    """The fused forward + LIF on member weights (hses_perturbed_linear_lif_mw):
    any of spikes (time-major (T, M, words), or (M, T, words) with time_inner),
    rate (M, a) and counts (M, P, words) given as tensors (or True to allocate)
    is written; returns (spikes, rate, counts)."""
    _dev(x, _FMT_DTYPE[FMT_BITS], "x")
    _dev(wm, torch.int16, "wm")
    units = fmt_width(FMT_BITS, b)
    M = n * rows_per_member
    if x.shape[-1] != units or x.numel() != n_time * M * units:
        raise ValueError(f"x has shape {tuple(x.shape)}, expected ({n_time}, {M}, {units})")
    wa = fmt_width(FMT_BITS, a)
    npl = count_planes(n_time)
    if spikes is True:
        spikes = torch.empty((M, n_time, wa) if time_inner else (n_time, M, wa),
                             dtype=torch.int64, device=x.device)
    if rate is True:
        rate = torch.empty((M, a), dtype=torch.float32, device=x.device)
    if counts is True:
        counts = torch.empty((M, npl, wa), dtype=torch.int64, device=x.device)
    for t, nm, dt, numel in ((spikes, "spikes", torch.int64, n_time * M * wa),
                             (rate, "rate", torch.float32, M * a),
                             (counts, "counts", torch.int64, M * npl * wa)):
        if t is not None:
            _dev(t, dt, nm)
            if t.numel() != numel:
                raise ValueError(f"{nm} has the wrong size")
    if time_inner:
        xs, xp, ss, sp = n_time * units, units, n_time * wa, wa
    else:
        xs, xp, ss, sp = units, M * units, wa, M * wa
    _lib.call("hses_perturbed_linear_lif_mw", _p(x), FMT_BITS, xs, xp, n_time, a, b, tid_lo, n,
              rows_per_member, tau_m, v_th, math, _p(wm), wm.numel() * 2,
              _p(spikes) if spikes is not None else None, ss, sp,
              _p(rate) if rate is not None else None, a,
              _p(counts) if counts is not None else None, npl * wa, _stream())
    return spikes, rate, counts


def perturbed_linear(x, W, key, rank, sigma, epoch, noise_reuse, tid_lo, n, rows_per_member,
                     x_fmt=FMT_F32, x_width=None, n_time=1, math=MATH_F32, out=None, act=0,
                     out_bf16=False, rec=None, img=None):
    """Batched do_mm.  x is (n_time, n*rows_per_member, units) in x_fmt (or 2-D
    when n_time == 1); returns y (n_time, n*rows_per_member, a) fp32 (bf16 with
    out_bf16), passed through the activation `act` (hses_act) when it is not 0.
    With `rec` (factor_record) the pairs' normals are also kept there; with
    `rec` and `img` filled by pair_factors they are read from there instead;
    with math=MATH_F32X, `img` is the split image (split_pair_image) and y is
    fp32-accurate (hses_perturbed_linear_pre_x)."""
    a, b = W.shape
    _dev(W, torch.float32, "W")
    _dev(x, _FMT_DTYPE[x_fmt], "x")
    units = fmt_width(x_fmt, b)
    M = n * rows_per_member
    if x.shape[-1] != units or x.numel() != n_time * M * units:
        raise ValueError(f"x has shape {tuple(x.shape)}, expected ({n_time}, {M}, {units})")
    ydt = torch.bfloat16 if out_bf16 else torch.float32
    if out is None:
        out = torch.empty((n_time, M, a), dtype=ydt, device=W.device)
    _dev(out, ydt, "out")
    if out.numel() != n_time * M * a:
        raise ValueError("out has the wrong size")
    wbytes = int(_lib.load().hses_perturbed_linear_workspace(a, b, rank, n, rows_per_member,
                                                              n_time, math))
    work = _workspace(wbytes, W.device)
    if img is not None:
        if rec is None or act or out_bf16 or math not in (MATH_BF16, MATH_F32X):
            raise ValueError("factors drawn ahead need rec, bf16 or split math and a plain "
                             "fp32 output")
        _lib.call("hses_perturbed_linear_pre_x" if math == MATH_F32X else
                  "hses_perturbed_linear_pre", _p(x), x_fmt, units, M * units, n_time, _p(W), a,
                  b, rank, sigma, tid_lo, n, rows_per_member, _p(out), a, M * a, _p(work),
                  wbytes, *_rec_arg(rec), *_img_arg(img), _stream())
    elif rec is not None:
        if act or out_bf16:
            raise ValueError("the factor record is kept by the plain fp32-output forward only")
        _lib.call("hses_perturbed_linear_rec", _p(x), x_fmt, units, M * units, n_time, _p(W), a,
                  b, key & (2**64 - 1), rank, sigma, epoch, noise_reuse, tid_lo, n,
                  rows_per_member, _p(out), a, M * a, math, _p(work), wbytes, *_rec_arg(rec),
                  _stream())
    elif act or out_bf16:
        _lib.call("hses_perturbed_linear_act", _p(x), x_fmt, units, M * units, n_time, _p(W), a,
                  b, key & (2**64 - 1), rank, sigma, epoch, noise_reuse, tid_lo, n,
                  rows_per_member, _p(out), a, M * a, math, 0, act,
                  FMT_BF16 if out_bf16 else FMT_F32, _p(work), wbytes, _stream())
    else:
        _lib.call("hses_perturbed_linear", _p(x), x_fmt, units, M * units, n_time, _p(W), a, b,
                  key & (2**64 - 1), rank, sigma, epoch, noise_reuse, tid_lo, n, rows_per_member,
                  _p(out), a, M * a, math, _p(work), wbytes, _stream())
    return out if n_time > 1 or x.dim() == 3 else out[0]


def perturbed_linear_t(x, W, key, rank, sigma, epoch, noise_reuse, tid_lo, n, rows_per_member,
                       x_fmt=FMT_F32, n_time=1, math=MATH_F32, out=None, act=0, out_bf16=False):
    """Batched do_Tmm: y = x W + (x A_m) B_m^T for W of shape (a, b).  x is
    (n_time, n*rows_per_member, a) in x_fmt (or 2-D when n_time == 1);
    returns y (n_time, n*rows_per_member, b) fp32."""
    a, b = W.shape
    _dev(W, torch.float32, "W")
    _dev(x, _FMT_DTYPE[x_fmt], "x")
    units = fmt_width(x_fmt, a)
    M = n * rows_per_member
    if x.shape[-1] != units or x.numel() != n_time * M * units:
        raise ValueError(f"x has shape {tuple(x.shape)}, expected ({n_time}, {M}, {units})")
    ydt = torch.bfloat16 if out_bf16 else torch.float32
    if out is None:
        out = torch.empty((n_time, M, b), dtype=ydt, device=W.device)
    _dev(out, ydt, "out")
    if out.numel() != n_time * M * b:
        raise ValueError("out has the wrong size")
    wbytes = int(_lib.load().hses_perturbed_linear_t_workspace(a, b, rank, n, rows_per_member,
                                                                n_time, math))
    work = _workspace(wbytes, W.device)
    if act or out_bf16:
        _lib.call("hses_perturbed_linear_act", _p(x), x_fmt, units, M * units, n_time, _p(W), a,
                  b, key & (2**64 - 1), rank, sigma, epoch, noise_reuse, tid_lo, n,
                  rows_per_member, _p(out), b, M * b, math, 1, act,
                  FMT_BF16 if out_bf16 else FMT_F32, _p(work), wbytes, _stream())
    else:
        _lib.call("hses_perturbed_linear_t", _p(x), x_fmt, units, M * units, n_time, _p(W), a,
                  b, key & (2**64 - 1), rank, sigma, epoch, noise_reuse, tid_lo, n,
                  rows_per_member, _p(out), b, M * b, math, _p(work), wbytes, _stream())
    return out if n_time > 1 or x.dim() == 3 else out[0]


def perturbed_linear_lif(x, W, key, rank, sigma, epoch, noise_reuse, tid_lo, n,
                         rows_per_member, n_time, tau_m, v_th, spikes=None, rate=None,
                         want_spikes=True, want_rate=False, rec=None, img=None,
                         time_inner=False, math=MATH_BF16):
    """Perturbed forward fused with LIF.  x is bit-packed (n_time, M, words(b));
    returns (spikes (n_time, M, words(a)) int64 or None, rate (M, a) or None).
    With time_inner, x and spikes are (M, n_time, words) (each row's time steps
    adjacent).  With `rec` (factor_record) the pairs' normals are also kept
    there; with `rec` and `img` filled by pair_factors they are read from there
    instead.  math=MATH_F32X (with `img` the split image of split_pair_image):
    fp32-accurate currents (hses_perturbed_linear_lif_pre_x)."""
    a, b = W.shape
    _dev(W, torch.float32, "W")
    _dev(x, _FMT_DTYPE[FMT_BITS], "x")
    units = fmt_width(FMT_BITS, b)
    M = n * rows_per_member
    if x.shape[-1] != units or x.numel() != n_time * M * units:
        raise ValueError(f"x has shape {tuple(x.shape)}, expected ({n_time}, {M}, {units})")
    wa = fmt_width(FMT_BITS, a)
    if want_spikes and spikes is None:
        shape = (M, n_time, wa) if time_inner else (n_time, M, wa)
        spikes = torch.empty(shape, dtype=torch.int64, device=W.device)
    if want_rate and rate is None:
        rate = torch.empty((M, a), dtype=torch.float32, device=W.device)
    if spikes is not None:
        _dev(spikes, torch.int64, "spikes")
        if spikes.numel() != n_time * M * wa:
            raise ValueError("spikes has the wrong size")
    if rate is not None:
        _dev(rate, torch.float32, "rate")
        if rate.numel() != M * a:
            raise ValueError("rate has the wrong size")
    if math not in (MATH_BF16, MATH_F32X) or (math == MATH_F32X and img is None):
        raise ValueError("the fused forward takes bf16 math, or split math with img")
    wbytes = int(_lib.load().hses_perturbed_linear_workspace(a, b, rank, n, rows_per_member,
                                                              n_time, math))
    work = _workspace(wbytes, W.device)
    if time_inner:
        xs, xp, ss, sp = n_time * units, units, n_time * wa, wa
        if x.dim() != 3 or x.shape[0] != M or (spikes is not None and spikes.shape[0] != M):
            raise ValueError("time_inner x and spikes are (M, n_time, words)")
    else:
        xs, xp, ss, sp = units, M * units, wa, M * wa
    args = (_p(x), FMT_BITS, xs, xp, n_time, _p(W), a, b, key & (2**64 - 1), rank,
            sigma, epoch, noise_reuse, tid_lo, n, rows_per_member, tau_m, v_th,
            _p(spikes) if spikes is not None else None, ss, sp,
            _p(rate) if rate is not None else None, a, _p(work), wbytes)
    if img is not None:
        if rec is None:
            raise ValueError("factors drawn ahead need rec")
        _lib.call("hses_perturbed_linear_lif_pre_x" if math == MATH_F32X else
                  "hses_perturbed_linear_lif_pre", _p(x), FMT_BITS, xs, xp, n_time,
                  _p(W), a, b, rank, sigma, tid_lo, n, rows_per_member, tau_m, v_th,
                  _p(spikes) if spikes is not None else None, ss, sp,
                  _p(rate) if rate is not None else None, a, _p(work), wbytes, *_rec_arg(rec),
                  *_img_arg(img), _stream())
    elif rec is None:
        _lib.call("hses_perturbed_linear_lif", *args, _stream())
    else:
        _lib.call("hses_perturbed_linear_lif_rec", *args, *_rec_arg(rec), _stream())
    return spikes, rate


def readout_counts(counts, W, rank, sigma, tid_lo, n, rows_per_member, n_time, rec, out=None):
    """The readout rate W_m^T on count planes (hses_perturbed_readout_counts):
    counts (M, P', words(b)) int64 with P' >= count_planes(n_time), W (a, b),
    the layer's factor record; returns y (M, a) fp32."""
    a, b = W.shape
    _dev(W, torch.float32, "W")
    _dev(counts, torch.int64, "counts")
    M = n * rows_per_member
    wb = fmt_width(FMT_BITS, b)
    if counts.dim() != 3 or counts.shape[0] != M or counts.shape[2] != wb or \
            counts.shape[1] < count_planes(n_time) or not counts.is_contiguous():
        raise ValueError(f"counts is (M, P' >= {count_planes(n_time)}, {wb}), contiguous")
    if out is None:
        out = torch.empty((M, a), dtype=torch.float32, device=W.device)
    _dev(out, torch.float32, "out")
    if out.numel() != M * a:
        raise ValueError("out has the wrong size")
    _lib.call("hses_perturbed_readout_counts", _p(counts), counts.shape[1] * wb, n_time, _p(W),
              a, b, rank, sigma, tid_lo, n, rows_per_member, *_rec_arg(rec), _p(out), a,
              _stream())
    return out


def count_planes(n_time):
    """Bit planes of a spike count over n_time steps (0..n_time)."""
    return int(n_time).bit_length()


def perturbed_linear_lif_counts_x(x, W, rank, sigma, tid_lo, n, rows_per_member, n_time, tau_m,
                                  v_th, rec, img, counts=None, time_inner=False):
    """The fp32-accurate fused forward + LIF on factors drawn ahead (`rec`,
    split `img`) leaving each output row's spike count as bit planes: returns
    counts (M, P, words(a)) int64, P = count_planes(n_time), bit c of plane p
    being bit p of neuron c's count (hses_perturbed_linear_lif_counts_pre_x).
    x as in perturbed_linear_lif."""
    a, b = W.shape
    _dev(W, torch.float32, "W")
    _dev(x, _FMT_DTYPE[FMT_BITS], "x")
    units = fmt_width(FMT_BITS, b)
    M = n * rows_per_member
    if x.shape[-1] != units or x.numel() != n_time * M * units:
        raise ValueError(f"x has shape {tuple(x.shape)}, expected ({n_time}, {M}, {units})")
    wa = fmt_width(FMT_BITS, a)
    npl = count_planes(n_time)
    if counts is None:
        counts = torch.empty((M, npl, wa), dtype=torch.int64, device=W.device)
    _dev(counts, torch.int64, "counts")
    if counts.numel() != M * npl * wa:
        raise ValueError("counts has the wrong size")
    wbytes = int(_lib.load().hses_perturbed_linear_workspace(a, b, rank, n, rows_per_member,
                                                              n_time, MATH_F32X))
    work = _workspace(wbytes, W.device)
    if time_inner:
        xs, xp = n_time * units, units
    else:
        xs, xp = units, M * units
    _lib.call("hses_perturbed_linear_lif_counts_pre_x", _p(x), FMT_BITS, xs, xp, n_time, _p(W),
              a, b, rank, sigma, tid_lo, n, rows_per_member, tau_m, v_th, _p(counts), npl * wa,
              _p(work), wbytes, *_rec_arg(rec), *_img_arg(img), _stream())
    return counts


def es_update(fit, tid_lo, key, rank, sigma, epoch, noise_reuse, a, b, scale, out=None,
              accumulate=False, work=None):
    """scale * sum_m fit[m] A_m B_m^T (factors regenerated in-kernel); adds into
    `out` when accumulate is set."""
    _dev(fit, torch.float32, "fit")
    n = fit.numel()
    lib = _lib.load()
    wbytes = int(lib.hses_es_update_workspace(a, b, rank, n))
    if work is None or work.numel() < wbytes:
        work = _workspace(wbytes, fit.device)
    if out is None:
        out = torch.zeros((a, b), dtype=torch.float32, device=fit.device)
    _lib.call("hses_es_update", _p(fit), n, tid_lo, key & (2**64 - 1), rank, sigma, epoch,
              noise_reuse, a, b, scale, int(bool(accumulate)), _p(out), _p(work), wbytes,
              _stream())
    return out


def es_update_rec(fit, tid_lo, rec, rank, sigma, a, b, scale, out=None, accumulate=False,
                  work=None):
    """es_update from the factor record a forward over the same members kept
    (the same result as es_update, without drawing the normals again)."""
    _dev(fit, torch.float32, "fit")
    n = fit.numel()
    lib = _lib.load()
    wbytes = int(lib.hses_es_update_workspace(a, b, rank, n))
    if work is None or work.numel() < wbytes:
        work = _workspace(wbytes, fit.device)
    if out is None:
        out = torch.zeros((a, b), dtype=torch.float32, device=fit.device)
    _lib.call("hses_es_update_rec", _p(fit), n, tid_lo, *_rec_arg(rec), rank, sigma, a, b, scale,
              int(bool(accumulate)), _p(out), _p(work), wbytes, _stream())
    return out


def member_loglik(logits, labels, n, rows_per_member):
    _dev(logits, torch.float32, "logits")
    _dev(labels, torch.int32, "labels")
    fit = torch.empty(n, dtype=torch.float32, device=logits.device)
    _lib.call("hses_member_loglik", _p(logits), logits.shape[-1], _p(labels), n, rows_per_member,
              _p(fit), _stream())
    return fit


def member_fitness(logits, labels, n, rows_per_member, reward=REWARD_LOGLIK, out=None,
                   correct=None):
    """Per-member mean reward (Loglik or Binary); `correct` (int64, 1 element)
    is incremented by the number of rows whose argmax is the label."""
    _dev(logits, torch.float32, "logits")
    _dev(labels, torch.int32, "labels")
    if correct is not None:
        _dev(correct, torch.int64, "correct")
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=logits.device)
    _lib.call("hses_member_fitness", _p(logits), logits.shape[-1], _p(labels), n, rows_per_member,
              reward, _p(out), _p(correct), _stream())
    return out


def fitness_moments(raw, moments, accumulate=False):
    """moments (float64, 2) = / += {sum raw, sum raw^2}."""
    _dev(raw, torch.float32, "raw")
    _dev(moments, torch.float64, "moments")
    _lib.call("hses_fitness_moments", _p(raw), raw.numel(), _p(moments), int(bool(accumulate)),
              _stream())
    return moments


def combine_affine(grad_acc, moments, batch, ones_acc=None, out=None):
    """(grad_acc - ones_acc*mean) * (-1/(std*sqrt(batch))) with mean/std from moments."""
    _dev(grad_acc, torch.float32, "grad_acc")
    _dev(moments, torch.float64, "moments")
    if ones_acc is not None:
        _dev(ones_acc, torch.float32, "ones_acc")
        assert ones_acc.numel() == grad_acc.numel()
    if out is None:
        out = torch.empty_like(grad_acc)
    assert out.numel() == grad_acc.numel()
    _lib.call("hses_combine_affine", _p(grad_acc), _p(ones_acc), _p(moments), batch,
              grad_acc.numel(), _p(out), _stream())
    return out


def convert_fitnesses(raw, group_size=0):
    _dev(raw, torch.float32, "raw")
    out = torch.empty_like(raw)
    stats = torch.empty(2, dtype=torch.float32, device=raw.device)
    _lib.call("hses_convert_fitnesses", _p(raw), raw.numel(), group_size, _p(out), _p(stats),
              _stream())
    return out, stats


def solver_step(kind, lr, param, grad, m=None, v=None, step_t=1, beta1=0.9, beta2=0.999,
                eps=1e-8, wd=0.0, gscale=None):
    """In-place Solver::update of one parameter tensor; with gscale (a device
    float32 scalar, e.g. from clip_global_norm) on grad * gscale."""
    _dev(param, torch.float32, "param")
    _dev(grad, torch.float32, "grad")
    if gscale is None:
        _lib.call("hses_solver_step", kind, lr, beta1, beta2, eps, wd, step_t, _p(param),
                  _p(grad), _p(m), _p(v), param.numel(), _stream())
    else:
        _dev(gscale, torch.float32, "gscale")
        _lib.call("hses_solver_step_scaled", kind, lr, beta1, beta2, eps, wd, step_t, _p(param),
                  _p(grad), _p(m), _p(v), param.numel(), _p(gscale), _stream())
    return param


def clip_global_norm(grads, max_norm, out=None):
    """clip_grads_global_norm's factor over a list of gradient tensors: a
    device float32 scalar, max_norm / ||g|| or 1."""
    if not grads:
        raise ValueError("need at least one gradient tensor")
    for g in grads:
        _dev(g, torch.float32, "grad")
    dev = grads[0].device
    work = torch.empty(64 * len(grads), dtype=torch.float64, device=dev)
    if out is None:
        out = torch.empty(1, dtype=torch.float32, device=dev)
    ptrs = (ctypes.c_void_p * len(grads))(*[g.data_ptr() for g in grads])
    lens = (ctypes.c_int64 * len(grads))(*[g.numel() for g in grads])
    _lib.call("hses_clip_global_norm", ptrs, lens, len(grads), max_norm, _p(work), _p(out),
              _stream())
    return out


def noisy_standard(param, key, sigma, epoch, noise_reuse, tids):
    """get_noisy_standard for n members: (n, a, b) = param + sign*sigma*noise.
    tids is an int sequence/tensor or (tid_lo, n)."""
    _dev(param, torch.float32, "param")
    a, b = param.shape
    if isinstance(tids, tuple):
        tid_lo, n = tids
        d_tids = None
    else:
        d_tids = torch.as_tensor(tids, dtype=torch.int32, device=param.device).contiguous()
        tid_lo, n = 0, d_tids.numel()
    out = torch.empty((n, a, b), dtype=torch.float32, device=param.device)
    _lib.call("hses_noisy_standard", _p(param), a, b, key & (2**64 - 1), sigma, epoch,
              noise_reuse, tid_lo, _p(d_tids), n, _p(out), _stream())
    return out


def full_update(fit, tid_lo, key, sigma, epoch, noise_reuse, a, b, scale, out=None,
                accumulate=False):
    """_simple_full_update of a dense (a, b) parameter: scale * sum_m fit[m] noise_m."""
    _dev(fit, torch.float32, "fit")
    n = fit.numel()
    wbytes = int(_lib.load().hses_full_update_workspace(a, b, n))
    work = _workspace(wbytes, fit.device)
    if out is None:
        out = torch.empty((a, b), dtype=torch.float32, device=fit.device)
    _lib.call("hses_full_update", _p(fit), n, tid_lo, key & (2**64 - 1), sigma, epoch, noise_reuse,
              a, b, scale, int(bool(accumulate)), _p(out), _p(work), wbytes, _stream())
    return out
