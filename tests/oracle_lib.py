"""ctypes binding of the CPU oracle (oracle/liboracle.so), test infrastructure only."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB = os.path.join(ORACLE_DIR, "_build", "liboracle.so")

_lib = None
f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
c_i32, c_i64, c_u32, c_u64, c_f32 = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32,
                                     ctypes.c_uint64, ctypes.c_float)


class SnnCfg(ctypes.Structure):
    _fields_ = [("n_layers", c_i32), ("dims", ctypes.POINTER(c_i32)), ("T", c_i32),
                ("rows", c_i32), ("tau_m", c_f32), ("v_th", c_f32), ("sigma", c_f32),
                ("rank", c_i32), ("noise_reuse", c_i32), ("epoch", c_i32),
                ("poisson_seed", c_u32 * 4)]


TM_VECTORS = ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")
TM_LINEAR = ("receptance", "key", "value", "output")
TM_TMM = ("w1", "w2", "v1", "v2", "a1", "a2", "g1", "g2")
TM_FIELDS = (TM_VECTORS + TM_LINEAR + ("w0", "v0", "a0") + ("w1", "v1", "a1", "g1")
             + ("w2", "v2", "a2", "g2") + ("k_k", "k_a", "r_k", "ln_w", "ln_b"))


class TmWeights(ctypes.Structure):
    _fields_ = ([(name, ctypes.c_void_p) for name in TM_FIELDS]
                + [("d_w", c_i32), ("d_v", c_i32), ("d_a", c_i32), ("d_g", c_i32)])


class RwkvBlock(ctypes.Structure):
    _fields_ = [("tm", TmWeights)] + [(n, ctypes.c_void_p) for n in
                                      ("ffn_x_k", "ffn_key", "ffn_value", "ln1_w", "ln1_b",
                                       "ln2_w", "ln2_b")]


class RwkvLm(ctypes.Structure):
    _fields_ = ([(n, c_i32) for n in ("n_layer", "C", "H", "F", "V")]
                + [(n, ctypes.c_void_p) for n in ("emb", "ln0_w", "ln0_b", "ln_out_w", "ln_out_b",
                                                  "head")]
                + [("blocks", ctypes.POINTER(RwkvBlock))])


SA_MAX_HEADS = 8


class SaCfg(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("T", "ntok", "tin", "d_model", "heads", "blocks", "classes",
                                      "n_iter")] + [("tau_m", c_f32), ("g_inh", c_f32)]


class SaBlock(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_void_p * SA_MAX_HEADS) for n in ("q", "k", "v")]
                + [(n, ctypes.c_void_p) for n in ("o", "ff1", "ff2")] + [("ff_th", c_f32)])


class SaParams(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_void_p) for n in ("in_q", "in_k", "in_v", "pos")]
                + [("blocks", ctypes.POINTER(SaBlock)), ("out", ctypes.c_void_p)]
                + [(n, c_f32) for n in ("out_gain", "beta", "q_th", "k_th", "v_th", "attn_th")])


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB):
        build()
    L = ctypes.CDLL(LIB)
    sig = {
        "or_noise_seed": (c_u64, [c_u64, c_i32, c_i32]),
        "or_xorshift64_step": (c_u64, [c_u64]),
        "or_unit_from_u64": (c_f32, [c_u64]),
        "or_bm_radius": (c_f32, [c_u32]),
        "or_bm_cos": (c_f32, [c_u32]),
        "or_bm_eval": (None, [c_u32, c_u32, f32p, f32p, f32p]),
        "or_base_sigma": (c_f32, [c_f32, c_i32]),
        "or_standard_normals": (None, [c_u64, f32p, c_i64]),
        "or_get_lora_update_params": (None, [c_f32, c_u64, c_i32, c_i32, c_i32, c_i32, c_i32,
                                             c_i32, f32p, f32p]),
        "or_batched_lora_noise": (None, [c_f32, c_u64, c_i32, i32p, c_i32, c_i32, c_i32, c_i32,
                                         c_i32, f32p, f32p]),
        "or_get_nonlora_update_params": (None, [c_f32, c_u64, c_i32, c_i32, c_i32, c_i32, c_i32,
                                                f32p]),
        "or_matmul_abt": (None, [f32p, c_i32, c_i32, f32p, c_i32, f32p]),
        "or_matmul_abt_f64": (None, [f32p, c_i32, c_i32, f32p, c_i32, f32p]),
        "or_do_mm": (None, [f32p, c_i32, f32p, c_i32, c_i32, ctypes.c_void_p, ctypes.c_void_p,
                            c_i32, f32p]),
        "or_do_Tmm": (None, [f32p, c_i32, f32p, c_i32, c_i32, ctypes.c_void_p, ctypes.c_void_p,
                             c_i32, f32p]),
        "or_lif_scan": (None, [f32p, ctypes.c_void_p, c_i32, c_i64, c_i32, c_f32, c_f32, f32p,
                               ctypes.c_void_p]),
        "or_poisson_encode": (None, [f32p, c_i64, c_i32, c_i32, c_u32, c_u32, c_u32, c_u32,
                                     f32p]),
        "or_mean_rate": (None, [f32p, c_i32, c_i64, c_i32, f32p]),
        "or_loglik": (None, [f32p, c_i64, c_i32, i32p, f32p]),
        "or_convert_fitnesses": (None, [f32p, c_i32, c_i32, f32p, ctypes.POINTER(c_f32),
                                        ctypes.POINTER(c_f32)]),
        "or_simple_lora_update": (None, [c_f32, c_u64, c_i32, c_i32, f32p, i32p, i32p, c_i32,
                                         c_i32, c_i32, f32p]),
        "or_do_update_lora": (None, [c_f32, c_u64, c_i32, c_i32, f32p, i32p, i32p, c_i32, c_i32,
                                     c_i32, f32p]),
        "or_do_update_full": (None, [c_f32, c_u64, c_i32, c_i32, f32p, i32p, i32p, c_i32, c_i32,
                                     c_i32, f32p]),
        "or_lora_einsum_f64": (None, [c_f32, c_u64, c_i32, c_i32, c_i32, f32p, i32p, c_i32,
                                      c_i32, c_i32, f64p]),
        "or_accumulated_lora_grad": (None, [c_f32, c_u64, c_i32, c_i32, c_i32, f32p, i32p, c_i32,
                                            c_i32, c_i32, c_i32, f32p]),
        "or_lora_einsum_raw": (None, [f32p, f32p, f32p, c_i32, c_i32, c_i32, c_i32, f32p]),
        "or_lora_einsum_ones": (None, [f32p, f32p, c_i32, c_i32, c_i32, c_i32, f32p]),
        "or_combine_affine": (None, [f32p, f32p, c_i64, c_f32, c_f32, c_i32, f32p]),
        "or_layer_norm": (None, [f32p, c_i64, c_i32, f32p, f32p, c_f32, f32p]),
        "or_group_norm": (None, [f32p, c_i64, c_i32, c_i32, c_i32, f32p, f32p, c_f32, f32p]),
        "or_rwkv7_inner_loop": (None, [f32p, f32p, f32p, f32p, f32p, f32p, f32p, c_i32, c_i32,
                                       c_i32, c_i32, ctypes.c_void_p, f32p, f32p]),
        "or_channel_mixing": (None, [f32p, c_i32, c_i32, f32p, f32p, f32p, c_i32, f32p, c_i32,
                                     ctypes.c_void_p, f32p, f32p]),
        "or_time_mixing": (None, [ctypes.POINTER(TmWeights), f32p, c_i32, c_i32, c_i32, f32p,
                                  f32p, c_i32, ctypes.c_void_p, c_i32, f32p, f32p]),
        "or_rwkv_lm_forward": (None, [ctypes.POINTER(RwkvLm), i32p, c_i32, f32p, f32p]),
        "or_solver_step": (None, [c_i32, c_f32, c_f32, c_f32, c_f32, c_f32, c_i32, f32p, f32p,
                                  f32p, f32p, c_i64, f32p]),
        "or_snn_forward_members": (None, [ctypes.POINTER(SnnCfg), ctypes.c_void_p,
                                          ctypes.c_void_p, f32p, i32p, c_i32, c_i32, c_i32,
                                          f32p]),
        "or_lora_grad_f64": (None, [c_f32, c_u64, c_i32, c_i32, c_i32, f32p, c_i32, c_i32, c_i32,
                                    c_i32, f32p]),
        "or_snn_forward_member": (None, [ctypes.POINTER(SnnCfg), ctypes.c_void_p,
                                         ctypes.c_void_p, f32p, i32p, c_i32, f32p]),
        "or_sa_softplus": (c_f32, [c_f32]),
        "or_sa_encode": (None, [f32p, f32p, f32p, c_i32, c_i32, c_i32, c_f32, c_f32, c_f32, c_f32,
                                f32p, f32p]),
        "or_sa_row_softmax_lif": (None, [f32p, c_i32, c_f32, c_f32, c_f32, c_i32, f32p]),
        "or_sa_attention_head": (None, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, c_i32,
                                        c_i32, c_i32, c_f32, c_f32, c_f32, c_f32, c_i32,
                                        ctypes.c_void_p]),
        "or_sa_ffn_spike": (None, [f32p, c_i32, c_i32, c_f32, f32p]),
        "or_sa_forward_member": (None, [ctypes.POINTER(SaCfg), ctypes.POINTER(SaParams), f32p,
                                        f32p]),
        "or_clip_global_norm_scale": (c_f32, [ctypes.c_void_p, ctypes.c_void_p, c_i32, c_f32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


# ---- numpy conveniences ------------------------------------------------------

def lora_factors(base_sigma, key, rank, epoch, tids, a, b, noise_reuse=0):
    L = load()
    tids = np.ascontiguousarray(tids, dtype=np.int32)
    n = tids.size
    A = np.zeros((n, a, rank), np.float32)
    B = np.zeros((n, b, rank), np.float32)
    L.or_batched_lora_noise(base_sigma, key & (2**64 - 1), rank, tids, n, epoch, noise_reuse, a,
                            b, A, B)
    return A, B


def do_mm(x, W, A=None, B=None):
    L = load()
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    rows, b = x.shape
    a = W.shape[0]
    y = np.zeros((rows, a), np.float32)
    r = 0 if A is None else A.shape[1]
    Ap = None if A is None else np.ascontiguousarray(A, np.float32)
    Bp = None if B is None else np.ascontiguousarray(B, np.float32)
    L.or_do_mm(x, rows, W, a, b, None if Ap is None else Ap.ctypes.data,
               None if Bp is None else Bp.ctypes.data, r, y)
    return y


def lif(cur, tau_m, v_th, v0=None):
    L = load()
    cur = np.ascontiguousarray(cur, np.float32)
    T, M, h = cur.shape
    spk = np.zeros_like(cur)
    v = np.zeros((M, h), np.float32)
    v0p = None if v0 is None else np.ascontiguousarray(v0, np.float32).ctypes.data
    L.or_lif_scan(cur, v0p, T, M, h, tau_m, v_th, spk, v.ctypes.data)
    return spk, v


def poisson(p, T, seeds=(0, 0, 0, 0)):
    L = load()
    p = np.ascontiguousarray(p, np.float32)
    M, d = p.shape
    out = np.zeros((T, M, d), np.float32)
    L.or_poisson_encode(p, M, d, T, *[int(s) & 0xFFFFFFFF for s in seeds], out)
    return out


def loglik(logits, labels):
    L = load()
    logits = np.ascontiguousarray(logits, np.float32)
    rows, c = logits.shape
    out = np.zeros(rows, np.float32)
    L.or_loglik(logits, rows, c, np.ascontiguousarray(labels, np.int32), out)
    return out


def convert_fitnesses(raw, group_size=0):
    L = load()
    raw = np.ascontiguousarray(raw, np.float32)
    out = np.zeros_like(raw)
    m, s = c_f32(), c_f32()
    L.or_convert_fitnesses(raw, raw.size, group_size, out, ctypes.byref(m), ctypes.byref(s))
    return out, m.value, s.value


def lora_grad_f64(sigma, key, rank, epoch, fit, a, b, noise_reuse=0, nthreads=8):
    """-sqrt(N)/N * sum_i f_i A_i B_i^T, double accumulation, tids 0..N-1."""
    L = load()
    fit = np.ascontiguousarray(fit, np.float32)
    g = np.zeros((a, b), np.float32)
    L.or_lora_grad_f64(sigma, key & (2**64 - 1), rank, noise_reuse, epoch, fit, fit.size, a, b,
                       nthreads, g)
    return g


def _f(a):
    return np.ascontiguousarray(a, np.float32)


def layer_norm(x, w, b, eps=1e-5):
    x = _f(x)
    y = np.empty_like(x)
    load().or_layer_norm(x, x.size // x.shape[-1], x.shape[-1], _f(w), _f(b), eps, y)
    return y


def group_norm(x, groups, w, b, eps=1e-5):
    """x (n, C) or (n, C, L)."""
    x = _f(x)
    L = x.shape[2] if x.ndim == 3 else 1
    y = np.empty_like(x)
    load().or_group_norm(x, x.shape[0], x.shape[1], L, groups, _f(w), _f(b), eps, y)
    return y


def rwkv7_inner_loop(r, w, k, v, a, b, s0, length, new_starts=None):
    """r..b (T, H, S), s0 (H, S, S) -> (out (T, H, S), out_s (H, S, S))."""
    T, H, S = r.shape
    out = np.zeros((T, H, S), np.float32)
    out_s = np.zeros((H, S, S), np.float32)
    ns = None if new_starts is None else np.ascontiguousarray(new_starts, np.uint8)
    load().or_rwkv7_inner_loop(_f(r), _f(w), _f(k), _f(v), _f(a), _f(b), _f(s0), T, H, S, length,
                               None if ns is None else ns.ctypes.data, out, out_s)
    return out, out_s


def channel_mixing(x, state, x_k, Wk, Wv, length, new_starts=None):
    """x (T, C), state (C,), Wk (F, C), Wv (C, F) -> (out (T, C), last (C,))."""
    T, C = x.shape
    F = Wk.shape[0]
    out = np.zeros((T, C), np.float32)
    last = np.zeros(C, np.float32)
    ns = None if new_starts is None else np.ascontiguousarray(new_starts, np.uint8)
    load().or_channel_mixing(_f(x), T, C, _f(state), _f(x_k), _f(Wk), F, _f(Wv), length,
                             None if ns is None else ns.ctypes.data, out, last)
    return out, last


def _tm_struct(keep):
    return TmWeights(*[keep[name].ctypes.data for name in TM_FIELDS],
                     *[keep[name].shape[1] for name in ("w1", "v1", "a1", "g1")])


def time_mixing(P, x, state, v_first, H, length, layer_id, new_starts=None):
    """TimeMixing::forward (llm.rs:348-480) of one sequence.  P maps the
    TM_FIELDS names to arrays (Linear weights (out, in), Tmm weights (in, out)).
    x (T, C), state (1 + S, C), v_first (T, C) -> (out (T, C), state (1 + S, C),
    v_first (T, C))."""
    T, C = x.shape
    S = C // H
    keep = {name: _f(P[name]) for name in TM_FIELDS}
    tw = _tm_struct(keep)
    vf = np.array(v_first, np.float32, copy=True).reshape(T, C)
    out = np.zeros((T, C), np.float32)
    st = np.zeros((1 + S, C), np.float32)
    ns = None if new_starts is None else np.ascontiguousarray(new_starts, np.uint8)
    load().or_time_mixing(ctypes.byref(tw), _f(x), T, C, H, _f(state), vf, length,
                          None if ns is None else ns.ctypes.data, layer_id, out, st)
    return out, st, vf


def rwkv_lm_forward(P, tokens, H, state=None):
    """The RWKV-7 LM (rwkv7.py:189-253) on one sequence.  P: emb (V, C), ln0_w,
    ln0_b, ln_out_w, ln_out_b, head (V, C) and `blocks`, a list of dicts with the
    TimeMixing names, ffn_x_k, ffn_key (F, C), ffn_value (C, F), ln1_w, ln1_b,
    ln2_w, ln2_b.  Returns (logits (T, V), state (n_layer, 2 + S, C))."""
    tokens = np.ascontiguousarray(tokens, np.int32)
    V, C = P["emb"].shape
    L = len(P["blocks"])
    S = C // H
    F = P["blocks"][0]["ffn_key"].shape[0]
    keep = {n: _f(P[n]) for n in ("emb", "ln0_w", "ln0_b", "ln_out_w", "ln_out_b", "head")}
    bkeep = [{n: _f(v) for n, v in b.items()} for b in P["blocks"]]
    blocks = (RwkvBlock * L)()
    for l, b in enumerate(bkeep):
        blocks[l].tm = _tm_struct(b)
        for n in ("ffn_x_k", "ffn_key", "ffn_value", "ln1_w", "ln1_b", "ln2_w", "ln2_b"):
            setattr(blocks[l], n, b[n].ctypes.data)
    lm = RwkvLm(L, C, H, F, V, *[keep[n].ctypes.data for n in ("emb", "ln0_w", "ln0_b",
                                                               "ln_out_w", "ln_out_b", "head")],
                blocks)
    st = (np.zeros((L, 2 + S, C), np.float32) if state is None
          else np.array(state, np.float32, copy=True))
    logits = np.zeros((tokens.size, V), np.float32)
    load().or_rwkv_lm_forward(ctypes.byref(lm), tokens, tokens.size, st, logits)
    return logits, st


def clip_scale(grads, max_norm):
    """or_clip_global_norm_scale over a list of float32 arrays."""
    gs = [np.ascontiguousarray(g, np.float32) for g in grads]
    ptrs = (ctypes.c_void_p * max(1, len(gs)))(*[g.ctypes.data for g in gs])
    lens = np.array([g.size for g in gs] or [0], np.int64)
    return float(load().or_clip_global_norm_scale(ptrs, lens.ctypes.data, len(gs), max_norm))


# ---- spiking self-attention (C4) ---------------------------------------------

def sa_cfg(c):
    """SaCfg from a hyperscalees_amd.snn_attention.SaConfig-like object."""
    out = SaCfg()
    for f in ("T", "ntok", "tin", "d_model", "heads", "blocks", "classes", "n_iter"):
        setattr(out, f, int(getattr(c, f)))
    out.tau_m, out.g_inh = float(c.tau_m), float(c.g_inh)
    return out


def sa_forward_member(c, P, x):
    """or_sa_forward_member on a member's parameter dict P (leaf name -> f32
    array, already perturbed) and its input spikes x (T, ntok, tin)."""
    keep = {k: np.ascontiguousarray(v, np.float32) for k, v in P.items()}
    blocks = (SaBlock * c.blocks)()
    for b in range(c.blocks):
        for kind in "qkv":
            arr = getattr(blocks[b], kind)
            for h in range(c.heads):
                arr[h] = keep[f"b{b}_{kind}{h}"].ctypes.data
        blocks[b].o = keep[f"b{b}_o"].ctypes.data
        blocks[b].ff1 = keep[f"b{b}_ff1"].ctypes.data
        blocks[b].ff2 = keep[f"b{b}_ff2"].ctypes.data
        blocks[b].ff_th = float(keep[f"b{b}_ff_th"].ravel()[0])
    sp = SaParams()
    for n, key in (("in_q", "in_q"), ("in_k", "in_k"), ("in_v", "in_v"), ("pos", "pos_emb"),
                   ("out", "out")):
        setattr(sp, n, keep[key].ctypes.data)
    sp.blocks = blocks
    for n in ("out_gain", "beta", "q_th", "k_th", "v_th", "attn_th"):
        setattr(sp, n, float(keep[n].ravel()[0]))
    logits = np.zeros(c.classes, np.float32)
    cfg = sa_cfg(c)
    load().or_sa_forward_member(ctypes.byref(cfg), ctypes.byref(sp),
                                np.ascontiguousarray(x, np.float32), logits)
    return logits


def sa_member_params(P, keys, leaves, sigma, rank, m, epoch=0, noise_reuse=0):
    """Member m's parameters: W + A_m B_m^T (float64 product, rounded to f32) for
    MM leaves, param + sign*sigma*noise for Parameter leaves."""
    L = load()
    bs = L.or_base_sigma(sigma, rank)
    out = {}
    for name, (a, b), cls in leaves:
        if cls == 1:
            A, B = lora_factors(bs, keys[name], rank, epoch, [m], a, b, noise_reuse=noise_reuse)
            out[name] = (P[name].astype(np.float64)
                         + A[0].astype(np.float64) @ B[0].T.astype(np.float64)).astype(np.float32)
        else:
            nz = np.zeros(a * b, np.float32)
            L.or_get_nonlora_update_params(sigma, keys[name], epoch, m, a, b, noise_reuse, nz)
            out[name] = P[name] + nz.reshape(a, b)
    return out
