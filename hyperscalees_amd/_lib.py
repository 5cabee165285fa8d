"""ctypes binding of libhses.so (the C ABI declared in include/hses.h).

The library is loaded from this package directory only.  There is no
fallback: if it is missing or fails to load, every call raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhses.so")

HSES_OK, HSES_ERR_INVALID_ARG, HSES_ERR_UNSUPPORTED, HSES_ERR_HIP, HSES_ERR_INTERNAL = range(5)
FMT_F32, FMT_BF16, FMT_U8, FMT_BITS = range(4)
MATH_F32, MATH_BF16, MATH_F32X = range(3)
SGD, ADAM, ADAMW = range(3)
REWARD_LOGLIK, REWARD_BINARY = range(2)
ACT_NONE, ACT_TANH, ACT_SIGMOID, ACT_RELU_SQ = range(4)

c_i32, c_i64, c_u32, c_u64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64
c_f32, c_vp, c_size = ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/hses.h
PROTOTYPES = {
    "hses_init": (ctypes.c_int, [ctypes.c_int]),
    "hses_last_error": (ctypes.c_int, [ctypes.c_char_p, c_size]),
    "hses_version": (ctypes.c_char_p, []),
    "hses_bm_stats": (ctypes.c_int, [ctypes.POINTER(c_u32)]),
    "hses_noise_seed": (c_u64, [c_u64, c_i32, c_i32]),
    "hses_bm_eval": (ctypes.c_int, [c_u32, c_u32, c_vp, c_vp, c_vp, c_vp]),
    "hses_lora_factors": (ctypes.c_int, [c_f32, c_u64, c_i32, c_i32, c_i32, c_i32, c_vp, c_i32,
                                         c_i32, c_i32, c_vp, c_vp, c_vp]),
    "hses_nonlora_noise": (ctypes.c_int, [c_f32, c_u64, c_i32, c_i32, c_i32, c_vp, c_i32, c_i32,
                                          c_i32, c_vp, c_vp]),
    "hses_poisson_encode": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i64, c_i32, c_i64, c_i32, c_u32, c_u32,
                                           c_u32, c_u32, c_vp, c_i32, c_i64, c_vp]),
    "hses_poisson_encode_planes": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i64, c_i32, c_i64, c_i32,
                                                  c_u32, c_u32, c_u32, c_u32, c_vp, c_i32, c_i64,
                                                  c_i64, c_vp]),
    "hses_poisson_pool_bytes": (c_size, [c_i64, c_i32]),
    "hses_poisson_pool_prepare": (ctypes.c_int, [c_vp, c_i64, c_i32, c_i64, c_vp, c_size, c_vp]),
    "hses_poisson_encode_pool": (ctypes.c_int, [c_vp, c_size, c_i64, c_i32, c_vp, c_i64, c_i32,
                                                c_u32, c_u32, c_u32, c_u32, c_vp, c_i64, c_i64,
                                                c_vp]),
    "hses_spike_rate": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i32, c_i64, c_i32, c_vp, c_vp]),
    "hses_lif_scan": (ctypes.c_int, [c_vp, c_vp, c_i32, c_i64, c_i32, c_i64, c_f32, c_f32, c_vp,
                                     c_i32, c_i64, c_vp, c_vp]),
    "hses_perturbed_linear": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32, c_i32,
                                             c_u64, c_i32, c_f32, c_i32, c_i32, c_i32, c_i32,
                                             c_i32, c_vp, c_i64, c_i64, c_i32, c_vp, c_size,
                                             c_vp]),
    "hses_perturbed_linear_lif": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32,
                                                 c_i32, c_u64, c_i32, c_f32, c_i32, c_i32, c_i32,
                                                 c_i32, c_i32, c_f32, c_f32, c_vp, c_i64, c_i64,
                                                 c_vp, c_i64, c_vp, c_size, c_vp]),
    "hses_perturbed_linear_workspace": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                                 c_i32]),
    "hses_factor_record_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "hses_perturbed_linear_rec": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32,
                                                 c_i32, c_u64, c_i32, c_f32, c_i32, c_i32, c_i32,
                                                 c_i32, c_i32, c_vp, c_i64, c_i64, c_i32, c_vp,
                                                 c_size, c_vp, c_size, c_vp]),
    "hses_perturbed_linear_lif_rec": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp,
                                                     c_i32, c_i32, c_u64, c_i32, c_f32, c_i32,
                                                     c_i32, c_i32, c_i32, c_i32, c_f32, c_f32,
                                                     c_vp, c_i64, c_i64, c_vp, c_i64, c_vp,
                                                     c_size, c_vp, c_size, c_vp]),
    "hses_pair_image_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "hses_pair_factors": (ctypes.c_int, [c_u64, c_i32, c_f32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                         c_i32, c_vp, c_size, c_vp, c_size, c_vp]),
    "hses_perturbed_linear_pre": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32,
                                                 c_i32, c_i32, c_f32, c_i32, c_i32, c_i32, c_vp,
                                                 c_i64, c_i64, c_vp, c_size, c_vp, c_size, c_vp,
                                                 c_size, c_vp]),
    "hses_perturbed_linear_lif_pre": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp,
                                                     c_i32, c_i32, c_i32, c_f32, c_i32, c_i32,
                                                     c_i32, c_f32, c_f32, c_vp, c_i64, c_i64,
                                                     c_vp, c_i64, c_vp, c_size, c_vp, c_size,
                                                     c_vp, c_size, c_vp]),
    "hses_pair_image_x_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "hses_member_weights_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32]),
    "hses_member_weights": (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_f32, c_i32, c_i32, c_vp,
                                           c_size, c_i32, c_vp, c_size, c_vp]),
    "hses_perturbed_linear_mw": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_i32, c_i32,
                                                c_i32, c_i32, c_i32, c_i32, c_vp, c_size, c_vp,
                                                c_i64, c_i64, c_vp]),
    "hses_perturbed_linear_lif_mw": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_i32,
                                                    c_i32, c_i32, c_i32, c_i32, c_f32, c_f32,
                                                    c_i32, c_vp, c_size, c_vp, c_i64, c_i64, c_vp,
                                                    c_i64, c_vp, c_i64, c_vp]),
    "hses_perturbed_readout_counts": (ctypes.c_int, [c_vp, c_i64, c_i32, c_vp, c_i32, c_i32,
                                                     c_i32, c_f32, c_i32, c_i32, c_i32, c_vp,
                                                     c_size, c_vp, c_i64, c_vp]),
    "hses_perturbed_linear_lif_counts_pre_x": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32,
                                                              c_vp, c_i32, c_i32, c_i32, c_f32,
                                                              c_i32, c_i32, c_i32, c_f32, c_f32,
                                                              c_vp, c_i64, c_vp, c_size, c_vp,
                                                              c_size, c_vp, c_size, c_vp]),
    "hses_pair_factors_x": (ctypes.c_int, [c_u64, c_i32, c_f32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                           c_i32, c_vp, c_size, c_vp, c_size, c_vp]),
    "hses_pair_image_x": (ctypes.c_int, [c_i32, c_i32, c_i32, c_f32, c_i32, c_i32, c_vp, c_size,
                                         c_vp, c_size, c_vp]),
    "hses_perturbed_linear_pre_x": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32,
                                                   c_i32, c_i32, c_f32, c_i32, c_i32, c_i32, c_vp,
                                                   c_i64, c_i64, c_vp, c_size, c_vp, c_size, c_vp,
                                                   c_size, c_vp]),
    "hses_perturbed_linear_lif_pre_x": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp,
                                                       c_i32, c_i32, c_i32, c_f32, c_i32, c_i32,
                                                       c_i32, c_f32, c_f32, c_vp, c_i64, c_i64,
                                                       c_vp, c_i64, c_vp, c_size, c_vp, c_size,
                                                       c_vp, c_size, c_vp]),
    "hses_perturbed_linear_t": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32,
                                               c_i32, c_u64, c_i32, c_f32, c_i32, c_i32, c_i32,
                                               c_i32, c_i32, c_vp, c_i64, c_i64, c_i32, c_vp,
                                               c_size, c_vp]),
    "hses_perturbed_linear_t_workspace": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                                   c_i32]),
    "hses_es_update_workspace": (c_size, [c_i32, c_i32, c_i32, c_i32]),
    "hses_es_update": (ctypes.c_int, [c_vp, c_i32, c_i32, c_u64, c_i32, c_f32, c_i32, c_i32,
                                      c_i32, c_i32, c_f32, c_i32, c_vp, c_vp, c_size, c_vp]),
    "hses_es_update_rec": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_size, c_i32, c_f32, c_i32,
                                          c_i32, c_f32, c_i32, c_vp, c_vp, c_size, c_vp]),
    "hses_es_update_noalloc": (ctypes.c_int, [c_vp, c_i32, c_i32, c_u64, c_i32, c_f32, c_i32,
                                              c_i32, c_i32, c_i32, c_f32, c_i32, c_vp, c_vp]),
    "hses_noisy_standard": (ctypes.c_int, [c_vp, c_i32, c_i32, c_u64, c_f32, c_i32, c_i32, c_i32,
                                           c_vp, c_i32, c_vp, c_vp]),
    "hses_full_update_workspace": (c_size, [c_i32, c_i32, c_i32]),
    "hses_full_update": (ctypes.c_int, [c_vp, c_i32, c_i32, c_u64, c_f32, c_i32, c_i32, c_i32,
                                        c_i32, c_f32, c_i32, c_vp, c_vp, c_size, c_vp]),
    "hses_solver_step_scaled": (ctypes.c_int, [c_i32, c_f32, c_f32, c_f32, c_f32, c_f32, c_i32,
                                               c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp]),
    "hses_clip_global_norm": (ctypes.c_int, [c_vp, c_vp, c_i32, c_f32, c_vp, c_vp, c_vp]),
    "hses_softplus": (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp]),
    "hses_sa_encode": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp,
                                      c_vp, c_f32, c_vp, c_i32, c_vp, c_vp]),
    "hses_sa_attention": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i32, c_i32, c_i32,
                                         c_vp, c_vp, c_f32, c_f32, c_i32, c_vp, c_vp]),
    "hses_sa_ffn_spike": (ctypes.c_int, [c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "hses_add_inplace": (ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    "hses_sa_pool": (ctypes.c_int, [c_vp, c_i64, c_i32, c_i32, c_vp, c_vp]),
    "hses_scale_rows": (ctypes.c_int, [c_vp, c_i64, c_i32, c_vp, c_vp]),
    "hses_member_loglik": (ctypes.c_int, [c_vp, c_i32, c_vp, c_i32, c_i32, c_vp, c_vp]),
    "hses_member_fitness": (ctypes.c_int, [c_vp, c_i32, c_vp, c_i32, c_i32, c_i32, c_vp, c_vp,
                                           c_vp]),
    "hses_fitness_moments": (ctypes.c_int, [c_vp, c_i32, c_vp, c_i32, c_vp]),
    "hses_combine_affine": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i32, c_i64, c_vp, c_vp]),
    "hses_convert_fitnesses": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "hses_layer_norm": (ctypes.c_int, [c_vp, c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_vp]),
    "hses_group_norm": (ctypes.c_int, [c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_f32, c_vp,
                                       c_vp]),
    "hses_token_shift_mix": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i32, c_i64, c_i32, c_i32,
                                            c_vp, c_i32, c_vp]),
    "hses_relu_sq": (ctypes.c_int, [c_vp, c_i64, c_vp]),
    "hses_rwkv7_wkv": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32,
                                      c_i32, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "hses_perturbed_linear_act": (ctypes.c_int, [c_vp, c_i32, c_i64, c_i64, c_i32, c_vp, c_i32,
                                                 c_i32, c_u64, c_i32, c_f32, c_i32, c_i32, c_i32,
                                                 c_i32, c_i32, c_vp, c_i64, c_i64, c_i32, c_i32,
                                                 c_i32, c_i32, c_vp, c_size, c_vp]),
    "hses_tm_wkv_post": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64,
                                        c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_f32, c_vp,
                                        c_vp, c_i32, c_vp, c_vp]),
    "hses_tm_gates_kk": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                        c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "hses_tm_fused": (ctypes.c_int, [c_vp] * 14 + [c_i64, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp,
                                                   c_vp, c_f32, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "hses_rwkv_act": (ctypes.c_int, [c_vp, c_i64, c_i32, c_vp]),
    "hses_tm_gates": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32,
                                     c_vp]),
    "hses_tm_kk": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "hses_tm_post": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp]),
    "hses_embed_layer_norm": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i32, c_i32, c_vp, c_vp, c_f32,
                                             c_vp, c_vp]),
    "hses_add_layer_norm": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i32, c_vp, c_vp, c_f32, c_vp,
                                           c_vp]),
    "hses_add_ln_shift": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_f32, c_vp,
                                         c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32, c_vp]),
    "hses_read_idx_images": (ctypes.c_int, [c_vp, c_size, c_vp, c_i64, c_vp, c_vp]),
    "hses_read_idx_labels": (ctypes.c_int, [c_vp, c_size, c_vp, c_i64, c_vp]),
    "hses_shuffled_indices": (ctypes.c_int, [c_i64, c_i64, c_u64, c_vp]),
    "hses_solver_step": (ctypes.c_int, [c_i32, c_f32, c_f32, c_f32, c_f32, c_f32, c_i32, c_vp,
                                        c_vp, c_vp, c_vp, c_i64, c_vp]),
}

_lib = None


class HsesError(RuntimeError):
    """A libhses entry point returned a non-zero status."""

    def __init__(self, code, msg):
        super().__init__(f"[hses status {code}] {msg}")
        self.code = code


def load():
    """Load libhses.so and declare every prototype.  Raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m hyperscalees_amd.build` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error():
    buf = ctypes.create_string_buffer(1024)
    load().hses_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc):
    if rc != HSES_OK:
        raise HsesError(rc, last_error())
    return rc


def call(name, *args):
    """Call entry point `name` and raise HsesError on a non-zero status."""
    return check(getattr(load(), name)(*args))
