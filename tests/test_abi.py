"""CPU checks of the C ABI: libhses.so loads, exports every entry point that
include/hses.h declares, and rejects bad arguments before touching a GPU."""
import ctypes
import os
import re

import pytest

from hyperscalees_amd import _lib
from tests import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "hses.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(hses_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = declared_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), f"libhses.so does not export {s}"
    assert set(syms) == set(_lib.PROTOTYPES), "ctypes prototypes out of sync with hses.h"


def test_version_string():
    assert b"gfx950" in _lib.load().hses_version()


def test_noise_seed_matches_oracle():
    lib = _lib.load()
    for k, e, t in [(0, 0, 0), (42, 1, 2), (2**64 - 1, -3, 17), (0x9E3779B97F4A7C15 * 3 % 2**64, 0, 4095)]:
        assert lib.hses_noise_seed(k, e, t) == O.load().or_noise_seed(k, e, t)


def _expect_invalid(name, *args):
    rc = getattr(_lib.load(), name)(*args)
    assert rc == _lib.HSES_ERR_INVALID_ARG, (name, rc)
    assert _lib.last_error(), "no error message"


NULL = None


def test_add_ln_shift_validation_without_a_gpu():
    lib = _lib.load()
    v = ctypes.c_void_p(256)  # aligned stand-ins: rejected before anything is read
    _expect_invalid("hses_add_ln_shift", v, v, 4, 8, 512, v, v, 1e-5, v, NULL, v, 6, v, 7, NULL, 8,
                    NULL)  # out_fmt
    _expect_invalid("hses_add_ln_shift", v, v, 4, 8, 512, v, v, 1e-5, v, NULL, v, 6, v,
                    _lib.FMT_BF16, v, 9, NULL)  # length past T with y_last
    _expect_invalid("hses_add_ln_shift", NULL, v, 4, 8, 512, v, v, 1e-5, v, NULL, v, 6, v,
                    _lib.FMT_BF16, NULL, 8, NULL)
    for C, n_mix, x in ((64, 6, v), (512, 3, v), (512, 6, ctypes.c_void_p(260))):
        rc = lib.hses_add_ln_shift(x, v, 4, 8, C, v, v, 1e-5, v, NULL, v, n_mix, v, _lib.FMT_BF16,
                                   NULL, 8, NULL)
        assert rc == _lib.HSES_ERR_UNSUPPORTED, (C, n_mix, rc)


def test_validation_rejects_bad_arguments_without_a_gpu():
    _expect_invalid("hses_bm_eval", 2**24 - 4, 8, NULL, NULL, NULL, NULL)
    _expect_invalid("hses_lora_factors", 0.1, 1, 4, 0, -1, 0, NULL, 2, 3, 4, NULL, NULL, NULL)
    _expect_invalid("hses_lora_factors", 0.1, 1, 4, 0, 0, 0, NULL, 2, 3, 4, NULL, NULL, NULL)
    _expect_invalid("hses_poisson_encode", NULL, 0, NULL, -1, 784, 784, 8, 0, 0, 0, 0, NULL, 0, 784, NULL)
    _expect_invalid("hses_poisson_encode", ctypes.c_void_p(16), 4, NULL, 4, 784, 700, 8, 0, 0, 0, 0,
                    ctypes.c_void_p(16), 0, 784, NULL)
    _expect_invalid("hses_poisson_encode", ctypes.c_void_p(16), 4, NULL, 4, 784, 784, 8, 0, 0, 0, 0,
                    ctypes.c_void_p(16), 3, 12, NULL)  # 784 bits need 13 words
    _expect_invalid("hses_poisson_encode", ctypes.c_void_p(16), 4, NULL, 4, 784, 784, 8, 0, 0, 0, 0,
                    ctypes.c_void_p(16), 9, 784, NULL)
    _expect_invalid("hses_poisson_encode", ctypes.c_void_p(16), 2**23, NULL, 2**23, 1024, 1024, 8, 0, 0, 0, 0,
                    ctypes.c_void_p(16), 0, 1024, NULL)  # flat index beyond u32
    _expect_invalid("hses_lif_scan", ctypes.c_void_p(16), NULL, 8, 4, 128, 128, 0.0, 1.0,
                    ctypes.c_void_p(16), 0, 128, NULL, NULL)
    _expect_invalid("hses_lif_scan", ctypes.c_void_p(16), NULL, 8, 4, 128, 100, 10.0, 1.0,
                    ctypes.c_void_p(16), 0, 128, NULL, NULL)
    _expect_invalid("hses_convert_fitnesses", NULL, 0, 0, NULL, NULL, NULL)
    _expect_invalid("hses_convert_fitnesses", ctypes.c_void_p(16), 10, 3, ctypes.c_void_p(16),
                    NULL, NULL)
    _expect_invalid("hses_solver_step", 7, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, ctypes.c_void_p(16),
                    ctypes.c_void_p(16), NULL, NULL, 4, NULL)
    _expect_invalid("hses_solver_step", 1, 0.1, 0.9, 0.999, 1e-8, 0.0, 0, ctypes.c_void_p(16),
                    ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 4, NULL)
    _expect_invalid("hses_member_loglik", NULL, 0, NULL, 4, 2, NULL, NULL)
    _expect_invalid("hses_member_fitness", ctypes.c_void_p(16), 10, ctypes.c_void_p(16), 4, 2, 2,
                    ctypes.c_void_p(16), NULL, NULL)  # unknown reward
    _expect_invalid("hses_member_fitness", NULL, 10, NULL, 4, 2, 0, NULL, NULL, NULL)
    _expect_invalid("hses_fitness_moments", ctypes.c_void_p(16), 4, NULL, 0, NULL)
    _expect_invalid("hses_combine_affine", ctypes.c_void_p(16), NULL, ctypes.c_void_p(16), 0, 4,
                    ctypes.c_void_p(16), NULL)  # batch 0
    _expect_invalid("hses_combine_affine", ctypes.c_void_p(16), NULL, NULL, 8, 4,
                    ctypes.c_void_p(16), NULL)
    _expect_invalid("hses_poisson_encode", ctypes.c_void_p(16), 3, NULL, 4, 784, 784, 8, 0, 0, 0,
                    0, ctypes.c_void_p(16), 0, 784, NULL)  # p has fewer rows than the output
    _expect_invalid("hses_spike_rate", ctypes.c_void_p(16), 3, 1, 16, 4, 128, ctypes.c_void_p(16),
                    NULL)  # 128 bits need 2 words
    _expect_invalid("hses_perturbed_linear", ctypes.c_void_p(16), 5, 784, 0, 1,
                    ctypes.c_void_p(16), 128, 784, 1, 4, 0.02, 0, 0, 0, 4, 8,
                    ctypes.c_void_p(16), 128, 0, 0, NULL, 0, NULL)
    _expect_invalid("hses_es_update", ctypes.c_void_p(16), 8, 0, 1, 4, 0.02, 0, 0, 16, 16, 1.0,
                    0, ctypes.c_void_p(16), NULL, 0, NULL)
    _expect_invalid("hses_perturbed_linear_act", ctypes.c_void_p(16), 0, 512, 0, 1,
                    ctypes.c_void_p(16), 512, 512, 1, 1, 0.02, 0, 0, 0, 4, 128,
                    ctypes.c_void_p(16), 512, 0, 1, 2, 0, 0, NULL, 0, NULL)  # transposed 2
    _expect_invalid("hses_perturbed_linear_act", ctypes.c_void_p(16), 7, 512, 0, 1,
                    ctypes.c_void_p(16), 512, 512, 1, 1, 0.02, 0, 0, 0, 4, 128,
                    ctypes.c_void_p(16), 512, 0, 1, 0, 1, 0, NULL, 0, NULL)  # unknown x format
    _expect_invalid("hses_token_shift_mix", ctypes.c_void_p(16), ctypes.c_void_p(16), NULL,
                    ctypes.c_void_p(16), 6, 2, 4, 8, ctypes.c_void_p(16), 3, NULL)  # out_fmt U8
    _expect_invalid("hses_tm_kk", ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                    ctypes.c_void_p(16), 4, 2, 65, ctypes.c_void_p(16), ctypes.c_void_p(16), NULL)
    _expect_invalid("hses_add_layer_norm", ctypes.c_void_p(16), ctypes.c_void_p(32), 4, 8,
                    ctypes.c_void_p(16), ctypes.c_void_p(16), 1e-5, ctypes.c_void_p(16), NULL)
    _expect_invalid("hses_rwkv_act", ctypes.c_void_p(16), 4, 5, NULL)
    _expect_invalid("hses_full_update", ctypes.c_void_p(16), 8, 0, 1, 0.02, 0, 0, 1024, 1024,
                    1.0, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), 1 << 30, NULL)  # a*b > 2^19
    _expect_invalid("hses_noisy_standard", ctypes.c_void_p(16), -1, 4, 1, 0.02, 0, 0, 0, NULL, 2,
                    ctypes.c_void_p(16), NULL)
    _expect_invalid("hses_clip_global_norm", NULL, NULL, 0, 1.0, ctypes.c_void_p(16),
                    ctypes.c_void_p(16), NULL)
    _expect_invalid("hses_solver_step_scaled", 9, 0.1, 0.9, 0.999, 1e-8, 0.0, 1,
                    ctypes.c_void_p(16), ctypes.c_void_p(16), NULL, NULL, 4, NULL, NULL)
    # the allocation-free ES update: one a x b partial must fit its fixed 32 MiB scratch
    _expect_invalid("hses_es_update_noalloc", ctypes.c_void_p(16), 8, 0, 1, 4, 0.02, 0, 0,
                    2048, 4096, 1.0, 0, ctypes.c_void_p(16), NULL)
    # hses_tm_fused: the output may not alias an input plane that other waves read
    P = [ctypes.c_void_p(4096 * (i + 1)) for i in range(24)]
    for alias in (0, 1, 2, 3, 4, 19):  # r, w, k, v, a, g
        _expect_invalid("hses_tm_fused", P[0], P[1], P[2], P[3], P[4], NULL, NULL, P[7], P[8],
                        NULL, P[10], P[11], P[12], NULL, 2, 8, 2, 64, 8, P[19], P[20], P[21],
                        64e-5, P[22], P[alias], 1, P[23], NULL)


def test_factor_record_bytes_and_validation():
    lib = _lib.load()
    c = ctypes.c_void_p
    # members [1, 5) span pairs 0, 1, 2; members [0, 4) pairs 0, 1
    assert lib.hses_factor_record_bytes(10, 20, 32, 1, 4) == 3 * 30 * 32 * 4
    assert lib.hses_factor_record_bytes(10, 20, 32, 0, 4) == 2 * 30 * 32 * 4
    assert lib.hses_factor_record_bytes(10, 20, 32, 0, 0) == 0
    assert lib.hses_factor_record_bytes(10, 20, 0, 0, 4) == 0
    # update from a record: rank >= 32, a record, and one large enough
    _expect_invalid("hses_es_update_rec", c(16), 8, 0, c(16), 1 << 20, 16, 0.02, 16, 16, 1.0, 0,
                    c(16), c(16), 1 << 20, NULL)
    _expect_invalid("hses_es_update_rec", c(16), 8, 0, NULL, 1 << 20, 32, 0.02, 16, 16, 1.0, 0,
                    c(16), c(16), 1 << 20, NULL)
    _expect_invalid("hses_es_update_rec", c(16), 8, 0, c(16), 4 * 32 * 32 * 4 - 4, 32, 0.02, 16,
                    16, 1.0, 0, c(16), c(16), 1 << 20, NULL)


def test_pair_image_bytes_and_validation():
    lib = _lib.load()
    c = ctypes.c_void_p
    # per pair: B^T as rank rows of b rounded up to 64, then A as a rows of 136, bf16
    assert lib.hses_pair_image_bytes(10, 20, 32, 1, 4) == 3 * (32 * 64 + 10 * 136) * 2
    assert lib.hses_pair_image_bytes(128, 784, 128, 0, 8192) == 4096 * (128 * 832 + 128 * 136) * 2
    assert lib.hses_pair_image_bytes(10, 20, 32, 0, 0) == 0
    rec = lib.hses_factor_record_bytes(128, 784, 128, 0, 8)
    img = lib.hses_pair_image_bytes(128, 784, 128, 0, 8)
    draw = lambda rank, sigma, a, r_ptr, r_bytes, i_ptr, i_bytes: (
        _expect_invalid("hses_pair_factors", 7, rank, sigma, 0, 0, 0, 8, a, 784, r_ptr, r_bytes,
                        i_ptr, i_bytes, NULL))
    draw(128, 0.02, 128, c(16), rec, c(16), img - 2)    # image too small
    draw(128, 0.02, 128, c(16), rec, NULL, img)         # no image
    draw(128, 0.02, 128, c(16), rec - 4, c(16), img)    # record too small
    draw(128, 0.02, 128, NULL, rec, c(16), img)         # no record
    draw(8, 0.02, 128, c(16), rec, c(16), img)          # rank below the pair kernels'
    draw(120, 0.02, 128, c(16), rec, c(16), img)        # rank not a multiple of 16
    draw(128, 0.0, 128, c(16), rec, c(16), img)         # sigma 0: nothing to draw
    draw(128, 0.02, 200, c(16), 1 << 30, c(16), 1 << 30)  # output wider than 128
    # the forwards on drawn factors check the same buffers before anything else
    M, words = 8 * 64, 13
    _expect_invalid("hses_perturbed_linear_lif_pre", c(16), 3, words, M * words, 16, c(16), 128,
                    784, 128, 0.02, 0, 8, 64, 10.0, 1.0, c(16), 2, M * 2, NULL, 0, c(16),
                    1 << 20, c(16), rec, c(16), img - 2, NULL)
    _expect_invalid("hses_perturbed_linear_pre", c(16), 0, 784, M * 784, 1, c(16), 128, 784,
                    128, 0.02, 0, 8, 64, c(16), 128, M * 128, c(16), 1 << 20, c(16), rec - 4,
                    c(16), img, NULL)


def test_empty_inputs_are_no_ops_without_a_gpu():
    lib = _lib.load()
    assert lib.hses_poisson_encode(NULL, 0, NULL, 0, 784, 784, 8, 0, 0, 0, 0, NULL, 0, 784, NULL) == 0
    assert lib.hses_lif_scan(NULL, NULL, 8, 0, 128, 128, 10.0, 1.0, NULL, 0, 128, NULL, NULL) == 0
    assert lib.hses_lora_factors(0.1, 1, 4, 0, 0, 0, NULL, 0, 3, 4, NULL, NULL, NULL) == 0
    assert lib.hses_solver_step(0, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, NULL, NULL, NULL, NULL, 0,
                                NULL) == 0
    assert lib.hses_member_fitness(NULL, 10, NULL, 0, 4, 1, NULL, NULL, NULL) == 0
    assert lib.hses_combine_affine(NULL, NULL, NULL, 8, 0, NULL, NULL) == 0


def test_poisson_pool_validation_without_a_gpu():
    lib = _lib.load()
    assert lib.hses_poisson_pool_bytes(10, 3000) == 0
    assert lib.hses_poisson_pool_bytes(0, 784) == 0
    # 10 rows of 784: counts (80 B), thresholds (10 x 784 x 4), columns (10 x 784 x 2)
    assert lib.hses_poisson_pool_bytes(10, 784) == 80 + 31360 + 15680
    v = ctypes.c_void_p(256)
    nb = lib.hses_poisson_pool_bytes(10, 784)
    _expect_invalid("hses_poisson_encode_pool", v, nb, 10, 784, NULL, 10, 12, 0, 0, 0, 0, v,
                    13 * 12, 13, NULL)  # T not a power of two
    _expect_invalid("hses_poisson_encode_pool", v, nb - 16, 10, 784, NULL, 10, 16, 0, 0, 0, 0, v,
                    13 * 16, 13, NULL)  # pool buffer too small
    _expect_invalid("hses_poisson_encode_pool", v, nb, 10, 784, NULL, 11, 16, 0, 0, 0, 0, v,
                    13 * 16, 13, NULL)  # more rows than the pool without an index
    _expect_invalid("hses_poisson_encode_pool", v, nb, 10, 784, NULL, 10, 16, 0, 0, 0, 0, v,
                    13 * 16, 12, NULL)  # time planes overlap
    _expect_invalid("hses_poisson_pool_prepare", v, 10, 784, 700, v, nb, NULL)  # p_stride
    _expect_invalid("hses_poisson_pool_prepare", v, 10, 784, 784, ctypes.c_void_p(264), nb, NULL)
