"""Host-side logic of the RWKV-7 LM ES step (no GPU): sizing, parameter layout,
FLOP accounting and configuration checks."""
import numpy as np
import pytest

from hyperscalees_amd import rwkv_lm


def test_lora_widths_follow_the_rwkv7_sizing_rule():
    # C = 512: decay / in-context rate max(32, round(1.8 sqrt(C) / 32) * 32) = 32,
    # value 1.3 sqrt(C) -> 32, gate 0.6 C^0.8 = 88.4 -> 96
    assert rwkv_lm.lora_widths(512) == (32, 32, 32, 96)
    assert rwkv_lm.lora_widths(2048) == (96, 64, 96, 256)


def test_mm_parameters_and_shapes():
    cfg = rwkv_lm.RwkvLmConfig(n_layer=2, d_model=64, head_size=32, widths=(16, 8, 16, 32))
    P = rwkv_lm.init_params(cfg, seed=0)
    names = rwkv_lm.mm_names(cfg.n_layer)
    assert len(names) == 2 * 14 and len(set(names)) == len(names)
    B = P["blocks"][1]
    C, F = 64, 256
    for n in ("receptance", "key", "value", "output"):
        assert B[n].shape == (C, C)
    assert B["w1"].shape == (C, 16) and B["w2"].shape == (16, C)
    assert B["v1"].shape == (C, 8) and B["g2"].shape == (32, C)
    assert B["ffn_key"].shape == (F, C) and B["ffn_value"].shape == (C, F)
    assert np.all(B["ln_w"] == 1) and np.all(B["ln_b"] == 0)
    assert P["emb"].shape == (cfg.vocab, C) and P["head"].shape == (cfg.vocab, C)


def test_forward_flops_hand_count():
    # one layer, C=4, F=8, V=3, widths (2, 2, 2, 2), r=1, 2 sequences of 5 tokens
    cfg = rwkv_lm.RwkvLmConfig(n_layer=1, d_model=4, head_size=4, vocab=3, ffn_mult=2,
                               seq_len=5, n=2, rank=1, widths=(2, 2, 2, 2))
    per_row = 0
    for a, b in [(4, 4)] * 4 + [(4, 2), (2, 4)] * 3 + [(8, 4), (4, 8)]:   # no v1/v2 at layer 0
        per_row += 2 * a * b + 2 * (a + b)
    per_row += 2 * 3 * 4
    assert rwkv_lm.forward_flops(cfg) == 10 * per_row


def test_config_rejects_heads_wider_than_a_wave():
    with pytest.raises(ValueError):
        rwkv_lm.RwkvLmConfig(d_model=256, head_size=128)
    with pytest.raises(ValueError):
        rwkv_lm.RwkvLmConfig(d_model=100, head_size=64)
