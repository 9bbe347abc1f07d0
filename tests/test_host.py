"""Host-side logic without a GPU: the presets' shapes and the algorithmic
bytes model the bench prices its roofline with."""

from __future__ import annotations

from cherenkov_amd import presets


def test_decode_bytes_per_token_matches_the_term_table():
    """Per-token decode bytes of the 48-layer 80B-A3B-shape preset, Q4,
    drafts 0: MoE 48 x 21,565,440; HC reads 48 x 5,967,872; DeltaNet
    projections 36 x 18,948,096 and state/conv 36 x 4,456,448; attention
    projections 12 x 15,335,424 and index projections 12 x 737,280; final
    mixer 2,965,504; LM head 175,030,272; plus 13,056 bytes of q8 KV per
    context token (12 layers x 2 sides x (512 + 32))."""
    cfg = presets.qwen3next_80b_shape()
    fixed = (48 * 21_565_440 + 48 * 5_967_872 + 36 * 18_948_096 + 36 * 4_456_448 + 12 * 15_335_424
             + 12 * 737_280 + 2_965_504 + 175_030_272)
    assert fixed == 2_535_030_784
    for T in (1, 2048, 4096):
        assert presets.decode_bytes_per_token(cfg, T, 4) == fixed + 13_056 * T


def test_lowbit_experts_shrink_only_routed_records():
    cfg = presets.qwen3next_80b_shape()
    q4 = presets.decode_bytes_per_token(cfg, 2048, 4)
    per_weight = {3: 0.4375, 2: 0.3125}
    routed_weights = 48 * 10 * 3 * 512 * 2048
    for bits, bpw in per_weight.items():
        saved = presets.decode_bytes_per_token(cfg, 2048, 4) - presets.decode_bytes_per_token(cfg, 2048, bits)
        assert saved == int(routed_weights * (0.5625 - bpw))
    assert q4 > 0


def test_presets_meet_kernel_layout_rules():
    for cfg in (presets.tiny(), presets.qwen3next_80b_shape()):
        assert cfg.hidden_size % 256 == 0
        assert cfg.moe_intermediate_size % 64 == 0
        assert cfg.num_experts_per_tok * 4 < 64
        assert cfg.head_dim in (128, 256)
        assert cfg.num_attention_heads // cfg.num_key_value_heads in (1, 2, 4, 8, 12)
