"""Model presets (qwen4_exp semantics, Qwen3-Next-80B-A3B dimensions).

qwen3next_80b_shape: 48 layers in a repeating (DeltaNet, DeltaNet,
DeltaNet, gated attention) pattern, hidden 2048, 512 experts top-10 plus a
shared expert of width 512, vocab 151936, DeltaNet 16 key heads / 32 value
heads of 128, attention 16 q / 2 kv heads of 256 with RoPE on 25% of the
dims, hyper-connections hc = 4 with low rank 320 (the qwen4_exp fixture's
values, tests/fixtures/qwen4_exp/config.json), the QSA indexer present
(4 x 128) with a budget above every context this engine runs (so selection
is exactly dense), one MTP layer, no PLE block.

tiny: the CPU-runnable parity model — 4 layers (3 DeltaNet + 1 attention),
hidden 512, 16 experts top-2 plus a shared expert, expert width 256, vocab
4096; the remaining dimensions are this build's choice: DeltaNet 4 key /
8 value heads of 128, attention 4 q / 2 kv heads of 256, hc 4 / low rank
64, indexer 2 x 128, one MTP layer.
"""

from __future__ import annotations

from .abi import ChkConfig, make_config

QSA_DENSE_BUDGET = 65536


def qwen3next_80b_shape(seed: int = 20261201, layers: int = 48, mtp: int = 1) -> ChkConfig:
    return make_config(
        hidden_size=2048,
        num_hidden_layers=layers,
        full_attention_interval=4,
        vocab_size=151936,
        num_attention_heads=16,
        num_key_value_heads=2,
        head_dim=256,
        linear_num_key_heads=16,
        linear_num_value_heads=32,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        hc_count=4,
        hc_lowrank=320,
        num_experts=512,
        num_experts_per_tok=10,
        moe_intermediate_size=512,
        shared_expert_intermediate_size=512,
        norm_topk_prob=1,
        indexer_n_heads=4,
        indexer_head_dim=128,
        indexer_budget=QSA_DENSE_BUDGET,
        indexer_compress_ratio=4,
        mtp_num_hidden_layers=mtp,
        eos_token_id=151645,
        ple_layer=0,
        rms_norm_eps=1e-6,
        partial_rotary_factor=0.25,
        rope_theta=1e7,
        seed=seed,
    )


def tiny(seed: int = 1234, layers: int = 4, mtp: int = 1, indexer_budget: int = QSA_DENSE_BUDGET) -> ChkConfig:
    return make_config(
        hidden_size=512,
        num_hidden_layers=layers,
        full_attention_interval=4,
        vocab_size=4096,
        num_attention_heads=4,
        num_key_value_heads=2,
        head_dim=256,
        linear_num_key_heads=4,
        linear_num_value_heads=8,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        hc_count=4,
        hc_lowrank=64,
        num_experts=16,
        num_experts_per_tok=2,
        moe_intermediate_size=256,
        shared_expert_intermediate_size=256,
        norm_topk_prob=1,
        indexer_n_heads=2,
        indexer_head_dim=128,
        indexer_budget=indexer_budget,
        indexer_compress_ratio=4,
        mtp_num_hidden_layers=mtp,
        eos_token_id=4095,
        ple_layer=0,
        rms_norm_eps=1e-6,
        partial_rotary_factor=0.25,
        rope_theta=1e7,
        seed=seed,
    )


def qwen4_exp_fixture(seed: int = 1234) -> ChkConfig:
    """The qwen4_exp test checkpoint's text_config (the reference's
    tests/fixtures/qwen4_exp/config.json: 4 layers with the attention
    layer last, hidden 256, hc 4 / low rank 320, 8 experts top-4 of width
    256 plus a shared expert of 256, DeltaNet 16 key / 48 value heads of
    128, attention 8 q / 2 kv heads of 256, the QSA indexer 4 x 128 with
    budget 2048, vocab 248,320, one MTP layer, a PLE block before layer 2
    with 3-grams, 8 heads per order, embed dim 256 and conv kernel 4),
    on synthetic weights; the n-gram rows are groups of 16
    (tests/import.rs:52) and the synthetic table holds 1021 - h rows in
    head h."""
    return with_ple(make_config(
        hidden_size=256,
        num_hidden_layers=4,
        full_attention_interval=4,
        vocab_size=248320,
        num_attention_heads=8,
        num_key_value_heads=2,
        head_dim=256,
        linear_num_key_heads=16,
        linear_num_value_heads=48,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        hc_count=4,
        hc_lowrank=320,
        num_experts=8,
        num_experts_per_tok=4,
        moe_intermediate_size=256,
        shared_expert_intermediate_size=256,
        norm_topk_prob=1,
        indexer_n_heads=4,
        indexer_head_dim=128,
        indexer_budget=2048,
        indexer_compress_ratio=4,
        mtp_num_hidden_layers=1,
        eos_token_id=248044,
        ple_layer=0,
        rms_norm_eps=1e-6,
        partial_rotary_factor=0.25,
        rope_theta=1e7,
        seed=seed,
    ), layer=2, embed_dim=256, ngram_size=3, heads_per_ngram=8, group=16, head_rows=1021, kernel=4)


def wide(seed: int = 4096, layers: int = 4) -> ChkConfig:
    """A 4096-wide model for parity at the engine's widest hidden size:
    the 80B shape's DeltaNet (16 / 32 heads of 128) and attention (16 q /
    2 kv heads of 256) with hidden 4096, 32 experts top-4 of width 512
    plus a shared expert, vocab 4096, one MTP layer."""
    return make_config(
        hidden_size=4096,
        num_hidden_layers=layers,
        full_attention_interval=4,
        vocab_size=4096,
        num_attention_heads=16,
        num_key_value_heads=2,
        head_dim=256,
        linear_num_key_heads=16,
        linear_num_value_heads=32,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        hc_count=4,
        hc_lowrank=320,
        num_experts=32,
        num_experts_per_tok=4,
        moe_intermediate_size=512,
        shared_expert_intermediate_size=512,
        norm_topk_prob=1,
        indexer_n_heads=4,
        indexer_head_dim=128,
        indexer_budget=QSA_DENSE_BUDGET,
        indexer_compress_ratio=4,
        mtp_num_hidden_layers=1,
        eos_token_id=4095,
        ple_layer=0,
        rms_norm_eps=1e-6,
        partial_rotary_factor=0.25,
        rope_theta=1e7,
        seed=seed,
    )


def with_ple(c: ChkConfig, layer: int = 2, embed_dim: int = 256, ngram_size: int = 3, heads_per_ngram: int = 8,
             group: int = 16, head_rows: int = 1021, kernel: int = 4) -> ChkConfig:
    """`c` with a PLE n-gram block before decoder layer `layer` (1-based, as
    ple_layer_ids writes it).  The defaults are the qwen4_exp fixture's
    (tests/fixtures/qwen4_exp/config.json: ple_layer_ids [2], embed dim 256,
    3-grams, 8 heads per order, conv kernel 4; its n-gram rows are groups of
    16, tests/import.rs:52); the synthetic table has head_rows - h rows in
    head h."""
    c.ple_layer = layer
    c.ple_embed_dim = embed_dim
    c.ngram_size = ngram_size
    c.heads_per_ngram = heads_per_ngram
    c.ngram_group = group
    c.ngram_head_rows = head_rows
    c.ple_conv_kernel_size = kernel
    return c


def decode_bytes_per_token(c: ChkConfig, ctx: int, expert_bits: int = 4) -> int:
    """Algorithmic HBM bytes of one batch-1 decode step (drafts = 0):
    every weight the step reads once, DeltaNet state read + write, conv
    history read + write, KV rows of the visible context, routed experts at
    `expert_bits` (the shared expert stays Q4).  Matches the per-term
    accounting of the blueprint's row D1 for the 80B-shape preset."""
    q4 = lambda out, inp: out * inp // 2 + 2 * 2 * (out * inp // 64)  # noqa: E731
    H, hc = c.hidden_size, c.hc_count
    hh = H * hc
    lr = c.hc_lowrank
    hc_read = q4(lr, hh) + q4(hh, lr) + q4(hc, hh) + 2 * hh
    final_mix = q4(lr, hh) + q4(hh, lr) + 2 * hh
    nk, nv, dk, dv = c.linear_num_key_heads, c.linear_num_value_heads, c.linear_key_head_dim, c.linear_value_head_dim
    conv_dim = 2 * nk * dk + nv * dv
    dn_proj = q4(conv_dim, H) + q4(nv * dv, H) + 2 * q4(nv, H) + q4(H, nv * dv)
    dn_state = 2 * nv * dk * dv * 4 + 2 * conv_dim * (c.linear_conv_kernel_dim - 1) * 4 + conv_dim * c.linear_conv_kernel_dim * 2
    nh, nkv, hd = c.num_attention_heads, c.num_key_value_heads, c.head_dim
    at_proj = q4(2 * nh * hd, H) + 2 * q4(nkv * hd, H) + q4(H, nh * hd)
    idx_proj = q4((c.indexer_n_heads + 1) * c.indexer_head_dim, H)
    I = c.moe_intermediate_size
    rec = {4: 3 * q4(I, H), 3: 3 * (I * H * 3 // 8) + 6 * (I * H // 32), 2: 3 * (I * H // 4) + 6 * (I * H // 32)}[expert_bits]
    moe = c.num_experts * H * 2 + c.num_experts_per_tok * rec + 3 * q4(I, H) + 2 * H
    kv_row = nkv * hd
    kv_per_tok = 2 * (kv_row + kv_row // 32 * 2)
    L = c.num_hidden_layers
    n_at = sum(1 for l in range(L) if (l + 1) % c.full_attention_interval == 0)
    n_dn = L - n_at
    lm = q4(c.vocab_size, H)
    total = (
        L * moe
        + L * 2 * hc_read
        + n_dn * (dn_proj + dn_state)
        + n_at * (at_proj + idx_proj)
        + final_mix
        + lm
        + n_at * kv_per_tok * ctx
    )
    return int(total)
