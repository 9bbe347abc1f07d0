/* Public C types shared by the engine ABI (engine.h), the kernel-level test
 * ABI (kernels.h) and the synthetic weight specification (synth.h).
 *
 * ChkConfig restates the reference's `Qwen4ExpConfig`
 * (/root/reference/src/qwen4_exp/config.rs:9-54) as a flat C struct with the
 * same field meanings.  Two encodings differ, both for a C ABI:
 *   - `layer_types: Vec<String>` becomes `full_attention_interval`: layer l is
 *     full ("qwen_sparse_attention") attention iff (l + 1) % interval == 0,
 *     which is how every qwen4_exp config lays layers out
 *     (tests/fixtures/qwen4_exp/config.json "full_attention_interval": 4);
 *   - `output_gate_type` must be "sigmoid" (the reference engine refuses any
 *     other, src/qwen4_exp/gpu/load.rs:49-52), so it is not a field.
 * PLE (`ple_layer_ids`, config.rs:36-43): `ple_layer` is the first entry
 * of ple_layer_ids (1-based, as the config writes it; Qwen4ExpConfig::
 * ple_layer, config.rs:119-122), 0 for none.  The n-gram table's row group
 * comes from the store's manifest (manifest.rs:42-55); a synthetic table
 * has ngram_head_rows - h rows in head h.
 */
#ifndef CHERENKOV_TYPES_H
#define CHERENKOV_TYPES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ChkConfig {
    uint32_t hidden_size;
    uint32_t num_hidden_layers;
    uint32_t full_attention_interval;
    uint32_t vocab_size;
    /* gated attention */
    uint32_t num_attention_heads;
    uint32_t num_key_value_heads;
    uint32_t head_dim;
    /* gated DeltaNet */
    uint32_t linear_num_key_heads;
    uint32_t linear_num_value_heads;
    uint32_t linear_key_head_dim;
    uint32_t linear_value_head_dim;
    uint32_t linear_conv_kernel_dim;
    /* hyper-connections */
    uint32_t hc_count;
    uint32_t hc_lowrank;
    /* mixture of experts */
    uint32_t num_experts;
    uint32_t num_experts_per_tok;
    uint32_t moe_intermediate_size;
    uint32_t shared_expert_intermediate_size;
    uint32_t norm_topk_prob;
    /* QSA indexer */
    uint32_t indexer_n_heads;
    uint32_t indexer_head_dim;
    uint32_t indexer_budget;
    uint32_t indexer_compress_ratio;
    /* misc */
    uint32_t mtp_num_hidden_layers;
    uint32_t eos_token_id;
    uint32_t ple_layer; /* 1-based layer of the PLE block, 0 = none */
    double rms_norm_eps;
    double partial_rotary_factor;
    double rope_theta;
    /* synthetic weights: seed of the counter-hash generator (synth.h) */
    uint64_t seed;
    /* PLE n-gram block (read when ple_layer != 0) */
    uint32_t ple_conv_kernel_size; /* dilated depthwise conv taps */
    uint32_t ple_embed_dim;        /* n-gram embedding width: ids x row dim */
    uint32_t ngram_size;           /* largest n-gram (3: bigram + trigram heads); the conv dilation */
    uint32_t heads_per_ngram;
    uint32_t ngram_group;          /* quantisation group of a table row */
    uint32_t ngram_head_rows;      /* synthetic table: rows of head 0 */
} ChkConfig;

/* Expert precision of the routed-expert store (Options::experts,
 * src/options.rs:97-99).  The shared expert always stays 4-bit. */
enum { CHK_EXPERTS_Q4 = 4, CHK_EXPERTS_Q3 = 3, CHK_EXPERTS_Q2 = 2 };

/* Engine options that reach `Gpu::load` (src/options.rs:94-141). */
typedef struct ChkOptions {
    uint32_t experts;  /* 4, 3 or 2 */
    uint32_t drafts;   /* MTP drafts 0..3 */
    uint32_t max_t;    /* context capacity */
    uint32_t no_eos;   /* ignore EOS in the runner */
} ChkOptions;

#ifdef __cplusplus
}
#endif

#endif
