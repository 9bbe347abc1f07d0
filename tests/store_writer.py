"""Writes a packed store in the reference's on-disk format from the oracle's
synthetic weights (test infrastructure: the fixture generator of the
packed-store loader tests).

Format (the reference's pack.rs output, read by Packed::open,
src/qwen4_exp/packed.rs:66-231):
  config.json    HF-style, the text model under "text_config"
                 (Qwen4ExpConfig, src/qwen4_exp/config.rs:9-122);
  manifest.json  {version 1, source_dir, dense: [{name, dtype, shape,
                 offset, nbytes}], experts: ExpertLayout, ngram:
                 NgramLayout} (src/qwen4_exp/manifest.rs:7-110);
  dense.bin      every dense tensor at its manifest offset: Q4 linears as
                 {prefix}.weight U32 [out, in/8], .scales / .biases BF16
                 [out, in/64]; norms, router and conv weights BF16;
  experts.bin    record (layer, expert) at (layer * experts + expert) *
                 record_stride, fields gate_w, up_w, down_w, gate_s,
                 gate_b, up_s, up_b, down_s, down_b (pack.rs:351-393),
                 the stride padded to 16 KiB pages;
  ngram.bin      the n-gram table's rows (weight | scales | biases) of a
                 PLE layer, else empty; its hash metadata are I64 dense
                 tensors {layer}.ple.ple_embedding.{layer_multipliers,
                 ngram_heads_offsets, ngram_heads_vocab_sizes}
                 (packed.rs:134-148, 233-256; pack.rs:476-592).
Tensor names follow src/qwen4_exp/cpu.rs:143-272.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from oracle.oracle import OracleModel

PAGE = 16384


def _names(cfg) -> list[tuple[str, str, int, str, tuple]]:
    """(store name, kind, layer, oracle name, shape) of every dense tensor;
    kind "q4" (shape = (out, in)) or "bf16" (shape = store shape)."""
    c = cfg
    H, hc, L = c.hidden_size, c.hc_count, c.num_hidden_layers
    hh, lr = H * hc, c.hc_lowrank
    m = "language_model.model"
    qk, vd = c.linear_num_key_heads * c.linear_key_head_dim, c.linear_num_value_heads * c.linear_value_head_dim
    conv_dim = 2 * qk + vd
    hd, ihd = c.head_dim, c.indexer_head_dim
    out = [(f"{m}.embed_tokens", "q4", 0, "embed", (c.vocab_size, H)),
           ("language_model.lm_head", "q4", 0, "lm_head", (c.vocab_size, H))]

    def hc_block(prefix, grp, layer, inject):
        out.append((f"{prefix}.hc_norm.weight", "bf16", layer, f"{grp}.norm", (hh,)))
        out.append((f"{prefix}.input_mix_weight_down", "q4", layer, f"{grp}.down", (lr, hh)))
        out.append((f"{prefix}.input_mix_weight_up", "q4", layer, f"{grp}.up", (hh, lr)))
        if inject:
            out.append((f"{prefix}.block_inject_weight", "q4", layer, f"{grp}.inject", (hc, hh)))

    def layer(lp, l, linear):
        hc_block(f"{lp}.attn_hyper_connection", "attn_hc", l, True)
        hc_block(f"{lp}.mlp_hyper_connection", "mlp_hc", l, True)
        if linear:
            d = f"{lp}.linear_attn"
            out.extend([
                (f"{d}.in_proj_qkv", "q4", l, "dn.qkv", (conv_dim, H)),
                (f"{d}.in_proj_z", "q4", l, "dn.z", (vd, H)),
                (f"{d}.in_proj_a", "q4", l, "dn.a", (c.linear_num_value_heads, H)),
                (f"{d}.in_proj_b", "q4", l, "dn.b", (c.linear_num_value_heads, H)),
                (f"{d}.out_proj", "q4", l, "dn.out", (H, vd)),
                (f"{d}.conv1d.weight", "bf16", l, "dn.conv", (conv_dim, 1, c.linear_conv_kernel_dim)),
                (f"{d}.A_log", "bf16", l, "dn.a_log", (c.linear_num_value_heads,)),
                (f"{d}.dt_bias", "bf16", l, "dn.dt_bias", (c.linear_num_value_heads,)),
                (f"{d}.norm.weight", "bf16", l, "dn.norm", (c.linear_value_head_dim,)),
            ])
        else:
            a = f"{lp}.self_attn"
            out.extend([
                (f"{a}.q_proj", "q4", l, "at.q", (2 * c.num_attention_heads * hd, H)),
                (f"{a}.k_proj", "q4", l, "at.k", (c.num_key_value_heads * hd, H)),
                (f"{a}.v_proj", "q4", l, "at.v", (c.num_key_value_heads * hd, H)),
                (f"{a}.o_proj", "q4", l, "at.o", (H, c.num_attention_heads * hd)),
                (f"{a}.q_norm.weight", "bf16", l, "at.q_norm", (hd,)),
                (f"{a}.k_norm.weight", "bf16", l, "at.k_norm", (hd,)),
                (f"{a}.indexer.index_qk_proj", "q4", l, "at.idx", ((c.indexer_n_heads + 1) * ihd, H)),
                (f"{a}.indexer.q_layernorm.weight", "bf16", l, "at.idx_q_norm", (ihd,)),
                (f"{a}.indexer.k_layernorm.weight", "bf16", l, "at.idx_k_norm", (ihd,)),
            ])
        out.extend([
            (f"{lp}.mlp.gate.weight", "bf16", l, "moe.router", (c.num_experts, H)),
            (f"{lp}.mlp.shared_expert_gate.weight", "bf16", l, "moe.shared_gate", (1, H)),
            (f"{lp}.mlp.shared_expert.gate_proj", "q4", l, "moe.sh_gate", (c.shared_expert_intermediate_size, H)),
            (f"{lp}.mlp.shared_expert.up_proj", "q4", l, "moe.sh_up", (c.shared_expert_intermediate_size, H)),
            (f"{lp}.mlp.shared_expert.down_proj", "q4", l, "moe.sh_down", (H, c.shared_expert_intermediate_size)),
        ])

    for l in range(L):
        layer(f"{m}.layers.{l}", l, (l + 1) % c.full_attention_interval != 0)
        if c.ple_layer == l + 1:
            p = f"{m}.layers.{l}.ple"
            E, K = c.ple_embed_dim, c.ple_conv_kernel_size
            out.extend([
                (f"{p}.key_proj", "q4", l, "ple.key", (hh, E)),
                (f"{p}.value_proj", "q4", l, "ple.value", (H, E)),
                (f"{p}.norm_key.weight", "bf16", l, "ple.norm_key", (hh,)),
                (f"{p}.norm_query.weight", "bf16", l, "ple.norm_query", (hh,)),
                (f"{p}.norm_conv.weight", "bf16", l, "ple.norm_conv", (hh,)),
                (f"{p}.conv1d.weight", "bf16", l, "ple.conv", (hh, 1, K)),
            ])
    hc_block(f"{m}.hyper_connection_mixer", "final", 0, False)
    if c.mtp_num_hidden_layers:
        out.extend([
            ("mtp.pre_fc_norm_embedding.weight", "bf16", L, "mtp.enorm", (H,)),
            ("mtp.pre_fc_norm_hidden.weight", "bf16", L, "mtp.hnorm", (hh,)),
            ("mtp.fc_embedding", "q4", L, "mtp.fc_e", (H, H)),
            ("mtp.fc_hidden", "q4", L, "mtp.fc_h", (H, H)),
        ])
        layer("mtp.layers.0", L, False)
        hc_block("mtp.hyper_connection_mixer", "mtp_mixer", L, False)
    return out


def text_config(cfg) -> dict:
    c = cfg
    L = c.num_hidden_layers
    types = ["linear_attention" if (l + 1) % c.full_attention_interval else "full_attention" for l in range(L)]
    return {
        "model_type": "qwen4_exp_text",
        "hidden_size": c.hidden_size, "num_hidden_layers": L, "layer_types": types,
        "vocab_size": c.vocab_size, "num_attention_heads": c.num_attention_heads,
        "num_key_value_heads": c.num_key_value_heads, "head_dim": c.head_dim,
        "linear_num_key_heads": c.linear_num_key_heads, "linear_num_value_heads": c.linear_num_value_heads,
        "linear_key_head_dim": c.linear_key_head_dim, "linear_value_head_dim": c.linear_value_head_dim,
        "linear_conv_kernel_dim": c.linear_conv_kernel_dim, "rms_norm_eps": c.rms_norm_eps,
        "partial_rotary_factor": c.partial_rotary_factor, "rope_parameters": {"rope_theta": c.rope_theta},
        "hc_count": c.hc_count, "hc_lowrank": c.hc_lowrank, "num_experts": c.num_experts,
        "num_experts_per_tok": c.num_experts_per_tok, "moe_intermediate_size": c.moe_intermediate_size,
        "shared_expert_intermediate_size": c.shared_expert_intermediate_size,
        "norm_topk_prob": bool(c.norm_topk_prob), "ple_layer_ids": [c.ple_layer] if c.ple_layer else [],
        "ple_embed_dim": c.ple_embed_dim, "ple_conv_kernel_size": c.ple_conv_kernel_size,
        "ngram_size": c.ngram_size, "heads_per_ngram": c.heads_per_ngram,
        "indexer_n_heads": c.indexer_n_heads, "indexer_kv_heads": 1, "indexer_head_dim": c.indexer_head_dim,
        "indexer_budget": c.indexer_budget, "indexer_compress_ratio": c.indexer_compress_ratio,
        "output_gate_type": "sigmoid", "eos_token_id": c.eos_token_id,
        "mtp_num_hidden_layers": c.mtp_num_hidden_layers,
    }


def write_store(cfg, path, shuffle_dense: bool = True, field_order: tuple | None = None) -> Path:
    """Write the store of the synthetic model `cfg` under `path`.
    shuffle_dense writes dense.bin in reverse name order (offsets are what
    the reader must follow); field_order permutes the record fields (the
    manifest's offsets then differ from the engine's own layout)."""
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    orc = OracleModel(cfg)
    c = cfg
    entries = []
    chunks = []
    off = 0
    names = _names(cfg)
    if shuffle_dense:
        names = names[::-1]
    for name, kind, layer, oname, shape in names:
        if kind == "q4":
            w, s, b = orc.get_q4(layer, oname, shape[0], shape[1])
            parts = [(".weight", "U32", [shape[0], shape[1] // 8], w), (".scales", "BF16", [shape[0], shape[1] // 64], s),
                     (".biases", "BF16", [shape[0], shape[1] // 64], b)]
        else:
            v = orc.get_bf16(layer, oname, int(np.prod(shape)))
            parts = [("", "BF16", list(shape), v)]
        for suffix, dtype, shp, arr in parts:
            data = np.ascontiguousarray(arr).tobytes()
            pad = (-off) % 64
            if pad:
                chunks.append(b"\0" * pad)
                off += pad
            entries.append({"name": name + suffix, "dtype": dtype, "shape": shp, "offset": off, "nbytes": len(data)})
            chunks.append(data)
            off += len(data)
    ngram = {"rows": 0, "row_bytes": 0, "dim": 0, "group": 64, "weight_bytes": 0, "scale_bytes": 0,
             "head_offsets": [], "head_vocab_sizes": [], "layer_multipliers": []}
    table = b""
    if c.ple_layer:
        mult, offs, sz = orc.ngram_meta()
        pre = f"language_model.model.layers.{c.ple_layer - 1}.ple.ple_embedding"
        for leaf, arr in (("layer_multipliers", mult), ("ngram_heads_offsets", offs.astype(np.int64)),
                          ("ngram_heads_vocab_sizes", sz.astype(np.int64))):
            data = np.ascontiguousarray(arr, dtype="<i8").tobytes()
            pad = (-off) % 64
            chunks.append(b"\0" * pad)
            off += pad
            entries.append({"name": f"{pre}.{leaf}", "dtype": "I64", "shape": [len(arr)], "offset": off,
                            "nbytes": len(data)})
            chunks.append(data)
            off += len(data)
        dim = c.ple_embed_dim // orc.ngram_heads()
        table = orc.ngram_table().tobytes()
        wb, sb = dim // 2, dim // c.ngram_group * 2
        # the manifest keeps copies of the metadata; readers use the dense
        # tensors (packed.rs:134-148), so these copies are deliberately off
        ngram = {"rows": len(table) // (wb + 2 * sb), "row_bytes": wb + 2 * sb, "dim": dim, "group": c.ngram_group,
                 "weight_bytes": wb, "scale_bytes": sb, "head_offsets": [0] * len(offs),
                 "head_vocab_sizes": [1] * len(sz), "layer_multipliers": [0] * len(mult)}
    (path / "dense.bin").write_bytes(b"".join(chunks))
    # experts: main layers then the MTP layer
    I, H = c.moe_intermediate_size, c.hidden_size
    codes = I * H
    su, sd = I * (H // 64) * 2, H * (I // 64) * 2
    sizes = {"gate_w": codes // 2, "up_w": codes // 2, "down_w": codes // 2, "gate_s": su, "gate_b": su,
             "up_s": su, "up_b": su, "down_s": sd, "down_b": sd}
    src_order = list(sizes)  # the oracle's records are in pack.rs order
    src_off, o = {}, 0
    for k in src_order:
        src_off[k] = o
        o += sizes[k]
    order = list(field_order) if field_order else src_order
    dst_off, o = {}, 0
    for k in order:
        dst_off[k] = o
        o += sizes[k]
    rec_bytes = o
    stride = (rec_bytes + PAGE - 1) // PAGE * PAGE
    prefixes = [f"language_model.model.layers.{l}.mlp.switch_mlp" for l in range(c.num_hidden_layers)]
    rls = list(range(c.num_hidden_layers))
    if c.mtp_num_hidden_layers:
        prefixes.append("mtp.layers.0.mlp.switch_mlp")
        rls.append(c.num_hidden_layers)
    with open(path / "experts.bin", "wb") as f:
        for rl in rls:
            for e in range(c.num_experts):
                rec = orc.expert_record(rl, e)
                out = np.zeros(stride, np.uint8)
                for k in order:
                    out[dst_off[k]:dst_off[k] + sizes[k]] = rec[src_off[k]:src_off[k] + sizes[k]]
                f.write(out.tobytes())
    (path / "ngram.bin").write_bytes(table)
    manifest = {
        "version": 1,
        "source_dir": "synthetic (seed %d)" % c.seed,
        "dense": entries,
        "experts": {"layers": len(prefixes), "experts": c.num_experts, "inter": I, "hidden": H, "group": 64,
                    "record_bytes": rec_bytes, "record_stride": stride, "layer_prefixes": prefixes, **dst_off},
        "ngram": ngram,
    }
    (path / "manifest.json").write_text(json.dumps(manifest, indent=1))
    (path / "config.json").write_text(json.dumps({"model_type": "qwen4_exp", "text_config": text_config(cfg)},
                                                 indent=1))
    return path
