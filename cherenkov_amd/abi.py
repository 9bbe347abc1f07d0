"""ctypes view of the C ABI in include/cherenkov/{types,engine,kernels}.h.

The engine, its kernels and its runner are native (libcherenkov.so); this
module only loads the library and declares signatures so that tests and
bench.py can drive it.  Loading fails loudly when the library is missing:
there is no Python or CPU fallback for any engine call.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libcherenkov.so"
NO_TOKEN = 0xFFFFFFFF  # CHK_NO_TOKEN: an absent optional token

u32, u64, f32, f64, i32 = C.c_uint32, C.c_uint64, C.c_float, C.c_double, C.c_int
P = C.c_void_p


class ChkConfig(C.Structure):
    _fields_ = [
        ("hidden_size", u32),
        ("num_hidden_layers", u32),
        ("full_attention_interval", u32),
        ("vocab_size", u32),
        ("num_attention_heads", u32),
        ("num_key_value_heads", u32),
        ("head_dim", u32),
        ("linear_num_key_heads", u32),
        ("linear_num_value_heads", u32),
        ("linear_key_head_dim", u32),
        ("linear_value_head_dim", u32),
        ("linear_conv_kernel_dim", u32),
        ("hc_count", u32),
        ("hc_lowrank", u32),
        ("num_experts", u32),
        ("num_experts_per_tok", u32),
        ("moe_intermediate_size", u32),
        ("shared_expert_intermediate_size", u32),
        ("norm_topk_prob", u32),
        ("indexer_n_heads", u32),
        ("indexer_head_dim", u32),
        ("indexer_budget", u32),
        ("indexer_compress_ratio", u32),
        ("mtp_num_hidden_layers", u32),
        ("eos_token_id", u32),
        ("ple_layer", u32),
        ("rms_norm_eps", f64),
        ("partial_rotary_factor", f64),
        ("rope_theta", f64),
        ("seed", u64),
        ("ple_conv_kernel_size", u32),
        ("ple_embed_dim", u32),
        ("ngram_size", u32),
        ("heads_per_ngram", u32),
        ("ngram_group", u32),
        ("ngram_head_rows", u32),
    ]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


class ChkOptions(C.Structure):
    _fields_ = [("experts", u32), ("drafts", u32), ("max_t", u32), ("no_eos", u32)]


class ChkMemoryStats(C.Structure):
    _fields_ = [
        ("dense", u64),
        ("experts", u64),
        ("experts_low_bit", u64),
        ("state", u64),
        ("kv_cache", u64),
        ("scratch", u64),
        ("total", u64),
    ]


class ChkExpertCounters(C.Structure):
    _fields_ = [
        ("selected_rows", u64),
        ("cache_hits", u64),
        ("cache_misses", u64),
        ("prefetch_requests", u64),
        ("read_requests", u64),
        ("read_bytes_requested", u64),
    ]


class ChkSampling(C.Structure):
    _fields_ = [
        ("temperature", f64),
        ("top_p", f64),
        ("top_k", u32),
        ("has_seed", u32),
        ("seed", u64),
        ("presence_penalty", f64),
        ("frequency_penalty", f64),
    ]


def make_config(**kw) -> ChkConfig:
    c = ChkConfig()
    for k, v in kw.items():
        if not hasattr(c, k):
            raise KeyError(k)
        setattr(c, k, v)
    return c


# (name, restype, argtypes) of every exported symbol, in header order.
SIGNATURES = [
    # engine.h
    ("chk_last_error", C.c_char_p, []),
    ("chk_engine_load", i32, [C.POINTER(ChkConfig), C.POINTER(ChkOptions), C.POINTER(P)]),
    ("chk_engine_free", None, [P]),
    ("chk_engine_load_store", i32, [C.c_char_p, C.POINTER(ChkOptions), C.POINTER(P)]),
    ("chk_engine_load_bounded", i32, [C.POINTER(ChkConfig), C.POINTER(ChkOptions), u64, u64, u32, C.POINTER(P)]),
    ("chk_engine_load_store_bounded", i32, [C.c_char_p, C.POINTER(ChkOptions), u64, u64, u32, C.POINTER(P)]),
    ("chk_store_config", i32, [C.c_char_p, C.POINTER(ChkConfig)]),
    ("chk_step_rows", i32, [P, C.POINTER(u32), u32, i32, i32, C.POINTER(u32)]),
    ("chk_step", i32, [P, u32, C.POINTER(u32)]),
    ("chk_commit", i32, [P, u32]),
    ("chk_reset", i32, [P]),
    ("chk_mtp_draft", i32, [P, C.POINTER(u32), u32, u32, C.POINTER(u32), C.POINTER(u32)]),
    ("chk_mtp_chain", i32, [P, u32, C.POINTER(u32)]),
    ("chk_prefill_chunk", i32, [P, C.POINTER(u32), u32, u32, i32, C.POINTER(u32), C.POINTER(u32)]),
    ("chk_prefill_release", None, [P]),
    ("chk_prefill_rows_fit", i32, [P, i32, C.POINTER(u32)]),
    ("chk_debug_engine_blocks", i32, [P, u32, C.POINTER(u32), u32, C.POINTER(u32)]),
    ("chk_debug_row_vis", i32, [P, u32, C.POINTER(u32), u32, C.POINTER(u32)]),
    ("chk_pf_logits_row", C.POINTER(f32), [P, u32]),
    ("chk_logits_row", C.POINTER(f32), [P, u32]),
    ("chk_logits", C.POINTER(f32), [P]),
    ("chk_last_logits_row", u32, [P]),
    ("chk_mtp_logits_row", C.POINTER(f32), [P, u32]),
    ("chk_pos", u32, [P]),
    ("chk_eos_token", u32, [P]),
    ("chk_vocab_size", u32, [P]),
    ("chk_max_t", u32, [P]),
    ("chk_trunk_rows", u32, [P]),
    ("chk_has_mtp", i32, [P]),
    ("chk_memory_stats", i32, [P, C.POINTER(ChkMemoryStats)]),
    ("chk_allocated_gb", f64, [P]),
    ("chk_kv_cache_bytes", u64, [P]),
    ("chk_kv_cache_capacity", u64, [P]),
    ("chk_kv_cache_fullness", f64, [P]),
    ("chk_context_fullness", f64, [P]),
    ("chk_reset_request", i32, [P]),
    ("chk_clear_profile", i32, [P]),
    ("chk_prefix_state_bytes", u64, [P]),
    ("chk_state_bytes_at", u64, [P, u32, u32]),
    ("chk_save_prefix", i32, [P, C.POINTER(P)]),
    ("chk_save_into", i32, [P, C.POINTER(P)]),
    ("chk_restore_prefix", i32, [P, P]),
    ("chk_prefix_free", None, [P]),
    ("chk_prefix_pos", u32, [P]),
    ("chk_prefix_mtp_len", u32, [P]),
    ("chk_prefix_tokens", u32, [P, C.POINTER(u32), u32]),
    ("chk_pool_slots", u32, [P]),
    ("chk_pool_budget", u32, [P]),
    ("chk_pool_resident", u32, [P]),
    ("chk_pool_is_member", i32, [P, u32]),
    ("chk_pool_acquire", i32, [P, C.POINTER(u32), u32, u64, C.POINTER(u32), C.POINTER(u32)]),
    ("chk_pool_plan_reads", i32, [P, C.POINTER(u32), u32, C.POINTER(u32), C.POINTER(u32)]),
    ("chk_pool_finish", i32, [P, C.POINTER(u32), u32]),
    ("chk_pool_addr", u64, [P, u32]),
    ("chk_pool_buf", i32, [P, u32, C.POINTER(P), C.POINTER(u64)]),
    ("chk_pool_kind", u32, [P, u32]),
    ("chk_pool_set_kind", i32, [P, u32, u32]),
    ("chk_pool_store", i32, [P, u32, C.POINTER(P), C.POINTER(u64)]),
    ("chk_pool_bytes", u64, [P]),
    ("chk_throttle_ms", i32, [P, C.POINTER(f64)]),
    ("chk_working_set_limit_gb", f64, [P]),
    ("chk_expert_activity", i32, [P, C.POINTER(ChkExpertCounters), u32, C.POINTER(f64)]),
    ("chk_last_routes", i32, [P, u32, u32, C.POINTER(u32), C.POINTER(f32)]),
    ("chk_last_probs", i32, [P, u32, u32, P]),
    # kernels.h
    ("chk_q4_matvec", i32, [P, P, P, u32, u32, P, P, u32, P]),
    ("chk_q4_gemm", i32, [P, P, P, u32, u32, P, u32, P, P]),
    ("chk_lm_head_argmax", i32, [P, P, P, u32, u32, P, u32, P, P, P]),
    ("chk_lm_head_argmax_noalloc", i32, [P, P, P, u32, u32, P, u32, P, P, P]),
    ("chk_attn_decode_q8", i32, [P, P, P, P, P, u32, u32, u32, u32, P, P]),
    ("chk_qsa_select", i32, [P, u32, u32, u32, P, P]),
    ("chk_dn_scan", i32, [P, P, P, P, P, u32, u32, u32, u32, u32, i32, P]),
    ("chk_moe_block", i32, [P, u32, P, u32, P, P, P, P]),
    ("chk_deltanet_block", i32, [P, u32, P, u32, i32, P]),
    ("chk_deltanet_state", i32, [P, u32, P, P]),
    ("chk_deltanet_rollback", i32, [P, u32, u32]),
    ("chk_attention_block", i32, [P, u32, P, u32, u32, P]),
    ("chk_kv_fill", i32, [P, u32, u32, P, P, u32]),
    ("chk_attention_block2", i32, [P, u32, P, C.POINTER(u32), P]),
    ("chk_hc_read", i32, [P, u32, u32, P, u32, P, P]),
    ("chk_expert_record", i32, [P, u32, u32, u32, P, u64]),
    ("chk_record_stride", u64, [P, u32]),
    ("chk_trace_enable", i32, [P, i32]),
    ("chk_layer_hyper", i32, [P, u32, u32, P]),
    ("chk_profile_kernel", i32, [P, i32]),
    ("chk_profile_read", i32, [P, C.POINTER(f64), C.POINTER(u64), C.POINTER(u64)]),
    ("chk_prefix_regions", i32, [P, u32, u32, C.POINTER(u64), C.POINTER(u64), u32, C.POINTER(u32)]),
    ("chk_prefix_read", i32, [P, u32, P, u64]),
    ("chk_fill_u8", i32, [P, u32, u64, P]),
    ("chk_copy_f32", i32, [P, P, u64, P]),
    ("chk_pf_flash_plan", i32, [u32, u32, u32, C.POINTER(u32), C.POINTER(u32), P, u64, P, u64, C.POINTER(u32)]),
    ("chk_profile_graph", i32, [P, i32, u32, C.POINTER(C.c_double), C.POINTER(u64), C.POINTER(u64)]),
    ("chk_time_decode", i32, [P, u32, u32, C.POINTER(f32), C.POINTER(u32)]),
    ("chk_time_blocks", i32, [P, C.c_int, u32, C.POINTER(u32), u32, P, u32, C.POINTER(u32), u32, C.POINTER(f32)]),
    ("chk_phase_bench", i32, [i32, u32, u32, u64, C.POINTER(f64), C.POINTER(u32)]),
    # sampling
    ("chk_sampling_validate", i32, [C.POINTER(ChkSampling)]),
    ("chk_sampling_greedy", i32, [C.POINTER(ChkSampling)]),
    ("chk_sampler_new", i32, [C.POINTER(ChkSampling), C.POINTER(u32), u32, u32, C.POINTER(P)]),
    ("chk_sampler_free", None, [P]),
    ("chk_sampler_accept", i32, [P, u32]),
    ("chk_sampler_sample", i32, [P, C.POINTER(f32), u32, C.POINTER(u32)]),
    ("chk_rng_u64", i32, [C.c_char_p, u64, C.POINTER(u64), u32]),
    ("chk_pcg32", None, [u64, u64, C.POINTER(u32), u32]),
    ("chk_chacha_block", None, [C.POINTER(u32), i32, C.POINTER(u32)]),
    # prefix cache
    ("chk_prefix_matches", i32, [C.POINTER(u32), u32, i32, u32, i32, C.POINTER(u32), u32]),
    ("chk_prefill_chunk_len", i32, [u32, u32, u32, C.POINTER(u32)]),
    ("chk_prefill_pacing_sample", i32, [u32, u32, u32, i32]),
    ("chk_prefix_cache_new", i32, [u64, u64, u64, C.POINTER(P)]),
    ("chk_prefix_cache_free", None, [P]),
    ("chk_prefix_cache_expire", None, [P]),
    ("chk_prefix_cache_stats", None, [P, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
    ("chk_prefix_cache_begin", i32, [P, P, C.POINTER(u32), u32, C.POINTER(u32), u32, u32, C.POINTER(P)]),
    ("chk_prefill_free", None, [P]),
    ("chk_prefill_cached", u32, [P]),
    ("chk_prefill_advance", i32, [P, P, P, C.POINTER(u32), u32, u32, u32, C.POINTER(i32), C.POINTER(u32)]),
    ("chk_prefill_next", u32, [P]),
    ("chk_prefill_drafts", u32, [P, C.POINTER(u32), u32]),
    ("chk_prefill_logits", C.POINTER(f32), [P]),
    # runner (decode loop)
    ("chk_decode_new", i32, [P, u32, C.POINTER(u32), u32, u32, u32, u32, C.POINTER(P)]),
    ("chk_decode_new_sampling", i32, [P, C.POINTER(ChkSampling), C.POINTER(u32), u32, C.POINTER(f32), u32,
                                      C.POINTER(u32), u32, u32, u32, u32, C.POINTER(P)]),
    ("chk_decode_free", None, [P]),
    ("chk_decode_set_eos", i32, [P, C.POINTER(u32), u32]),
    ("chk_decode_step", i32, [P, C.POINTER(u32), C.POINTER(u32)]),
    ("chk_decode_finished", i32, [P]),
    ("chk_decode_stats", i32, [P, C.POINTER(u32), C.POINTER(u32)]),
    ("chk_decode_error", C.c_char_p, []),
]

_lib = None


class EngineError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load libcherenkov.so (built by cherenkov_amd.build); raise if absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise EngineError(
                f"{LIB_PATH} is missing: build it with `python -m cherenkov_amd.build` "
                "(there is no CPU fallback)"
            )
        L = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | C.RTLD_GLOBAL)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise EngineError(lib().chk_last_error().decode())
