"""Python handle over the native engine (libcherenkov.so).

Method names follow the reference's `Gpu` API (src/qwen4_exp/gpu.rs and
gpu/*.rs): load, step_rows, step, commit, reset, mtp_draft, mtp_chain,
prefill_chunk, logits_row, ...; errors raise EngineError with the engine's
message (the reference's anyhow::Result).  Every call goes to the HIP
library; nothing here computes model math.
"""

from __future__ import annotations

import ctypes as C
from typing import Iterable, Sequence

import numpy as np

from .abi import NO_TOKEN, ChkConfig, ChkMemoryStats, ChkOptions, EngineError, check, lib

U32P = C.POINTER(C.c_uint32)


def _u32(arr: Sequence[int]):
    a = (C.c_uint32 * max(len(arr), 1))(*arr)
    return a


class Engine:
    def __init__(self, cfg: ChkConfig, experts: int = 4, drafts: int = 0, max_t: int = 2048, no_eos: bool = False):
        self.cfg = cfg
        self.opt = ChkOptions(experts, drafts, max_t, 1 if no_eos else 0)
        self._h = C.c_void_p()
        L = lib()
        check(L.chk_engine_load(C.byref(cfg), C.byref(self.opt), C.byref(self._h)))
        self.L = L

    @classmethod
    def load_bounded(cls, cfg: ChkConfig, reserve: int, memory_bytes: int, prefill_rows: int, experts: int = 4,
                     drafts: int = 0, max_t: int = 2048, no_eos: bool = False) -> "Engine":
        """Gpu::load_bounded: the engine under a server memory budget of
        memory_bytes - reserve (chk_engine_load_bounded)."""
        self = cls.__new__(cls)
        self.cfg = cfg
        self.opt = ChkOptions(experts, drafts, max_t, 1 if no_eos else 0)
        self._h = C.c_void_p()
        L = lib()
        check(L.chk_engine_load_bounded(C.byref(cfg), C.byref(self.opt), reserve, memory_bytes, prefill_rows,
                                        C.byref(self._h)))
        self.L = L
        return self

    @classmethod
    def load_store(cls, path, experts: int = 4, drafts: int = 0, max_t: int = 2048,
                   no_eos: bool = False) -> "Engine":
        """Gpu::load over a packed store directory (chk_engine_load_store)."""
        self = cls.__new__(cls)
        self.opt = ChkOptions(experts, drafts, max_t, 1 if no_eos else 0)
        self._h = C.c_void_p()
        L = lib()
        check(L.chk_engine_load_store(str(path).encode(), C.byref(self.opt), C.byref(self._h)))
        self.cfg = store_config(path)
        self.L = L
        return self

    def close(self) -> None:
        if self._h:
            self.L.chk_engine_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    # ---- Gpu API ----
    def step_rows(self, tokens: Sequence[int], snap: bool = False, fold_mtp: bool = False) -> list[int]:
        n = len(tokens)
        out = (C.c_uint32 * max(n, 1))()
        check(self.L.chk_step_rows(self._h, _u32(tokens), n, int(snap), int(fold_mtp), out))
        return list(out[:n])

    def step(self, token: int) -> int:
        out = C.c_uint32()
        check(self.L.chk_step(self._h, token, C.byref(out)))
        return out.value

    def commit(self, n: int) -> None:
        check(self.L.chk_commit(self._h, n))

    def reset(self) -> None:
        check(self.L.chk_reset(self._h))

    def mtp_draft(self, nxt: Sequence[int], chain: int) -> list[int]:
        d = (C.c_uint32 * 4)()
        nd = C.c_uint32()
        check(self.L.chk_mtp_draft(self._h, _u32(nxt), len(nxt), chain, d, C.byref(nd)))
        return list(d[: nd.value])

    def mtp_chain(self, draft: int) -> int:
        out = C.c_uint32()
        check(self.L.chk_mtp_chain(self._h, draft, C.byref(out)))
        return out.value

    def prefill_chunk(self, tokens: Sequence[int], next_after: int | None = None,
                      all_logits: bool = False) -> tuple[int, int | None]:
        """Gpu::prefill_chunk(tokens, next_after, all_logits) -> (next, draft)."""
        nxt, dr = C.c_uint32(), C.c_uint32()
        na = NO_TOKEN if next_after is None else int(next_after)
        check(self.L.chk_prefill_chunk(self._h, _u32(tokens), len(tokens), na, int(all_logits), C.byref(nxt),
                                       C.byref(dr)))
        return nxt.value, (None if dr.value == NO_TOKEN else dr.value)

    def prefill_release(self) -> None:
        self.L.chk_prefill_release(self._h)

    def _ids(self, fn, r: int) -> list[int]:
        n = C.c_uint32()
        check(fn(self._h, r, None, 0, C.byref(n)))
        out = (C.c_uint32 * max(1, n.value))()
        check(fn(self._h, r, out, n.value, C.byref(n)))
        return list(out[: n.value])

    def debug_engine_blocks(self, r: int) -> list[int]:
        """Gpu::debug_engine_blocks: QSA blocks selected for row r of the last
        prefill chunk (its latest attention layer)."""
        return self._ids(self.L.chk_debug_engine_blocks, r)

    def debug_row_vis(self, r: int) -> list[int]:
        """Gpu::debug_row_vis: tokens row r of the last row step attended to
        (its latest attention layer)."""
        return self._ids(self.L.chk_debug_row_vis, r)

    def prefill_rows_fit(self, all_logits: bool = False) -> int:
        r = C.c_uint32()
        check(self.L.chk_prefill_rows_fit(self._h, int(all_logits), C.byref(r)))
        return r.value

    def pf_logits_row(self, r: int) -> np.ndarray:
        return self._vocab_row(self.L.chk_pf_logits_row(self._h, r))

    def _vocab_row(self, p) -> np.ndarray:
        if not p:
            raise EngineError(self.L.chk_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

    def logits_row(self, r: int) -> np.ndarray:
        return self._vocab_row(self.L.chk_logits_row(self._h, r))

    def logits(self) -> np.ndarray:
        return self._vocab_row(self.L.chk_logits(self._h))

    def last_logits_row(self) -> int:
        return self.L.chk_last_logits_row(self._h)

    def mtp_logits_row(self, r: int) -> np.ndarray:
        p = self.L.chk_mtp_logits_row(self._h, r)
        if not p:
            raise EngineError(self.L.chk_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

    def throttle_ms(self) -> float:
        ms = C.c_double()
        check(self.L.chk_throttle_ms(self._h, C.byref(ms)))
        return ms.value

    def working_set_limit_gb(self) -> float:
        return self.L.chk_working_set_limit_gb(self._h)

    def expert_activity(self) -> tuple[np.ndarray, float]:
        """Gpu::expert_activity: (counters [record layers][experts][6] as
        ChkExpertCounters fields, seconds since load)."""
        from .abi import ChkExpertCounters
        n = (self.cfg.num_hidden_layers + (1 if self.has_mtp else 0)) * self.cfg.num_experts
        buf = (ChkExpertCounters * n)()
        sec = C.c_double()
        check(self.L.chk_expert_activity(self._h, buf, n, C.byref(sec)))
        arr = np.frombuffer(buf, dtype=np.uint64).reshape(-1, self.cfg.num_experts, 6).copy()
        return arr, sec.value

    @property
    def pos(self) -> int:
        return self.L.chk_pos(self._h)

    @property
    def max_t(self) -> int:
        return self.L.chk_max_t(self._h)

    @property
    def trunk_rows(self) -> int:
        return self.L.chk_trunk_rows(self._h)

    @property
    def has_mtp(self) -> bool:
        return bool(self.L.chk_has_mtp(self._h))

    def allocated_gb(self) -> float:
        return self.L.chk_allocated_gb(self._h)

    def kv_cache_bytes(self) -> int:
        return self.L.chk_kv_cache_bytes(self._h)

    def kv_cache_capacity(self) -> int:
        return self.L.chk_kv_cache_capacity(self._h)

    def kv_cache_fullness(self) -> float:
        return self.L.chk_kv_cache_fullness(self._h)

    def context_fullness(self) -> float:
        return self.L.chk_context_fullness(self._h)

    def reset_request(self) -> None:
        check(self.L.chk_reset_request(self._h))

    def clear_profile(self) -> None:
        check(self.L.chk_clear_profile(self._h))

    # ---- sequence checkpoints (gpu/state.rs:85-230) ----
    def prefix_state_bytes(self) -> int:
        return self.L.chk_prefix_state_bytes(self._h)

    def state_bytes_at(self, pos: int, mtp_len: int) -> int:
        return self.L.chk_state_bytes_at(self._h, pos, mtp_len)

    def save_prefix(self) -> "PrefixState":
        h = C.c_void_p()
        check(self.L.chk_save_prefix(self._h, C.byref(h)))
        return PrefixState(self, h)

    def save_into(self, checkpoint: "PrefixState | None") -> "PrefixState":
        if checkpoint is None:
            return self.save_prefix()
        check(self.L.chk_save_into(self._h, C.byref(checkpoint._h)))
        return checkpoint

    def restore_prefix(self, state: "PrefixState") -> None:
        check(self.L.chk_restore_prefix(self._h, state._h))

    def prefix_regions(self, pos: int, mtp_len: int) -> list[tuple[int, int]]:
        n = C.c_uint32()
        check(self.L.chk_prefix_regions(self._h, pos, mtp_len, None, None, 0, C.byref(n)))
        ptrs = (C.c_uint64 * max(n.value, 1))()
        lens = (C.c_uint64 * max(n.value, 1))()
        check(self.L.chk_prefix_regions(self._h, pos, mtp_len, ptrs, lens, n.value, C.byref(n)))
        return [(ptrs[i], lens[i]) for i in range(n.value)]

    # ---- expert-cache interface (residency::Pool) ----
    def pool_acquire(self, rids: Sequence[int], step: int) -> list[int]:
        need = (C.c_uint32 * max(len(rids), 1))()
        nn = C.c_uint32()
        check(self.L.chk_pool_acquire(self._h, _u32(rids), len(rids), step, need, C.byref(nn)))
        return list(need[: nn.value])

    def pool_plan_reads(self, need: Sequence[int]) -> tuple[int, int]:
        nr, warm = C.c_uint32(), C.c_uint32()
        check(self.L.chk_pool_plan_reads(self._h, _u32(need), len(need), C.byref(nr), C.byref(warm)))
        return nr.value, warm.value

    def pool_finish(self, rids: Sequence[int]) -> None:
        check(self.L.chk_pool_finish(self._h, _u32(rids), len(rids)))

    def pool_addr(self, rid: int) -> int:
        return self.L.chk_pool_addr(self._h, rid)

    def pool_buf(self, rid: int) -> tuple[int, int]:
        base, off = C.c_void_p(), C.c_uint64()
        check(self.L.chk_pool_buf(self._h, rid, C.byref(base), C.byref(off)))
        return base.value or 0, off.value

    def pool_kind(self, rid: int) -> int:
        return self.L.chk_pool_kind(self._h, rid)

    def pool_set_kind(self, rid: int, kind: int) -> None:
        check(self.L.chk_pool_set_kind(self._h, rid, kind))

    def pool_store(self, kind: int) -> tuple[int, int]:
        base, stride = C.c_void_p(), C.c_uint64()
        check(self.L.chk_pool_store(self._h, kind, C.byref(base), C.byref(stride)))
        return base.value or 0, stride.value

    def memory_stats(self) -> dict:
        m = ChkMemoryStats()
        check(self.L.chk_memory_stats(self._h, C.byref(m)))
        return {k: getattr(m, k) for k, _ in m._fields_}

    def last_routes(self, layer: int, row: int) -> tuple[list[int], list[float]]:
        k = self.cfg.num_experts_per_tok
        ids = (C.c_uint32 * k)()
        w = (C.c_float * k)()
        check(self.L.chk_last_routes(self._h, layer, row, ids, w))
        return list(ids), list(w)

    def last_probs(self, layer: int, row: int) -> np.ndarray:
        p = np.empty(self.cfg.num_experts, np.float32)
        check(self.L.chk_last_probs(self._h, layer, row, p.ctypes.data))
        return p

    # ---- tracing / kernel-level helpers ----
    def trace(self, on: bool = True) -> None:
        check(self.L.chk_trace_enable(self._h, int(on)))

    def layer_hyper(self, layer: int, row: int) -> np.ndarray:
        out = np.empty(self.cfg.hidden_size * self.cfg.hc_count, dtype=np.float32)
        check(self.L.chk_layer_hyper(self._h, layer, row, out.ctypes.data))
        return out

    def expert_record(self, layer: int, expert: int, bits: int = 4) -> np.ndarray:
        n = self.L.chk_record_stride(self._h, bits)
        if n == 0:
            raise EngineError(f"no {bits}-bit store")
        out = np.empty(n, dtype=np.uint8)
        check(self.L.chk_expert_record(self._h, layer, expert, bits, out.ctypes.data, n))
        return out

    def profile_kernel(self, kind: int) -> None:
        check(self.L.chk_profile_kernel(self._h, kind))

    def profile_read(self) -> tuple[float, int, int]:
        ms, n, by = C.c_double(), C.c_uint64(), C.c_uint64()
        check(self.L.chk_profile_read(self._h, C.byref(ms), C.byref(n), C.byref(by)))
        return ms.value, n.value, by.value

    def profile_graph(self, kind: int, reps: int) -> tuple[float, int, int]:
        """(ms, launches, algorithmic bytes) of a graph of `reps` rounds of
        one kernel class's per-layer launches (chk_profile_graph)."""
        ms, n, by = C.c_double(), C.c_uint64(), C.c_uint64()
        check(self.L.chk_profile_graph(self._h, kind, reps, C.byref(ms), C.byref(n), C.byref(by)))
        return ms.value, n.value, by.value

    def time_decode(self, first_token: int, steps: int) -> tuple[float, int]:
        ms, last = C.c_float(), C.c_uint32()
        check(self.L.chk_time_decode(self._h, first_token, steps, C.byref(ms), C.byref(last)))
        return ms.value, last.value


def store_config(path) -> ChkConfig:
    """The ChkConfig of a packed store (chk_store_config: file reads only)."""
    cfg = ChkConfig()
    check(lib().chk_store_config(str(path).encode(), C.byref(cfg)))
    return cfg


class PrefixState:
    """A sequence checkpoint (Gpu's PrefixState) held by the engine library."""

    def __init__(self, eng: Engine, h: C.c_void_p):
        self.eng = eng
        self._h = h

    def throttle_ms(self) -> float:
        ms = C.c_double()
        check(self.L.chk_throttle_ms(self._h, C.byref(ms)))
        return ms.value

    def working_set_limit_gb(self) -> float:
        return self.L.chk_working_set_limit_gb(self._h)

    def expert_activity(self) -> tuple[np.ndarray, float]:
        """Gpu::expert_activity: (counters [record layers][experts][6] as
        ChkExpertCounters fields, seconds since load)."""
        from .abi import ChkExpertCounters
        n = (self.cfg.num_hidden_layers + (1 if self.has_mtp else 0)) * self.cfg.num_experts
        buf = (ChkExpertCounters * n)()
        sec = C.c_double()
        check(self.L.chk_expert_activity(self._h, buf, n, C.byref(sec)))
        arr = np.frombuffer(buf, dtype=np.uint64).reshape(-1, self.cfg.num_experts, 6).copy()
        return arr, sec.value

    @property
    def pos(self) -> int:
        return self.eng.L.chk_prefix_pos(self._h)

    @property
    def mtp_len(self) -> int:
        return self.eng.L.chk_prefix_mtp_len(self._h)

    @property
    def tokens(self) -> list[int]:
        n = self.eng.L.chk_prefix_tokens(self._h, None, 0)
        out = (C.c_uint32 * max(n, 1))()
        self.eng.L.chk_prefix_tokens(self._h, out, n)
        return list(out[:n])

    def region(self, i: int, n: int) -> np.ndarray:
        out = np.empty(n, np.uint8)
        check(self.eng.L.chk_prefix_read(self._h, i, out.ctypes.data, n))
        return out

    def free(self) -> None:
        if self._h:
            self.eng.L.chk_prefix_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Decode:
    """The runner's decode loop (native, runner.cpp; decode.rs:6-171).

    Greedy options (the default) verify MTP drafts against the trunk's
    argmax.  Other sampling options draw each token from the request's
    sampler: the first from `final_logits` (the prompt's last-row logits),
    the sampler's counts starting from `prompt`, and no drafts."""

    def __init__(self, eng: Engine, nxt: int, drafts: Iterable[int], n_draft: int, limit: int, no_eos: bool = True,
                 sampling=None, prompt: Sequence[int] = (), final_logits=None):
        self.eng = eng
        dl = list(drafts)
        self._h = C.c_void_p()
        if sampling is None:
            rc = eng.L.chk_decode_new(eng.handle, nxt, _u32(dl), len(dl), n_draft, limit, int(no_eos),
                                      C.byref(self._h))
        else:
            self._opts = sampling.native()
            fl = None
            if final_logits is not None:
                self._fl = np.ascontiguousarray(final_logits, dtype=np.float32)
                fl = self._fl.ctypes.data_as(C.POINTER(C.c_float))
            rc = eng.L.chk_decode_new_sampling(eng.handle, C.byref(self._opts), _u32(list(prompt)), len(prompt), fl,
                                               nxt, _u32(dl), len(dl), n_draft, limit, int(no_eos), C.byref(self._h))
        if rc != 0:
            raise EngineError(eng.L.chk_decode_error().decode())

    def set_eos(self, ids: Sequence[int]) -> None:
        """The stop ids (the tokenizer's [im_end, endoftext] in the
        reference); the config's eos_token_id alone until set."""
        ids = list(ids)
        if self.eng.L.chk_decode_set_eos(self._h, _u32(ids), len(ids)) != 0:
            raise EngineError(self.eng.L.chk_decode_error().decode())

    def step(self) -> list[int]:
        em = (C.c_uint32 * 4)()
        n = C.c_uint32()
        rc = self.eng.L.chk_decode_step(self._h, em, C.byref(n))
        if rc != 0:
            raise EngineError(self.eng.L.chk_decode_error().decode())
        return list(em[: n.value])

    @property
    def finished(self) -> int:
        return self.eng.L.chk_decode_finished(self._h)

    def stats(self) -> tuple[int, int]:
        s, a = C.c_uint32(), C.c_uint32()
        self.eng.L.chk_decode_stats(self._h, C.byref(s), C.byref(a))
        return s.value, a.value

    def run(self) -> list[int]:
        out: list[int] = []
        while not self.finished:
            out.extend(self.step())
        return out

    def __del__(self):
        try:
            if self._h:
                self.eng.L.chk_decode_free(self._h)
        except Exception:
            pass
