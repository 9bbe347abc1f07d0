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

from .abi import ChkConfig, ChkMemoryStats, ChkOptions, EngineError, check, lib

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

    def prefill_chunk(self, tokens: Sequence[int]) -> tuple[int, int | None]:
        nxt, dr = C.c_uint32(), C.c_uint32()
        check(self.L.chk_prefill_chunk(self._h, _u32(tokens), len(tokens), C.byref(nxt), C.byref(dr)))
        return nxt.value, (None if dr.value == 0xFFFFFFFF else dr.value)

    def logits_row(self, r: int) -> np.ndarray:
        p = self.L.chk_logits_row(self._h, r)
        if not p:
            raise EngineError(self.L.chk_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

    def mtp_logits_row(self, r: int) -> np.ndarray:
        p = self.L.chk_mtp_logits_row(self._h, r)
        if not p:
            raise EngineError(self.L.chk_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

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


class Decode:
    """The runner's greedy speculative decode loop (native, runner.cpp)."""

    def __init__(self, eng: Engine, nxt: int, drafts: Iterable[int], n_draft: int, limit: int, no_eos: bool = True):
        self.eng = eng
        dl = list(drafts)
        self._h = C.c_void_p()
        check(eng.L.chk_decode_new(eng.handle, nxt, _u32(dl), len(dl), n_draft, limit, int(no_eos), C.byref(self._h)))

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
