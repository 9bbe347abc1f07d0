"""Prefix cache and prompt cursor (reference: src/prefix_cache.rs:12-335)
over the native implementation (prefix_cache.cpp).

A `PrefixCache` keeps device checkpoints of prompt prefixes, least
recently used first out, within a byte capacity and an entry count; a
request's `begin` restores the longest prefix its prompt extends and
returns a `Prefill` cursor whose `advance` prefills one chunk at a time,
storing new entries at the prompt's stable boundaries.
"""

from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from .abi import EngineError, check, lib


def _u32(v: Sequence[int]):
    return (C.c_uint32 * max(len(v), 1))(*v)


def matches(tokens: Sequence[int], following: int | None, complete: bool, request: Sequence[int]) -> bool:
    """matches (prefix_cache.rs:35-45)."""
    return bool(lib().chk_prefix_matches(_u32(tokens), len(tokens), int(following is not None), following or 0,
                                         int(complete), _u32(request), len(request)))


def chunk_len(remaining: int, capacity: int, quantum: int) -> int:
    """chunk_len (prefix_cache.rs:256-266)."""
    out = C.c_uint32()
    check(lib().chk_prefill_chunk_len(remaining, capacity, quantum, C.byref(out)))
    return out.value


def pacing_sample(remaining: int, capacity: int, quantum: int, engine: bool) -> bool:
    """pacing_sample (prefix_cache.rs:251-253)."""
    return bool(lib().chk_prefill_pacing_sample(remaining, capacity, quantum, int(engine)))


class PrefixCache:
    """PrefixCache::new(capacity bytes, max entries, idle seconds)."""

    def __init__(self, capacity: int, max_entries: int = 64, idle_seconds: int = 0):
        self._h = C.c_void_p()
        check(lib().chk_prefix_cache_new(capacity, max_entries, idle_seconds, C.byref(self._h)))

    def stats(self) -> tuple[int, int, int]:
        """(entries, bytes used, evictions)."""
        n, u, e = C.c_uint64(), C.c_uint64(), C.c_uint64()
        lib().chk_prefix_cache_stats(self._h, C.byref(n), C.byref(u), C.byref(e))
        return n.value, u.value, e.value

    def expire(self) -> None:
        lib().chk_prefix_cache_expire(self._h)

    def begin(self, eng, ids: Sequence[int], stable_boundaries: Sequence[int] = (), drafts: int = 0) -> "Prefill":
        h = C.c_void_p()
        check(lib().chk_prefix_cache_begin(self._h, eng.handle, _u32(ids), len(ids), _u32(stable_boundaries),
                                           len(stable_boundaries), drafts, C.byref(h)))
        return Prefill(self, eng, list(ids), drafts, h)

    def __del__(self):
        try:
            if self._h:
                lib().chk_prefix_cache_free(self._h)
        except Exception:
            pass


class Prefill:
    """The prompt cursor (Prefill, prefix_cache.rs:183-249)."""

    def __init__(self, cache: PrefixCache, eng, ids: list[int], drafts: int, h):
        self.cache, self.eng, self.ids, self.drafts = cache, eng, ids, drafts
        self._ids = _u32(ids)
        self._h = h

    @property
    def cached(self) -> int:
        return lib().chk_prefill_cached(self._h)

    def advance(self, quantum: int = 4096) -> tuple[bool, int | None]:
        """One chunk: (done, pacing tokens or None)."""
        done, pacing = C.c_int(), C.c_uint32()
        check(lib().chk_prefill_advance(self._h, self.cache._h, self.eng.handle, self._ids, len(self.ids),
                                        self.drafts, quantum, C.byref(done), C.byref(pacing)))
        return bool(done.value), (pacing.value or None)

    def run(self, quantum: int = 4096) -> None:
        while not self.advance(quantum)[0]:
            pass

    def resume(self) -> tuple[int, list[int], np.ndarray | None]:
        """(next token, drafts, last-row logits) to start decode from."""
        L = lib()
        out = (C.c_uint32 * 8)()
        n = L.chk_prefill_drafts(self._h, out, 8)
        p = L.chk_prefill_logits(self._h)
        logits = np.ctypeslib.as_array(p, shape=(self.eng.cfg.vocab_size,)).copy() if p else None
        return L.chk_prefill_next(self._h), list(out[:n]), logits

    def __del__(self):
        try:
            if self._h:
                lib().chk_prefill_free(self._h)
        except Exception:
            pass


__all__ = ["PrefixCache", "Prefill", "matches", "chunk_len", "pacing_sample", "EngineError"]
