"""The prefix cache on the GPU (PrefixCache / Prefill, src/prefix_cache.rs:
12-335, native prefix_cache.cpp): a request that extends a cached prefix
restores it and prefills only the rest, and decodes as a request prefilled
from scratch; an entry made while drafting serves only the continuation
its MTP row was paired with; a complete entry serves an identical prompt
without prefill; the byte capacity evicts oldest first."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Decode, Engine
from cherenkov_amd.prefix_cache import PrefixCache
from tests.gpu_util import argmax_margin, assert_close

pytestmark = pytest.mark.gpu


def decode(eng, pf, drafts, n=12):
    nxt, dr, _ = pf.resume()
    return Decode(eng, nxt, dr, drafts, limit=n, no_eos=True).run()


@pytest.mark.parametrize("drafts", [0, 2])
def test_extending_a_cached_prefix_decodes_as_from_scratch(have_gpu, drafts):
    cfg = presets.tiny(mtp=1 if drafts else 0)
    rng = np.random.default_rng(80 + drafts)
    a = rng.integers(0, cfg.vocab_size, size=100).tolist()
    # b continues with a[64] at position 64: an entry made while drafting
    # pins the token after its prefix
    b = a[:65] + rng.integers(0, cfg.vocab_size, size=39).tolist()
    eng = Engine(cfg, experts=4, drafts=drafts, max_t=256)
    ref = Engine(cfg, experts=4, drafts=drafts, max_t=256)
    cache = PrefixCache(1 << 30)
    try:
        pf = cache.begin(eng, a, stable_boundaries=[64], drafts=drafts)
        assert pf.cached == 0
        pf.run(quantum=4096)
        assert eng.pos == 100
        n_entries = cache.stats()[0]
        assert n_entries >= 2  # the stable boundary and the prompt's last rows
        eng.reset_request()
        pf = cache.begin(eng, b, stable_boundaries=[64], drafts=drafts)
        assert pf.cached == 64 and eng.pos == 64
        pf.run()
        got_logits = pf.resume()[2]
        got = decode(eng, pf, drafts)
        pr = PrefixCache(0).begin(ref, b, drafts=drafts)
        pr.run()
        want_logits = pr.resume()[2]
        want = decode(ref, pr, drafts)
        # different chunkings (a restore at 64 then row steps, against one
        # 104-row GEMM chunk): the same model at float-reordering distance
        assert_close(got_logits, want_logits, "resume logits", abs_frac=2e-3, min_cos=0.9999)
        if argmax_margin(want_logits) > 1e-3:
            assert got == want
    finally:
        eng.close()
        ref.close()


def test_drafting_entry_serves_only_its_continuation(have_gpu):
    cfg = presets.tiny(mtp=1)
    rng = np.random.default_rng(82)
    a = rng.integers(0, cfg.vocab_size, size=80).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=256)
    cache = PrefixCache(1 << 30)
    try:
        pf = cache.begin(eng, a, stable_boundaries=[48], drafts=2)
        pf.run()
        eng.reset_request()
        same = a[:48] + [a[48]] + [1, 2, 3]
        assert cache.begin(eng, same, stable_boundaries=[48], drafts=2).cached == 48
        eng.reset_request()
        other = a[:48] + [(a[48] + 1) % cfg.vocab_size] + [1, 2, 3]
        assert cache.begin(eng, other, stable_boundaries=[48], drafts=2).cached == 0
        eng.reset_request()
        # entries of one drafting mode never serve the other
        assert cache.begin(eng, same, stable_boundaries=[48], drafts=0).cached == 0
    finally:
        eng.close()


def test_complete_entry_resumes_without_prefill(have_gpu):
    cfg = presets.tiny(mtp=0)
    prompt = np.random.default_rng(83).integers(0, cfg.vocab_size, size=70).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=256)
    cache = PrefixCache(1 << 30)
    try:
        pf = cache.begin(eng, prompt, drafts=0)
        pf.run()
        first = pf.resume()
        eng.reset_request()
        pf = cache.begin(eng, prompt, drafts=0)
        assert pf.cached == 70 and eng.pos == 70
        assert pf.advance()[0]  # nothing left to prefill
        again = pf.resume()
        assert again[0] == first[0]
        np.testing.assert_array_equal(again[2], first[2])
    finally:
        eng.close()


def test_capacity_evicts_oldest_first(have_gpu):
    cfg = presets.tiny(mtp=0)
    rng = np.random.default_rng(84)
    eng = Engine(cfg, experts=4, drafts=0, max_t=256)
    try:
        eng.prefill_chunk(list(range(40)))
        one = eng.prefix_state_bytes() + 40 * 4 + cfg.vocab_size * 4 + 4096
        eng.reset_request()
        cache = PrefixCache(2 * one, max_entries=8)
        prompts = [rng.integers(0, cfg.vocab_size, size=40).tolist() for _ in range(3)]
        for p in prompts:
            cache.begin(eng, p, drafts=0).run()
            eng.reset_request()
        n, used, ev = cache.stats()
        assert n <= 2 and used <= 2 * one and ev >= 1
        assert cache.begin(eng, prompts[0], drafts=0).cached == 0
        eng.reset_request()
        assert cache.begin(eng, prompts[2], drafts=0).cached == 40
    finally:
        eng.close()
