"""GPU tests of sequence checkpoints and request switching
(gpu/state.rs:85-263; the server worker's activate, server/worker.rs:308-332):
the byte-pattern round trip of every prefix region
(tests/unit/qwen4_exp/gpu/state.rs:3-50), and two interleaved requests,
each decoding exactly as it would alone."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import EngineError, check, lib
from cherenkov_amd.engine import Engine
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu


def fill(ptr: int, value: int, n: int) -> None:
    check(lib().chk_fill_u8(ptr, value, n, None))


@pytest.mark.parametrize("drafts", [0, 2])
def test_prefix_checkpoint_restores_all_hybrid_regions(have_gpu, drafts):
    """Every region (DeltaNet state and conv history, q8 K/V and their
    scales, index keys, the MTP layer's cache) at pos 9 (an incomplete QSA
    block) is written with its index's byte pattern, saved, overwritten,
    the request reset, and the checkpoint restored: positions, tokens and
    every region come back byte for byte."""
    cfg = presets.tiny(mtp=1 if drafts else 0)
    eng = Engine(cfg, experts=4, drafts=drafts, max_t=64)
    try:
        prompt = list(range(9))
        eng.prefill_chunk(prompt)
        assert eng.pos == 9
        mtp_len = 9 if drafts else 0
        regs = eng.prefix_regions(9, mtp_len)
        n_dn = sum(1 for l in range(cfg.num_hidden_layers) if (l + 1) % cfg.full_attention_interval)
        n_at = cfg.num_hidden_layers - n_dn + (1 if drafts else 0)
        assert len(regs) == 2 * n_dn + 5 * n_at
        for i, (p, n) in enumerate(regs):
            fill(p, i % 251, n)
        cp = eng.save_prefix()
        assert (cp.pos, cp.mtp_len, cp.tokens) == (9, mtp_len, prompt)
        expect = eng.state_bytes_at(9, mtp_len)
        assert eng.prefix_state_bytes() == expect
        assert expect >= sum(n for _, n in regs) + 9 * 4
        for p, n in regs:
            fill(p, 255, n)
        eng.reset_request()
        assert eng.pos == 0
        eng.restore_prefix(cp)
        assert eng.pos == 9
        again = eng.save_prefix()
        assert again.tokens == prompt and again.mtp_len == mtp_len
        for i, (_, n) in enumerate(regs):
            got = again.region(i, n)
            assert np.all(got == i % 251), f"region {i}"
            np.testing.assert_array_equal(got, cp.region(i, n))
        # save_into reuses the checkpoint (and grows it) at a longer prefix
        eng.prefill_chunk([11, 12, 13])
        cp2 = eng.save_into(cp)
        assert cp2 is cp and cp.pos == 12 and cp.tokens == prompt + [11, 12, 13]
    finally:
        eng.close()


def test_restore_rejects_a_foreign_layout(have_gpu):
    small = Engine(presets.tiny(mtp=0), experts=4, drafts=0, max_t=32)
    other = Engine(presets.tiny(mtp=0, layers=8), experts=4, drafts=0, max_t=32)
    try:
        small.prefill_chunk([1, 2, 3])
        cp = small.save_prefix()
        with pytest.raises(EngineError, match="layout mismatch"):
            other.restore_prefix(cp)
    finally:
        small.close()
        other.close()


def greedy(eng: Engine, tok: int, n: int) -> tuple[list[int], list[np.ndarray]]:
    toks, logs = [], []
    for _ in range(n):
        out = eng.step_rows([tok])
        logs.append(eng.logits_row(0))
        eng.commit(1)
        toks.append(tok)
        tok = out[0]
    return toks + [tok], logs


def test_interleaved_requests_decode_as_alone(have_gpu):
    """Two requests share one engine the way the server worker switches
    them (save_into the previous request, reset_request, restore_prefix the
    next): each request's greedy tokens and logits equal its run alone."""
    cfg = presets.tiny(mtp=1)
    rng = np.random.default_rng(700)
    pa = rng.integers(0, cfg.vocab_size, size=20).tolist()
    pb = rng.integers(0, cfg.vocab_size, size=13).tolist()
    alone = {}
    for name, prompt in (("a", pa), ("b", pb)):
        e = Engine(cfg, experts=4, drafts=2, max_t=128)
        try:
            nxt, _ = e.prefill_chunk(prompt)
            alone[name] = greedy(e, nxt, 8)
        finally:
            e.close()
    eng = Engine(cfg, experts=4, drafts=2, max_t=128)
    try:
        cps = {"a": None, "b": None}
        state = {}
        # A: prefill and 3 tokens
        nxt_a, _ = eng.prefill_chunk(pa)
        ta, la = greedy(eng, nxt_a, 3)
        cps["a"] = eng.save_into(cps["a"])
        # switch to B: prefill and 5 tokens
        eng.reset_request()
        nxt_b, _ = eng.prefill_chunk(pb)
        tb, lb = greedy(eng, nxt_b, 5)
        cps["b"] = eng.save_into(cps["b"])
        # back to A for 5 more
        eng.reset_request()
        eng.restore_prefix(cps["a"])
        ta2, la2 = greedy(eng, ta[-1], 5)
        cps["a"] = eng.save_into(cps["a"])
        # and B for 3 more
        eng.reset_request()
        eng.restore_prefix(cps["b"])
        tb2, lb2 = greedy(eng, tb[-1], 3)
        state["a"] = (ta[:-1] + ta2, la + la2)
        state["b"] = (tb[:-1] + tb2, lb + lb2)
        for name in ("a", "b"):
            toks, logs = state[name]
            ref_toks, ref_logs = alone[name]
            assert toks == ref_toks, f"request {name}: {toks} vs {ref_toks}"
            for i, (g, r) in enumerate(zip(logs, ref_logs)):
                assert_close(g, r, f"request {name} step {i}", abs_frac=1e-6, min_cos=0.9999999)
    finally:
        eng.close()
