"""End-to-end GPU parity of the token loop against the CPU oracle
(forward_token / mtp_forward of /root/reference/src/qwen4_exp/cpu.rs,
restated in oracle/oracle.cpp with the engine's q8 KV rule).

Bars (north star): greedy token ids exact wherever the logit margin
exceeds 1e-3; logits within max-abs 2e-2 * max(1, max|ref|) and cosine
>= 0.999 per position.
"""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Decode, Engine
from oracle.oracle import OracleModel
from tests.gpu_util import ROUTE_TIE_TOL, argmax_margin, assert_close, engine_routes

pytestmark = pytest.mark.gpu


def check_logits(got, ref, label):
    assert_close(got, ref, label)
    m = argmax_margin(ref)
    if m > 1e-3:
        assert int(np.argmax(got)) == int(np.argmax(ref)), f"{label}: argmax {np.argmax(got)} vs {np.argmax(ref)}"
        return 0
    return 1


def teacher_forced(cfg, eng_tokens, prompt, step_logits, label, kv_q8=True):
    """Run the oracle over prompt + generated tokens, comparing each
    position's logits with the engine's.  Entries are (pos, logits) or
    (pos, logits, engine routes [layers][k]); with routes the oracle
    follows the engine through router near-ties (ROUTE_TIE_TOL), at most
    two layers per position."""
    orc = OracleModel(cfg)
    st = orc.new_state()
    seq = list(prompt) + list(eng_tokens)
    exempt = 0
    for i, (pos, logits, *routes) in enumerate(step_logits):
        while st.pos < pos:
            st.forward_token(seq[st.pos], kv_q8)
        if routes:
            st.route_hints(routes[0], ROUTE_TIE_TOL)
        ref = st.forward_token(seq[pos], kv_q8)
        exempt += check_logits(logits, ref, f"{label} pos {pos}")
    assert st.route_swaps <= 2 * len(step_logits), f"{label}: {st.route_swaps} near-tie routes followed"
    return exempt


def test_tiny_prompt_and_greedy_decode(have_gpu):
    """Config 1: 32-token seeded prompt + 64 greedy tokens on the tiny model."""
    cfg = presets.tiny()
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, cfg.vocab_size, size=32).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=256)
    try:
        # prompt row by row, keeping every row's logits
        logs = []
        for p, t in enumerate(prompt):
            out = eng.step_rows([t])
            logs.append((p, eng.logits_row(0)))
            eng.commit(1)
        nxt = out[0]
        gen = []
        tok = nxt
        for i in range(64):
            gen.append(tok)
            out = eng.step_rows([tok])
            logs.append((len(prompt) + i, eng.logits_row(0)))
            eng.commit(1)
            tok = out[0]
        exempt = teacher_forced(cfg, gen, prompt, logs, "tiny")
        assert exempt <= 2
    finally:
        eng.close()


def test_tiny_verify_rows_match_single_rows(have_gpu):
    """A 3-row verify step gives each row the logits of stepping it alone,
    and commit(n) rolls DeltaNet state back to row n-1 (gpu/state.rs:10-56)."""
    cfg = presets.tiny()
    rng = np.random.default_rng(2)
    toks = rng.integers(0, cfg.vocab_size, size=12).tolist()
    a = Engine(cfg, experts=4, drafts=3, max_t=128)
    b = Engine(cfg, experts=4, drafts=3, max_t=128)
    try:
        for t in toks[:5]:
            a.step(t)
            b.step(t)
        rows = toks[5:8]
        res = a.step_rows(rows, snap=True)
        la = [a.logits_row(r) for r in range(3)]
        for r, t in enumerate(rows):
            o = b.step_rows([t])
            assert o[0] == res[r]
            np.testing.assert_allclose(b.logits_row(0), la[r], rtol=1e-5, atol=1e-4)
            b.commit(1)
        # keep only the first row of the verify batch, then continue both
        a.commit(1)
        b2 = Engine(cfg, experts=4, drafts=3, max_t=128)
        try:
            for t in toks[:6]:
                b2.step(t)
            for t in toks[8:12]:
                oa = a.step(t)
                ob = b2.step(t)
                assert oa == ob
                np.testing.assert_allclose(a.logits_row(0), b2.logits_row(0), rtol=1e-5, atol=1e-4)
        finally:
            b2.close()
    finally:
        a.close()
        b.close()


def test_tiny_mtp_draft_matches_oracle(have_gpu):
    cfg = presets.tiny()
    rng = np.random.default_rng(3)
    toks = rng.integers(0, cfg.vocab_size, size=10).tolist()
    eng = Engine(cfg, experts=4, drafts=1, max_t=128)
    orc = OracleModel(cfg)
    st = orc.new_state()
    try:
        for p in range(len(toks) - 1):
            eng.step_rows([toks[p]])
            eng.commit(1)
            d = eng.mtp_draft([toks[p + 1]], 1)
            got = eng.mtp_logits_row(0)
            st.forward_token(toks[p])
            ref, _ = st.mtp_forward(toks[p + 1], st.last_hyper(), p)
            check_logits(got, ref, f"mtp pos {p}")
            assert len(d) == 1
    finally:
        eng.close()


def test_tiny_speculative_decode_equals_greedy(have_gpu):
    """The runner with 2 MTP drafts (3-row verify) emits the same tokens as
    plain greedy decode: verification is exact."""
    cfg = presets.tiny()
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, cfg.vocab_size, size=16).tolist()
    outs = []
    for drafts in (0, 2):
        eng = Engine(cfg, experts=4, drafts=drafts, max_t=256)
        try:
            nxt, dr = eng.prefill_chunk(prompt)
            d = Decode(eng, nxt, [dr] if (drafts and dr is not None) else [], drafts, limit=48, no_eos=True)
            outs.append(d.run())
            if drafts:
                steps, acc = d.stats()
                assert steps + acc == 48
        finally:
            eng.close()
    assert outs[0] == outs[1]


def test_full_shape_model_few_tokens(have_gpu):
    """Config 5 shape (48 layers, 512 experts, vocab 151936): 4 prompt tokens
    and 4 greedy decode tokens against the oracle."""
    cfg = presets.qwen3next_80b_shape(mtp=0)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab_size, size=4).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=64)
    try:
        logs = []
        out = None
        L = cfg.num_hidden_layers
        for p, t in enumerate(prompt):
            out = eng.step_rows([t])
            logs.append((p, eng.logits_row(0), engine_routes(eng, L)))
            eng.commit(1)
        gen = []
        tok = out[0]
        for i in range(4):
            gen.append(tok)
            out = eng.step_rows([tok])
            logs.append((len(prompt) + i, eng.logits_row(0), engine_routes(eng, L)))
            eng.commit(1)
            tok = out[0]
        exempt = teacher_forced(cfg, gen, prompt, logs, "full")
        assert exempt <= 1
    finally:
        eng.close()
