"""GPU parity of the PLE n-gram block (CpuModel::ple, src/qwen4_exp/cpu.rs:
889-967; gpu/ple.rs and gpu/prefill/ple.rs) in the engine: the row path and
the GEMM prefill against the oracle run token by token, verify steps whose
drafts are rejected (the ring rows they overwrote restored), checkpoints
(the ring is a prefix region), and a packed store's n-gram table and hash
metadata (ngram.bin and the I64 dense tensors) against the generated model.
The tiny preset with the qwen4_exp fixture's PLE dimensions: the block
before decoder layer 2 (ple_layer_ids [2]), 16 heads of 16-wide rows in
groups of 16, conv kernel 4 with dilation 3 (a 9-slot ring)."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Decode, Engine
from oracle.oracle import OracleModel
from tests.gpu_util import argmax_margin, assert_close
from tests.store_writer import write_store

pytestmark = pytest.mark.gpu


def ple_tiny(mtp=1, seed=1234):
    return presets.with_ple(presets.tiny(mtp=mtp, seed=seed), layer=2)


def test_row_path_matches_oracle(have_gpu):
    """One token per step for 24 positions (the ring wraps twice; a prompt
    EOS resets the n-gram window): every step's logits and greedy token."""
    cfg = ple_tiny(mtp=0)
    rng = np.random.default_rng(70)
    toks = rng.integers(0, cfg.vocab_size, size=24).tolist()
    toks[9] = cfg.eos_token_id
    eng = Engine(cfg, experts=4, drafts=0, max_t=64)
    st = OracleModel(cfg).new_state()
    try:
        for p, t in enumerate(toks):
            nxt = eng.step_rows([t])[0]
            eng.commit(1)
            ref = st.forward_token(t, True)
            assert_close(eng.logits_row(0), ref, f"position {p}")
            if argmax_margin(ref) > 1e-3:
                assert nxt == int(np.argmax(ref)), p
    finally:
        eng.close()


@pytest.mark.parametrize("splits", [[40], [13, 27]])
def test_gemm_prefill_matches_oracle(have_gpu, splits):
    """The GEMM prefill (chunks of 40, or 13 then 27 so the second chunk's
    taps reach into the ring the first one left): every row's logits
    (all-logits mode) and the MTP draft's, against the oracle."""
    cfg = ple_tiny(mtp=1)
    rng = np.random.default_rng(71 + len(splits))
    prompt = rng.integers(0, cfg.vocab_size, size=sum(splits)).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=128)
    rows = []
    try:
        i = 0
        for k in splits:
            after = prompt[i + k] if i + k < len(prompt) else None
            nxt, dr = eng.prefill_chunk(prompt[i:i + k], next_after=after, all_logits=True)
            rows += [eng.pf_logits_row(r) for r in range(k)]
            i += k
        got_mtp = eng.mtp_logits_row(0)
    finally:
        eng.close()
    st = OracleModel(cfg).new_state()
    ref = None
    for p, t in enumerate(prompt):
        ref = st.forward_token(t, True)
        assert_close(rows[p], ref, f"prefill row {p}")
    if argmax_margin(ref) > 1e-3:
        assert nxt == int(np.argmax(ref))
    st2 = OracleModel(cfg).new_state()
    mref = None
    for p, t in enumerate(prompt):
        st2.forward_token(t, True)
        after = prompt[p + 1] if p + 1 < len(prompt) else nxt
        mref, _ = st2.mtp_forward(after, st2.last_hyper(), p)
    assert_close(got_mtp, mref, "MTP draft logits", abs_frac=2e-3, min_cos=0.99999)
    if argmax_margin(mref) > 1e-3:
        assert dr == int(np.argmax(mref))


def test_rejected_rows_leave_the_ring_as_before(have_gpu):
    """After 12 positions, a 3-row snapshotting step committed at 1 (rows 2
    and 3 rejected), then 12 more single steps: each step's logits equal a
    run that never saw the rejected rows (tight: same kernels), and the
    oracle's.  Position 13's oldest tap reads the slot row 2 overwrote."""
    cfg = ple_tiny(mtp=1)
    rng = np.random.default_rng(72)
    prompt = rng.integers(0, cfg.vocab_size, size=12).tolist()
    cont = rng.integers(0, cfg.vocab_size, size=13).tolist()
    a = Engine(cfg, experts=4, drafts=2, max_t=64)
    b = Engine(cfg, experts=4, drafts=2, max_t=64)
    st = OracleModel(cfg).new_state()
    try:
        for t in prompt:
            st.forward_token(t, True)
        a.prefill_chunk(prompt)
        b.prefill_chunk(prompt)
        bogus = [(cont[1] + 7) % cfg.vocab_size, (cont[2] + 11) % cfg.vocab_size]
        a.step_rows([cont[0]] + bogus, snap=True)
        a.commit(1)
        b.step_rows([cont[0]])
        b.commit(1)
        ref = st.forward_token(cont[0], True)
        assert_close(a.logits_row(0), ref, "verify row 0")
        for p, t in enumerate(cont[1:], start=1):
            a.step_rows([t])
            a.commit(1)
            b.step_rows([t])
            b.commit(1)
            ref = st.forward_token(t, True)
            assert_close(a.logits_row(0), b.logits_row(0), f"after rollback, step {p}", abs_frac=1e-5,
                         min_cos=0.9999999)
            assert_close(a.logits_row(0), ref, f"after rollback vs oracle, step {p}")
    finally:
        a.close()
        b.close()


def test_speculative_decode_equals_greedy(have_gpu):
    """The runner with 2 drafts emits plain greedy decode's tokens on a PLE
    model (rejections roll the ring back)."""
    cfg = ple_tiny(mtp=1, seed=99)
    cfg.vocab_size = 16
    cfg.eos_token_id = 15
    prompt = np.random.default_rng(99).integers(0, 15, size=8).tolist()
    outs, stats = [], []
    for drafts in (0, 2):
        eng = Engine(cfg, experts=4, drafts=drafts, max_t=128)
        try:
            nxt, dr = eng.prefill_chunk(prompt)
            d = Decode(eng, nxt, [dr] if (drafts and dr is not None) else [], drafts, limit=48, no_eos=True)
            outs.append(d.run())
            stats.append(d.stats())
        finally:
            eng.close()
    print(f"speculative: {stats[1]}", flush=True)
    assert outs[0] == outs[1]


def test_checkpoint_carries_the_ring(have_gpu):
    """Save after 11 tokens, decode 6, restore, decode the same 6: the same
    logits; the ring is one of the prefix regions."""
    cfg = ple_tiny(mtp=0)
    rng = np.random.default_rng(73)
    prompt = rng.integers(0, cfg.vocab_size, size=11).tolist()
    cont = rng.integers(0, cfg.vocab_size, size=6).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=64)
    try:
        eng.prefill_chunk(prompt)
        hh = cfg.hidden_size * cfg.hc_count
        regs = eng.prefix_regions(11, 0)
        assert regs[-1][1] == 9 * hh * 4
        cp = eng.save_prefix()
        first = []
        for t in cont:
            eng.step_rows([t])
            eng.commit(1)
            first.append(eng.logits_row(0).copy())
        eng.reset_request()
        eng.restore_prefix(cp)
        for i, t in enumerate(cont):
            eng.step_rows([t])
            eng.commit(1)
            np.testing.assert_array_equal(eng.logits_row(0), first[i])
    finally:
        eng.close()


def test_store_ple_equals_generated(have_gpu, tmp_path):
    """A store's key/value projections, norms, conv, n-gram table (ngram.bin)
    and hash metadata (I64 dense tensors; the manifest's copies are wrong on
    purpose) give the generated model's decode bit for bit."""
    cfg = ple_tiny(mtp=0)
    path = write_store(cfg, tmp_path / "packed")
    a = Engine.load_store(path, experts=4, drafts=0, max_t=64)
    b = Engine(cfg, experts=4, drafts=0, max_t=64)
    try:
        rng = np.random.default_rng(74)
        prompt = rng.integers(0, cfg.vocab_size, size=20).tolist()
        na, _ = a.prefill_chunk(prompt)
        nb, _ = b.prefill_chunk(prompt)
        assert na == nb
        np.testing.assert_array_equal(a.logits_row(0), b.logits_row(0))
        for t in rng.integers(0, cfg.vocab_size, size=4).tolist():
            assert a.step_rows([t]) == b.step_rows([t])
            a.commit(1)
            b.commit(1)
            np.testing.assert_array_equal(a.logits_row(0), b.logits_row(0))
    finally:
        a.close()
        b.close()
