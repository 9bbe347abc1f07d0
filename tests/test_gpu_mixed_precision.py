"""Per-record expert precision (Pool::kind / set_kind, src/qwen4_exp/gpu/
residency.rs:290-310; the expert kernels take each record's path from its
kind, kernels/qwen4_exp/experts.metal:181-296): an engine with a Q3 or Q2
store attached switches about half of its records back to 4-bit, and one
launch then mixes both kinds.

- Batch-1 decode steps (row path) and the GEMM prefill are compared with
  the oracle (forward_token, cpu.rs) whose records carry the same
  per-record precision (the midpoint rule for the low-bit ones,
  tests/unit/qwen4_exp/gpu/prefill.rs:177-198), at the north-star bar.
- A low-bit engine with every record switched to 4-bit decodes bit for
  bit like the 4-bit engine (the same Q4 fragments, from the 4-bit copy).
- Switching a record back restores its low-bit results exactly."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Engine
from oracle.oracle import OracleModel
from tests.gpu_util import argmax_margin, assert_close

pytestmark = pytest.mark.gpu


def mixed_kinds(cfg, rng, bits):
    """{(record layer, expert): bits} with about half of the records at 4."""
    E = cfg.num_experts
    return {(rl, e): (4 if rng.random() < 0.5 else bits) for rl in range(cfg.num_hidden_layers) for e in range(E)}


def apply_kinds(eng, orc, cfg, kinds, bits):
    E = cfg.num_experts
    kind_of = {4: 0, 3: 1, 2: 2}
    for (rl, e), b in kinds.items():
        eng.pool_set_kind(rl * E + e, kind_of[b])
        if orc is not None:
            orc.set_record_bits(rl, e, b)
    for (rl, e), b in kinds.items():
        assert eng.pool_kind(rl * E + e) == kind_of[b]


@pytest.mark.parametrize("bits", [3, 2])
def test_mixed_precision_decode_matches_oracle(have_gpu, bits):
    cfg = presets.tiny(mtp=0)
    rng = np.random.default_rng(60 + bits)
    kinds = mixed_kinds(cfg, rng, bits)
    assert 0 < sum(b == 4 for b in kinds.values()) < len(kinds)
    eng = Engine(cfg, experts=bits, drafts=0, max_t=64)
    orc = OracleModel(cfg, expert_bits=bits)
    try:
        apply_kinds(eng, orc, cfg, kinds, bits)
        st = orc.new_state()
        toks = rng.integers(0, cfg.vocab_size, size=6).tolist()
        tok = None
        for i in range(12):
            t = toks[i] if i < len(toks) else tok
            out = eng.step_rows([t])
            got = eng.logits_row(0)
            eng.commit(1)
            ref = st.forward_token(t, True)
            assert_close(got, ref, f"mixed Q4/Q{bits} decode position {i}")
            if argmax_margin(ref) > 1e-3:
                assert out[0] == int(np.argmax(ref)), f"position {i}"
            tok = out[0]
    finally:
        eng.close()


@pytest.mark.parametrize("bits", [3, 2])
def test_mixed_precision_prefill_matches_oracle(have_gpu, bits):
    """The grouped expert GEMMs of one prefill take each expert group's
    record from the store of its kind; the last row's logits match the
    oracle run token by token."""
    cfg = presets.tiny(mtp=0)
    rng = np.random.default_rng(70 + bits)
    kinds = mixed_kinds(cfg, rng, bits)
    prompt = rng.integers(0, cfg.vocab_size, size=90).tolist()
    eng = Engine(cfg, experts=bits, drafts=0, max_t=128)
    orc = OracleModel(cfg, expert_bits=bits)
    try:
        apply_kinds(eng, orc, cfg, kinds, bits)
        nxt, _ = eng.prefill_chunk(prompt)
        got = eng.logits_row(0)
    finally:
        eng.close()
    st = orc.new_state()
    ref = None
    for t in prompt:
        ref = st.forward_token(t, True)
    assert_close(got, ref, f"mixed Q4/Q{bits} prefill vs oracle")
    if argmax_margin(ref) > 1e-3:
        assert nxt == int(np.argmax(ref))


def test_all_records_switched_to_4bit_equal_the_4bit_engine(have_gpu):
    """A Q2 engine whose every record is set to kind 0 decodes exactly like
    the 4-bit engine; setting the records back to kind 2 gives exactly the
    plain Q2 engine's results."""
    cfg = presets.tiny(mtp=0)
    E, L = cfg.num_experts, cfg.num_hidden_layers
    toks = np.random.default_rng(80).integers(0, cfg.vocab_size, size=5).tolist()

    def run(eng):
        eng.reset()
        outs = []
        for t in toks:
            outs.append((eng.step_rows([t])[0], eng.logits_row(0).copy()))
            eng.commit(1)
        return outs

    q4 = Engine(cfg, experts=4, drafts=0, max_t=32)
    q2 = Engine(cfg, experts=2, drafts=0, max_t=32)
    try:
        ref4, ref2 = run(q4), run(q2)
        for rid in range(L * E):
            q2.pool_set_kind(rid, 0)
        for (ta, la), (tb, lb) in zip(run(q2), ref4):
            assert ta == tb
            np.testing.assert_array_equal(la, lb)
        for rid in range(L * E):
            q2.pool_set_kind(rid, 2)
        for (ta, la), (tb, lb) in zip(run(q2), ref2):
            assert ta == tb
            np.testing.assert_array_equal(la, lb)
    finally:
        q4.close()
        q2.close()
