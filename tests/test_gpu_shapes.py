"""Parity at model shapes other than the 80B preset and the tiny model:

- the reference's qwen4_exp test checkpoint shape (tests/fixtures/qwen4_exp/
  config.json: hidden 256, 48 DeltaNet value heads over 16 key heads,
  8 experts top-4, vocab 248,320, the PLE block before layer 2, QSA budget
  2048), on synthetic weights;
- hidden 4096, the widest the batch-1 kernels take (two 32-input chunks
  per lane in the expert gate/up and LM head kernels);
- a shared expert wider or narrower than the routed ones (the reference's
  CPU path loads shared_expert.* at its own shared_expert_intermediate_size,
  cpu.rs:236-240; its Metal loader refuses the case, gpu/load.rs:320-323).

Each runs a GEMM prefill and batch-1 decode steps against the oracle run
token by token (forward_token, cpu.rs, q8 KV rule) at the north-star bar:
every decode position's logits, the prefill's last row, and the greedy
token where the margin exceeds 1e-3."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Engine
from oracle.oracle import OracleModel
from tests.gpu_util import argmax_margin, assert_close

pytestmark = pytest.mark.gpu


def prefill_then_decode(cfg, label, prompt_len, steps, seed):
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, cfg.vocab_size, size=prompt_len).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=prompt_len + steps + 8)
    st = OracleModel(cfg).new_state()
    try:
        nxt, _ = eng.prefill_chunk(prompt)
        got = eng.logits_row(0)
        ref = None
        for t in prompt:
            ref = st.forward_token(t, True)
        assert_close(got, ref, f"{label}: prefill last row")
        if argmax_margin(ref) > 1e-3:
            assert nxt == int(np.argmax(ref)), f"{label}: prefill greedy"
        tok = nxt
        for i in range(steps):
            out = eng.step_rows([tok])
            got = eng.logits_row(0)
            eng.commit(1)
            ref = st.forward_token(tok, True)
            assert_close(got, ref, f"{label}: decode position {prompt_len + i}")
            if argmax_margin(ref) > 1e-3:
                assert out[0] == int(np.argmax(ref)), f"{label}: decode greedy {i}"
            tok = out[0]
    finally:
        eng.close()


def test_reference_fixture_shape_matches_oracle(have_gpu):
    prefill_then_decode(presets.qwen4_exp_fixture(), "fixture shape", prompt_len=24, steps=6, seed=121)


def test_hidden_4096_matches_oracle(have_gpu):
    prefill_then_decode(presets.wide(), "hidden 4096", prompt_len=20, steps=5, seed=122)


def test_hc_lowrank_512_matches_oracle(have_gpu):
    """A hyper-connection low rank of 512 (8 quant groups: the up GEMM runs
    its staged-scale form, whose rows are then staged by their own pass)."""
    cfg = presets.tiny(mtp=0)
    cfg.hc_lowrank = 512
    prefill_then_decode(cfg, "hc low rank 512", prompt_len=40, steps=3, seed=123)


@pytest.mark.parametrize("si", [512, 128])
def test_shared_expert_width_differs_from_routed(have_gpu, si):
    """Routed experts of width 256 with a shared expert of `si`: GEMM
    prefill and batch-1 decode against the oracle, then a 3-row verify step
    (rows of topk I + SI activations each) whose every row matches the
    oracle, and the MTP head's draft logits."""
    cfg = presets.tiny(mtp=1)
    cfg.shared_expert_intermediate_size = si
    assert cfg.moe_intermediate_size == 256
    prefill_then_decode(cfg, f"shared width {si}", prompt_len=40, steps=4, seed=130 + si)

    rng = np.random.default_rng(140 + si)
    toks = rng.integers(0, cfg.vocab_size, size=9).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=64)
    st = OracleModel(cfg).new_state()
    try:
        for t in toks[:5]:
            eng.step_rows([t])
            eng.commit(1)
            st.forward_token(t, True)
        rows = toks[5:8]
        eng.step_rows(rows)
        got = [eng.logits_row(r).copy() for r in range(3)]
        for r, t in enumerate(rows):
            assert_close(got[r], st.forward_token(t, True), f"shared width {si}: verify row {r}")
    finally:
        eng.close()

    # the MTP head's own MoE block, position by position
    eng = Engine(cfg, experts=4, drafts=1, max_t=64)
    st = OracleModel(cfg).new_state()
    try:
        for p in range(4):
            eng.step_rows([toks[p]])
            eng.commit(1)
            eng.mtp_draft([toks[p + 1]], 1)
            st.forward_token(toks[p])
            ref, _ = st.mtp_forward(toks[p + 1], st.last_hyper(), p)
            assert_close(eng.mtp_logits_row(0), ref, f"shared width {si}: MTP position {p}")
    finally:
        eng.close()
