"""GPU parity of the QSA indexer (select_tokens, /root/reference/src/
qwen4_exp/cpu.rs:643-719): the block selection kernel against the
reference's tie test and random scores (oracle qsa_pick), and the whole
token loop with a budget the context passes, against the CPU oracle.

Reference tests followed: tests/unit/qwen4_exp/gpu/qsa.rs:143-372
(index_pipeline_matches_cpu, index_select_handles_ties).
"""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import check, lib
from cherenkov_amd.engine import Decode, Engine
from oracle.oracle import OracleModel, qsa_pick
from tests.gpu_util import argmax_margin, assert_close, empty_dev, to_dev, to_host
from tests.test_gpu_model import teacher_forced
from tests.test_oracle import _qsa_expect

pytestmark = pytest.mark.gpu


def gpu_select(scores, t_len, k, ratio):
    n = t_len // ratio
    words = (n + 1 + 31) // 32
    dmask = empty_dev((words,), np.uint32)
    check(lib().chk_qsa_select(to_dev(scores.astype(np.float32)).data_ptr(), t_len, k, ratio, dmask.data_ptr(), None))
    bits = to_host(dmask).view(np.uint32)
    blocks = [b for b in range(n) if (bits[b // 32] >> (b % 32)) & 1]
    vis = [t for b in blocks for t in range(b * ratio, (b + 1) * ratio)] + list(range(n * ratio, t_len))
    return sorted(vis)


def test_qsa_select_reference_ties(have_gpu):
    ratio, k, base_pos = 4, 512, 2401
    t_len = base_pos + 1
    n = t_len // ratio
    scores = np.array([0.0 if i % 3 == 0 else ((i * 7) % 5) * 0.5 for i in range(n + 8)], np.float32)
    assert gpu_select(scores, t_len, k, ratio) == _qsa_expect(scores, t_len, k, ratio)


@pytest.mark.parametrize("t_len,k,ratio", [(41, 3, 4), (2300, 512, 4), (9000, 100, 8), (65536 * 4 - 1, 5000, 4)])
def test_qsa_select_random(have_gpu, t_len, k, ratio):
    rng = np.random.default_rng(t_len)
    n = t_len // ratio
    scores = rng.choice(np.float32([0.0, 0.5, 1.0, 3.0]), size=n) + (rng.random(n) < 0.5) * rng.random(n)
    scores = scores.astype(np.float32)
    assert gpu_select(scores, t_len, k, ratio) == qsa_pick(scores, t_len, k, ratio).tolist()


def test_tiny_qsa_decode_matches_oracle(have_gpu):
    """Budget 16 tokens (4 blocks of 4): from the 21st token on each
    attention layer (and the MTP layer's) attends to its 4 best blocks plus
    the tail.  Prompt and greedy tokens against the oracle, teacher forced."""
    cfg = presets.tiny(indexer_budget=16)
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, cfg.vocab_size, size=30).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=128)
    try:
        logs = []
        out = None
        for p, t in enumerate(prompt):
            out = eng.step_rows([t])
            logs.append((p, eng.logits_row(0)))
            eng.commit(1)
        gen = []
        tok = out[0]
        for i in range(30):
            gen.append(tok)
            out = eng.step_rows([tok])
            logs.append((len(prompt) + i, eng.logits_row(0)))
            eng.commit(1)
            tok = out[0]
        exempt = teacher_forced(cfg, gen, prompt, logs, "qsa")
        assert exempt <= 2
    finally:
        eng.close()


def test_tiny_qsa_speculative_equals_greedy(have_gpu):
    """3-row verify steps past the budget (block keys completed inside a
    batch, rollback of drafts inside a block) emit the greedy tokens."""
    cfg = presets.tiny(indexer_budget=16)
    rng = np.random.default_rng(22)
    prompt = rng.integers(0, cfg.vocab_size, size=18).tolist()
    outs = []
    for drafts in (0, 2):
        eng = Engine(cfg, experts=4, drafts=drafts, max_t=256)
        try:
            nxt, dr = eng.prefill_chunk(prompt)
            d = Decode(eng, nxt, [dr] if (drafts and dr is not None) else [], drafts, limit=64, no_eos=True)
            outs.append(d.run())
        finally:
            eng.close()
    assert outs[0] == outs[1]


def test_tiny_qsa_changes_attention(have_gpu):
    """The selective engine is not the dense model: past the budget its
    logits leave the dense oracle's tolerance (so the parity test above has
    power)."""
    from oracle.oracle import OracleModel
    from tests.gpu_util import cosine

    cfg = presets.tiny(indexer_budget=16)
    dense = presets.tiny()
    rng = np.random.default_rng(23)
    toks = rng.integers(0, cfg.vocab_size, size=48).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=128)
    st = OracleModel(dense).new_state()
    try:
        worst = 1.0
        for p, t in enumerate(toks):
            eng.step_rows([t])
            got = eng.logits_row(0)
            eng.commit(1)
            ref = st.forward_token(t)
            if p >= 24:
                worst = min(worst, cosine(got, ref))
        assert worst < 0.999, f"selection left every logit row within the dense bar (cos {worst:.6f})"
    finally:
        eng.close()


@pytest.mark.parametrize("splits", [[60], [37, 23], [10, 50]])
def test_tiny_qsa_gemm_prefill_matches_oracle(have_gpu, splits):
    """The GEMM prefill past the budget (16 tokens: rows from position 19 on
    select their 4 best blocks): rows before the boundary through the flash
    kernel, later rows through block scores and masked partials, the
    chunk's block keys cached for the next chunk.  Every row's logits
    (all-logits mode) against the oracle, the MTP draft against its
    mtp_forward, then decode steps reading the cached block keys."""
    cfg = presets.tiny(indexer_budget=16, mtp=1)
    rng = np.random.default_rng(22 + len(splits))
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
        st = OracleModel(cfg).new_state()
        st2 = OracleModel(cfg).new_state()
        mref = None
        for p, t in enumerate(prompt):
            ref = st.forward_token(t, True)
            assert_close(rows[p], ref, f"prefill row {p}")
            st2.forward_token(t, True)
            after = prompt[p + 1] if p + 1 < len(prompt) else nxt
            mref, _ = st2.mtp_forward(after, st2.last_hyper(), p)
        if argmax_margin(ref) > 1e-3:
            assert nxt == int(np.argmax(ref))
        assert_close(got_mtp, mref, "MTP draft logits", abs_frac=2e-3, min_cos=0.99999)
        for t in rng.integers(0, cfg.vocab_size, size=6).tolist():
            eng.step_rows([t])
            eng.commit(1)
            assert_close(eng.logits_row(0), st.forward_token(t, True), "decode after prefill")
    finally:
        eng.close()


def test_selection_debug_views_match_oracle(have_gpu):
    """Gpu::debug_engine_blocks (gpu/prefill.rs:471-484) after a GEMM
    prefill past the budget, for every row of the chunk, and Gpu::
    debug_row_vis (gpu/prefill.rs:486-494) after each decode step: the
    blocks and tokens the engine's last attention layer selected equal the
    oracle's select_tokens (cpu.rs:643-719) at the same positions; rows
    within the budget select no block in the prefill view and every token
    in the row view."""
    cfg = presets.tiny(indexer_budget=16, mtp=0)
    ratio, kblk = cfg.indexer_compress_ratio, 16 // cfg.indexer_compress_ratio
    layer = cfg.num_hidden_layers - 1
    assert (layer + 1) % cfg.full_attention_interval == 0
    rng = np.random.default_rng(29)
    prompt = rng.integers(0, cfg.vocab_size, size=50).tolist()
    eng = Engine(cfg, experts=4, drafts=0, max_t=128)
    st = OracleModel(cfg).new_state()
    try:
        eng.prefill_chunk(prompt)
        selective = 0
        for p, t in enumerate(prompt):
            st.forward_token(t, True)
            sel = st.last_selection(layer)
            nblk = (p + 1) // ratio
            got = eng.debug_engine_blocks(p)
            if nblk <= kblk:
                assert sel == list(range(p + 1)) and got == [], f"row {p}"
            else:
                selective += 1
                assert got == sorted({t_ // ratio for t_ in sel if t_ < nblk * ratio}), f"row {p}"
        assert selective > 20
        for t in rng.integers(0, cfg.vocab_size, size=4).tolist():
            eng.step_rows([t])
            eng.commit(1)
            st.forward_token(t, True)
            assert eng.debug_row_vis(0) == st.last_selection(layer)
    finally:
        eng.close()
