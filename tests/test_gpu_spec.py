"""GPU tests of the speculative path with drafts accepted: a verify step
whose drafts are the trunk's own greedy continuation commits every row
(gpu/decode.rs:13-58, gpu/state.rs:10-56), a wrong draft commits the rows
before it and rolls the DeltaNet state back; the folded MTP pass over the
verify rows (gpu/decode.rs:163-193) leaves the draft that sequential steps
leave (gpu/mtp.rs:11-78); and the runner (runner/decode.rs:88-171) accepts
drafts and still emits the greedy tokens.  Also the 48-layer MTP head
against the oracle and the 48-layer speculative run after a 2048-token
prefill (config 5)."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import check, lib
from cherenkov_amd.engine import Decode, Engine
from oracle.oracle import OracleModel
from tests.gpu_util import ROUTE_TIE_TOL, argmax_margin, assert_close, engine_routes

pytestmark = pytest.mark.gpu


def dn_state(eng, cfg, layer):
    nv, dk, dv = cfg.linear_num_value_heads, cfg.linear_key_head_dim, cfg.linear_value_head_dim
    conv_dim = 2 * cfg.linear_num_key_heads * dk + nv * dv
    s = np.empty(nv * dk * dv, np.float32)
    c = np.empty(conv_dim * (cfg.linear_conv_kernel_dim - 1), np.float32)
    check(lib().chk_deltanet_state(eng.handle, layer, s.ctypes.data, c.ctypes.data))
    return s, c


def same_state(a, b, cfg, label):
    for layer in range(cfg.num_hidden_layers):
        if (layer + 1) % cfg.full_attention_interval == 0:
            continue
        sa, ca = dn_state(a, cfg, layer)
        sb, cb = dn_state(b, cfg, layer)
        assert_close(sa, sb, f"{label} layer {layer} state", abs_frac=1e-5, min_cos=0.9999999)
        assert_close(ca, cb, f"{label} layer {layer} conv history", abs_frac=1e-5, min_cos=0.9999999)


def sequential(b: Engine, tok: int, n: int, chain_last: int):
    """n single-row steps, each committed and followed by the MTP pass over
    that row paired with its greedy token (chain 1; the last `chain_last`)."""
    outs, logs, drafts = [], [], None
    for i in range(n):
        o = b.step_rows([tok])
        logs.append(b.logits_row(0))
        b.commit(1)
        drafts = b.mtp_draft([o[0]], chain_last if i == n - 1 else 1)
        outs.append(o[0])
        tok = o[0]
    return outs, logs, drafts, b.mtp_logits_row(0)


@pytest.mark.parametrize("wrong_at", [None, 2, 1])
def test_verify_commits_accepted_drafts(have_gpu, wrong_at):
    """rows = [cur, g1, g2] with g the trunk's greedy continuation (all
    accepted: commit 3), or one draft replaced by a wrong token (commit the
    rows before it: rollback to snapshot plane n-1).  Logits of the kept
    rows, the DeltaNet state after the commit and the MTP drafts from the
    folded pass equal those of sequential single-row steps."""
    cfg = presets.tiny(mtp=1)
    rng = np.random.default_rng(800 + (wrong_at or 0))
    prompt = rng.integers(0, cfg.vocab_size, size=12).tolist()
    a = Engine(cfg, experts=4, drafts=3, max_t=128)
    b = Engine(cfg, experts=4, drafts=3, max_t=128)
    try:
        cur, _ = a.prefill_chunk(prompt)
        cur_b, _ = b.prefill_chunk(prompt)
        assert cur == cur_b
        # the trunk's greedy continuation, from a probe that is discarded
        probe = Engine(cfg, experts=4, drafts=3, max_t=128)
        try:
            probe.prefill_chunk(prompt)
            g, _, _, _ = sequential(probe, cur, 3, 1)
        finally:
            probe.close()
        rows = [cur, g[0], g[1]]
        if wrong_at is not None:
            rows[wrong_at] = (g[wrong_at - 1] + 1) % cfg.vocab_size
        res = a.step_rows(rows, snap=True, fold_mtp=True)
        la = [a.logits_row(r) for r in range(3)]
        n = 1
        while n < 3 and res[n - 1] == rows[n]:
            n += 1
        assert n == (3 if wrong_at is None else wrong_at)
        a.commit(n)
        nxt = rows[1:n] + [res[n - 1]]
        chain = 2 if n == 3 else 1
        da = a.mtp_draft(nxt, chain)
        # the last draft pass: the chained one (row 0), or with chain 1 the
        # folded pass itself, whose row n-1 pairs the last kept row
        ma = a.mtp_logits_row(0 if chain > 1 else n - 1)
        outs, logs, db, mb = sequential(b, cur, n, chain)
        assert res[:n] == outs
        for r in range(n):
            assert_close(la[r], logs[r], f"row {r} logits", abs_frac=1e-5, min_cos=0.9999999)
        same_state(a, b, cfg, f"commit {n}")
        assert_close(ma, mb, "last MTP pass logits", abs_frac=1e-5, min_cos=0.9999999)
        assert len(da) == len(db) == chain
        if argmax_margin(mb) > 1e-3:
            assert da[-1] == db[-1]
        if chain == 1 or argmax_margin(mb) > 1e-3:
            assert da[0] == db[0]
        # both continue identically
        tok = res[n - 1]
        for i in range(4):
            oa = a.step(tok)
            ob = b.step(tok)
            assert oa == ob
            assert_close(a.logits_row(0), b.logits_row(0), f"after commit step {i}", abs_frac=1e-5,
                         min_cos=0.9999999)
            tok = ob
    finally:
        a.close()
        b.close()


def test_runner_accepts_drafts_and_equals_greedy(have_gpu):
    """The runner with 2 drafts on a model whose MTP head often agrees with
    the trunk (vocab 16, seed 99: the oracle's first drafts match the next
    greedy token at 8 of 32 positions) accepts drafts — committing 2- and
    3-row verify steps and redrafting with chain 2 after a full accept —
    and emits exactly the tokens of plain greedy decode."""
    cfg = presets.tiny(seed=99)
    cfg.vocab_size = 16
    rng = np.random.default_rng(99)
    prompt = rng.integers(0, cfg.vocab_size, size=8).tolist()
    outs, stats = [], []
    for drafts in (0, 2):
        eng = Engine(cfg, experts=4, drafts=drafts, max_t=256)
        try:
            nxt, dr = eng.prefill_chunk(prompt)
            d = Decode(eng, nxt, [dr] if (drafts and dr is not None) else [], drafts, limit=64, no_eos=True)
            outs.append(d.run())
            stats.append(d.stats())
        finally:
            eng.close()
    assert outs[0] == outs[1]
    steps, acc = stats[1]
    print(f"speculative: {steps} steps, {acc} accepted drafts", flush=True)
    assert steps + acc == 64
    assert acc > 0


def test_runner_stops_on_any_eos_id(have_gpu):
    """The runner stops on any id of its EOS set (the reference's
    [im_end, endoftext], runner/decode.rs:64,76-80): the stop id is not
    emitted, a verify step accepts no draft past it, and the output is the
    greedy tokens before the first stop id, with and without drafts."""
    cfg = presets.tiny(seed=99)
    cfg.vocab_size = 16
    rng = np.random.default_rng(99)
    prompt = rng.integers(0, cfg.vocab_size, size=8).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=512)
    try:
        nxt, dr = eng.prefill_chunk(prompt)
        cp = eng.save_prefix()
        g = Decode(eng, nxt, [], 0, limit=64, no_eos=True).run()
        first = {}
        for i, t in enumerate(g):
            first.setdefault(t, i)
        (ta, ka), (tb, kb) = sorted(first.items(), key=lambda kv: kv[1])[-2:]
        assert 1 <= ka < kb, (ka, kb)
        for ids, stop in (([tb, ta], ka), ([tb], kb)):
            for drafts in (0, 2):
                eng.reset_request()
                eng.restore_prefix(cp)
                d = Decode(eng, nxt, [dr] if drafts else [], drafts, limit=64, no_eos=False)
                d.set_eos(ids)
                out = d.run()
                assert out == g[:stop], (ids, drafts)
                assert d.finished == 1
    finally:
        eng.close()


def test_full_shape_mtp_draft_matches_oracle(have_gpu):
    """The 48-layer preset's MTP head (its own attention + MoE layer, the
    shared LM head) against the oracle's mtp_forward for a few positions."""
    cfg = presets.qwen3next_80b_shape(mtp=1)
    rng = np.random.default_rng(901)
    toks = rng.integers(0, cfg.vocab_size, size=4).tolist()
    eng = Engine(cfg, experts=4, drafts=1, max_t=64)
    st = OracleModel(cfg).new_state()
    try:
        for p in range(len(toks) - 1):
            eng.step_rows([toks[p]])
            got_t = eng.logits_row(0)
            eng.commit(1)
            d = eng.mtp_draft([toks[p + 1]], 1)
            got = eng.mtp_logits_row(0)
            # trunk layers then the MTP layer (index num_hidden_layers)
            st.route_hints(engine_routes(eng, cfg.num_hidden_layers + 1), ROUTE_TIE_TOL)
            ref_t = st.forward_token(toks[p])
            ref, _ = st.mtp_forward(toks[p + 1], st.last_hyper(), p)
            assert_close(got_t, ref_t, f"48-layer trunk pos {p}")
            assert_close(got, ref, f"48-layer MTP pos {p}")
            if argmax_margin(ref) > 1e-3:
                assert d[0] == int(np.argmax(ref))
        assert st.route_swaps <= 2 * (len(toks) - 1), f"{st.route_swaps} near-tie routes followed"
    finally:
        eng.close()


def test_full_shape_speculative_after_long_prefill_equals_greedy(have_gpu):
    """Config 5: a 2048-token GEMM prefill (MTP head included), then 2-draft
    speculative decode on the 48-layer preset emits the greedy tokens; the
    same sequence state serves both runs through a checkpoint."""
    cfg = presets.qwen3next_80b_shape(mtp=1)
    rng = np.random.default_rng(902)
    prompt = rng.integers(0, cfg.vocab_size, size=2048).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=2048 + 64)
    try:
        nxt, dr = eng.prefill_chunk(prompt)
        cp = eng.save_prefix()
        g = Decode(eng, nxt, [], 0, limit=24, no_eos=True).run()
        eng.reset_request()
        eng.restore_prefix(cp)
        d = Decode(eng, nxt, [dr], 2, limit=24, no_eos=True)
        s = d.run()
        steps, acc = d.stats()
        print(f"48-layer speculative: {steps} steps, {acc} accepted", flush=True)
        assert s == g
        assert steps + acc == 24
    finally:
        eng.close()
