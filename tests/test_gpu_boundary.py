"""GPU tests of the engine boundary beyond the step itself: prefill_chunk's
`next_after` and `all_logits` (gpu/prefill.rs:190-201), pf_logits_row,
prefill_release and prefill_rows_fit (prefill.rs:467-507,
prefill/allocation.rs:150-169), the logits / KV / context accessors
(gpu.rs:601-690), reset_request (gpu/state.rs:232-263) and the expert-pool
interface over the all-resident store (gpu/residency.rs:255-460).  All calls
go through the C ABI (libcherenkov.so)."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import EngineError, check, lib
from cherenkov_amd.engine import Engine
from oracle.oracle import OracleModel
from tests.gpu_util import argmax_margin, assert_close, empty_dev, to_host

pytestmark = pytest.mark.gpu


def mtp_regions(eng: Engine, cp) -> list[np.ndarray]:
    """The MTP layer's KV regions of a checkpoint (the last five: q8 K, K
    scales, q8 V, V scales, index keys; no block keys while dense)."""
    regs = eng.prefix_regions(cp.pos, cp.mtp_len)
    out = []
    for i in range(len(regs) - 5, len(regs)):
        out.append(cp.region(i, regs[i][1]))
    return out


@pytest.mark.parametrize("splits", [[25, 15], [10, 17, 13]])
def test_split_prefill_with_next_after_equals_one_call(have_gpu, splits):
    """A prompt prefilled in several calls, each passing the next chunk's
    first token as next_after (runner.rs:119-125), leaves the MTP head the
    same state as one call: MTP logits and draft at the end, the MTP KV
    rows (q8 codes and scales) and the trunk's last-row logits."""
    cfg = presets.tiny(mtp=1)
    rng = np.random.default_rng(600 + len(splits))
    prompt = rng.integers(0, cfg.vocab_size, size=sum(splits)).tolist()
    a = Engine(cfg, experts=4, drafts=2, max_t=128)
    b = Engine(cfg, experts=4, drafts=2, max_t=128)
    try:
        nxt_a, dr_a = a.prefill_chunk(prompt)
        i = 0
        for n in splits:
            after = prompt[i + n] if i + n < len(prompt) else None
            nxt_b, dr_b = b.prefill_chunk(prompt[i:i + n], next_after=after)
            i += n
        assert a.pos == b.pos == len(prompt)
        la, lb = a.logits_row(0), b.logits_row(0)
        assert_close(lb, la, "trunk last-row logits", abs_frac=1e-5, min_cos=0.9999999)
        ma, mb = a.mtp_logits_row(0), b.mtp_logits_row(0)
        assert_close(mb, ma, "MTP logits", abs_frac=1e-5, min_cos=0.9999999)
        if argmax_margin(la) > 1e-3:
            assert nxt_a == nxt_b
        if argmax_margin(ma) > 1e-3:
            assert dr_a == dr_b
        ca, cb = a.save_prefix(), b.save_prefix()
        assert ca.mtp_len == cb.mtp_len == len(prompt)
        names = ["K q8", "K scales", "V q8", "V scales", "index keys"]
        for name, ra, rb in zip(names, mtp_regions(a, ca), mtp_regions(b, cb)):
            if name.endswith("q8"):
                d = np.abs(ra.view(np.int8).astype(np.int32) - rb.view(np.int8).astype(np.int32))
                # codes may round across a half-step where f32 sums differ in order
                assert d.max() <= 1 and np.count_nonzero(d) <= max(2, d.size // 2000), f"MTP {name}: {np.count_nonzero(d)} codes differ"
            elif name.endswith("scales"):
                fa = ra.view(np.float16).astype(np.float32)
                fb = rb.view(np.float16).astype(np.float32)
                np.testing.assert_allclose(fb, fa, rtol=2e-3, atol=0, err_msg=f"MTP {name}")
            else:
                assert_close(rb.view(np.float32), ra.view(np.float32), f"MTP {name}", abs_frac=1e-5,
                             min_cos=0.9999999)
    finally:
        a.close()
        b.close()


def test_split_prefill_mtp_boundary_row_matches_oracle(have_gpu):
    """At a chunk boundary with next_after, the MTP head pairs the first
    chunk's last row with the next prompt token: the final MTP logits match
    the oracle's mtp_forward over those pairs at a bar the wrong pairing
    (the trunk's greedy token) fails."""
    cfg = presets.tiny(mtp=1)
    rng = np.random.default_rng(502)
    prompt = rng.integers(0, cfg.vocab_size, size=40).tolist()
    split = 25
    eng = Engine(cfg, experts=4, drafts=2, max_t=128)
    wrong = Engine(cfg, experts=4, drafts=2, max_t=128)
    try:
        eng.prefill_chunk(prompt[:split], next_after=prompt[split])
        nxt, dr = eng.prefill_chunk(prompt[split:])
        got = eng.mtp_logits_row(0)
        greedy, _ = wrong.prefill_chunk(prompt[:split])  # no next_after: pairs the greedy token
        wrong.prefill_chunk(prompt[split:])
        got_wrong = wrong.mtp_logits_row(0)
    finally:
        eng.close()
        wrong.close()
    st = OracleModel(cfg).new_state()
    mref = None
    for p, t in enumerate(prompt):
        st.forward_token(t, True)
        after = prompt[p + 1] if p + 1 < len(prompt) else nxt
        mref, _ = st.mtp_forward(after, st.last_hyper(), p)
    assert_close(got, mref, "MTP logits with next_after vs oracle", abs_frac=2e-3, min_cos=0.99999)
    if argmax_margin(mref) > 1e-3:
        assert dr == int(np.argmax(mref))
    # the bar above is tight enough to see the pairing
    if greedy == prompt[split]:
        return
    err_wrong = float(np.max(np.abs(got_wrong - mref))) / max(1.0, float(np.max(np.abs(mref))))
    err_right = float(np.max(np.abs(got - mref))) / max(1.0, float(np.max(np.abs(mref))))
    assert err_wrong > 4 * err_right, (err_wrong, err_right)


@pytest.mark.parametrize("path", ["gemm", "rows"])
def test_prefill_all_logits_rows(have_gpu, path):
    """all_logits keeps every row's logits (pf_logits_row); each equals the
    logits of stepping that row alone, on the GEMM path and on the 4-row
    path (QSA past its budget sends prefill there)."""
    if path == "gemm":
        cfg = presets.tiny(mtp=1)
    else:
        cfg = presets.tiny(mtp=1, indexer_budget=8)
    rng = np.random.default_rng(611)
    prompt = rng.integers(0, cfg.vocab_size, size=30).tolist()
    a = Engine(cfg, experts=4, drafts=0, max_t=64)
    b = Engine(cfg, experts=4, drafts=0, max_t=64)
    try:
        with pytest.raises(EngineError, match="prefill logits not kept"):
            a.pf_logits_row(0)
        nxt, _ = a.prefill_chunk(prompt, all_logits=True)
        for r, t in enumerate(prompt):
            b.step_rows([t])
            ref = b.logits_row(0)
            b.commit(1)
            assert_close(a.pf_logits_row(r), ref, f"{path} row {r}", abs_frac=1e-3, min_cos=0.99999)
        with pytest.raises(EngineError, match="out of range"):
            a.pf_logits_row(len(prompt))
        # the final row is also logits_row(0) / logits(); no step is in flight
        np.testing.assert_array_equal(a.logits(), a.logits_row(0))
        assert a.last_logits_row() == 0
        np.testing.assert_allclose(a.logits(), a.pf_logits_row(len(prompt) - 1), rtol=1e-5, atol=1e-5)
        with pytest.raises(EngineError, match="commit 1 of 0 rows"):
            a.commit(1)
        # a later chunk without all_logits drops them
        a.prefill_chunk(prompt[:3])
        with pytest.raises(EngineError, match="prefill logits not kept"):
            a.pf_logits_row(0)
    finally:
        a.close()
        b.close()


def test_prefill_release_and_rows_fit(have_gpu):
    cfg = presets.tiny(mtp=1)
    rng = np.random.default_rng(612)
    prompt = rng.integers(0, cfg.vocab_size, size=40).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=96)
    ref = Engine(cfg, experts=4, drafts=2, max_t=96)
    try:
        fit = eng.prefill_rows_fit(False)
        assert 1 <= fit <= 96
        assert eng.prefill_rows_fit(True) <= fit
        gb0 = eng.allocated_gb()
        eng.prefill_chunk(prompt[:20], next_after=prompt[20])
        gb1 = eng.allocated_gb()
        assert gb1 > gb0
        eng.prefill_release()
        assert abs(eng.allocated_gb() - gb0) < 1e-9
        nxt, dr = eng.prefill_chunk(prompt[20:])  # reallocates its scratch
        nxt_r, dr_r = ref.prefill_chunk(prompt)
        assert_close(eng.logits_row(0), ref.logits_row(0), "after release", abs_frac=1e-5, min_cos=0.9999999)
        if argmax_margin(ref.logits_row(0)) > 1e-3:
            assert nxt == nxt_r
    finally:
        eng.close()
        ref.close()


def test_sequence_accessors(have_gpu):
    """kv_cache_bytes / capacity / fullness and context_fullness follow the
    sequence (trunk attention layers at pos, the MTP layer at its own
    length); allocated_gb covers the engine's memory."""
    cfg = presets.tiny(mtp=1)
    max_t = 64
    eng = Engine(cfg, experts=4, drafts=1, max_t=max_t)
    try:
        kv_row = cfg.num_key_value_heads * cfg.head_dim
        per = lambda n: 2 * (n * kv_row + n * (kv_row // 32) * 2) + n * cfg.indexer_head_dim * 4
        n_attn = cfg.num_hidden_layers // cfg.full_attention_interval
        assert eng.kv_cache_capacity() == (n_attn + 1) * per(max_t)
        assert eng.kv_cache_bytes() == 0 and eng.context_fullness() == 0.0
        rng = np.random.default_rng(613)
        eng.prefill_chunk(rng.integers(0, cfg.vocab_size, size=16).tolist())
        assert eng.kv_cache_bytes() == (n_attn + 1) * per(16)
        assert abs(eng.kv_cache_fullness() - 16 / max_t) < 1e-12
        assert abs(eng.context_fullness() - 16 / max_t) < 1e-12
        ms = eng.memory_stats()
        assert eng.allocated_gb() * 1e9 >= 0.99 * (ms["dense"] + ms["experts"] + ms["state"] + ms["kv_cache"])
        eng.reset_request()
        assert eng.pos == 0 and eng.kv_cache_bytes() == 0
        with pytest.raises(EngineError, match="out of range"):
            eng.logits_row(0)
    finally:
        eng.close()


@pytest.mark.parametrize("bits", [4, 3])
def test_expert_pool_interface(have_gpu, bits):
    """The pool over the all-resident store: every record a member, no reads
    to plan, addr(rid) = store base + rid * stride with the kind tag in bits
    62-63 (residency.rs:437-451), and the bytes at that address are the
    record the store holds for (layer, expert)."""
    cfg = presets.tiny(mtp=1)
    eng = Engine(cfg, experts=bits, drafts=0, max_t=32)
    try:
        E = cfg.num_experts
        n_rec = (cfg.num_hidden_layers + 1) * E
        kind = {4: 0, 3: 1, 2: 2}[bits]
        assert eng.L.chk_pool_slots(eng.handle) == n_rec
        assert eng.L.chk_pool_budget(eng.handle) == n_rec
        assert eng.L.chk_pool_resident(eng.handle) == n_rec
        assert eng.L.chk_pool_is_member(eng.handle, n_rec - 1) == 1
        assert eng.L.chk_pool_is_member(eng.handle, n_rec) == 0
        rids = [0, 5, E + 3, n_rec - 1]
        assert eng.pool_acquire(rids, step=7) == []
        assert eng.pool_plan_reads(rids) == (0, len(rids))
        eng.pool_finish(rids)
        with pytest.raises(EngineError, match="out of range"):
            eng.pool_acquire([n_rec], step=8)
        base, stride = eng.pool_store(kind)
        assert stride == eng.L.chk_record_stride(eng.handle, bits)
        assert eng.L.chk_pool_bytes(eng.handle) == n_rec * stride
        tag = {0: 0, 1: 1 << 63, 2: 1 << 62}[kind]
        for rid in rids:
            assert eng.pool_kind(rid) == kind
            addr = eng.pool_addr(rid)
            assert addr == (base + rid * stride) | tag
            b2, off = eng.pool_buf(rid)
            assert (b2, off) == (base, rid * stride)
            # read the record through its pool address (a plain device copy)
            n = stride // 4
            dst = empty_dev((n,))
            check(lib().chk_copy_f32(dst.data_ptr(), addr & ~tag, n, None))
            got = to_host(dst).view(np.uint8)
            layer, e = divmod(rid, E)
            np.testing.assert_array_equal(got, eng.expert_record(layer, e, bits))
        eng.pool_set_kind(rids[0], kind)
        other = {0: 1, 1: 2, 2: 1}[kind]
        with pytest.raises(EngineError, match="low-bit store of that kind not attached"):
            eng.pool_set_kind(rids[0], other)
        if kind:
            # a record switched to 4-bit moves to the 4-bit store, untagged
            b4, s4 = eng.pool_store(0)
            eng.pool_set_kind(rids[1], 0)
            assert eng.pool_kind(rids[1]) == 0
            assert eng.pool_addr(rids[1]) == b4 + rids[1] * s4
            assert eng.pool_buf(rids[1]) == (b4, rids[1] * s4)
            assert eng.L.chk_pool_bytes(eng.handle) == (n_rec - 1) * stride + s4
            eng.pool_set_kind(rids[1], kind)
            assert eng.pool_addr(rids[1]) == (base + rids[1] * stride) | tag
    finally:
        eng.close()
