"""Cumulative routed-expert activity (Gpu::expert_activity, src/qwen4_exp/
gpu/activity.rs:11-110) on the GPU: every prefill and decode row adds its
top-k experts' selected rows and one lookup per distinct expert and layer
(a cache hit: the store is resident), trunk layers and the MTP layer alike,
counted whether or not the rows are later committed."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Engine

pytestmark = pytest.mark.gpu


def test_activity_counts_prefill_and_decode_rows(have_gpu):
    cfg = presets.tiny(mtp=1)
    L, E, k = cfg.num_hidden_layers, cfg.num_experts, cfg.num_experts_per_tok
    eng = Engine(cfg, experts=4, drafts=2, max_t=128)
    try:
        act0, _ = eng.expert_activity()
        assert act0.shape == (L + 1, E, 6) and not act0.any()
        prompt = np.random.default_rng(90).integers(0, cfg.vocab_size, size=20).tolist()
        nxt, dr = eng.prefill_chunk(prompt)
        act1, sec = eng.expert_activity()
        assert sec > 0
        # every prompt row picks k distinct experts in each trunk layer and
        # in the MTP layer (its pass runs over every prompt row)
        assert (act1[:, :, 0].sum(axis=1) == 20 * k).all()
        hits = act1[:, :, 1]
        assert ((hits >= 1) == (act1[:, :, 0] >= 1)).all() and hits.max() == 1
        assert not act1[:, :, 2:].any()
        # one committed decode row: each trunk layer's increment is its routes
        eng.step_rows([nxt])
        act2, _ = eng.expert_activity()
        d = act2 - act1
        for layer in range(L):
            ids, _ = eng.last_routes(layer, 0)
            want = np.zeros(E, np.uint64)
            want[np.asarray(ids, np.int64)] = 1
            np.testing.assert_array_equal(d[layer, :, 0], want, f"layer {layer}")
            np.testing.assert_array_equal(d[layer, :, 1], want)
        assert not d[L].any()  # no MTP pass in a plain step
        # a 3-row verify step counts all rows, rolled back or not
        eng.commit(1)
        eng.step_rows([nxt, dr, dr], snap=True)
        eng.commit(1)
        act3, _ = eng.expert_activity()
        assert ((act3 - act2)[:L, :, 0].sum(axis=1) == 3 * k).all()
    finally:
        eng.close()


def test_throttle_probe_and_working_set(have_gpu):
    eng = Engine(presets.tiny(mtp=0), experts=4, drafts=0, max_t=32)
    try:
        ms = eng.throttle_ms()
        assert 0.0 < ms < 1000.0
        gb = eng.working_set_limit_gb()
        assert gb > eng.allocated_gb() > 0.0
    finally:
        eng.close()
