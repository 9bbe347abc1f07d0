"""The engine under a server memory budget (Gpu::load_bounded,
src/qwen4_exp/gpu/load.rs:12-63, as src/server.rs:90-97 calls it): every
device buffer counts against memory_bytes - reserve, the load keeps room
for the prefill scratch of prefill_rows rows beside the resident store
(budget.rs:14-40), and the prefill then runs in chunks of those rows."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import EngineError
from cherenkov_amd.engine import Engine
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu


def allocated(eng) -> int:
    return int(round(eng.allocated_gb() * 1e9))


def test_bounded_load_and_prefill(have_gpu):
    cfg = presets.tiny(mtp=0)
    prompt = np.random.default_rng(91).integers(0, cfg.vocab_size, size=40).tolist()
    free = Engine(cfg, experts=4, drafts=0, max_t=64)
    try:
        fixed = allocated(free)
        nxt_ref, _ = free.prefill_chunk(prompt)
        ref = free.logits_row(0).copy()
        scratch64 = allocated(free) - fixed  # 64 rows (max_t) of prefill scratch
    finally:
        free.close()
    assert scratch64 > 0
    # no room for the prefill scratch beside the store
    with pytest.raises(EngineError, match="explicit expert pool exceeds server memory budget"):
        Engine.load_bounded(cfg, reserve=0, memory_bytes=fixed + scratch64 // 8, prefill_rows=64, max_t=64)
    # the reserve is taken off the budget
    with pytest.raises(EngineError, match="explicit expert pool exceeds server memory budget"):
        Engine.load_bounded(cfg, reserve=scratch64, memory_bytes=fixed + scratch64 + 4096, prefill_rows=64, max_t=64)
    # room for 64 rows: one chunk, the same logits as the unbounded engine
    eng = Engine.load_bounded(cfg, reserve=4096, memory_bytes=fixed + scratch64 + 8192, prefill_rows=64, max_t=64)
    try:
        assert eng.prefill_rows_fit() >= 40
        nxt, _ = eng.prefill_chunk(prompt)
        np.testing.assert_array_equal(eng.logits_row(0), ref)
        assert nxt == nxt_ref
        assert allocated(eng) <= fixed + scratch64 + 4096
    finally:
        eng.close()
    # room for 16 rows: the 40-token prompt runs in chunks of 16
    eng = Engine.load_bounded(cfg, reserve=0, memory_bytes=fixed + scratch64 // 2, prefill_rows=16, max_t=64)
    try:
        assert 16 <= eng.prefill_rows_fit() < 64
        eng.prefill_chunk(prompt)
        assert_close(eng.logits_row(0), ref, "prefill in 16-row chunks", abs_frac=1e-3, min_cos=0.99999)
        assert allocated(eng) <= fixed + scratch64 // 2
    finally:
        eng.close()
