"""The committed tiny-model fixtures (tests/golden/tiny_greedy.json, made by
tests/golden/make_golden.py from the oracle): the oracle must reproduce
them (CPU), and the HIP engine must match them through the C ABI (GPU):
greedy ids exact wherever the margin exceeds 1e-3, the logits' first
values within the north-star float bar, their norm within 1e-3."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "tiny_greedy.json"


@pytest.fixture(scope="module")
def golden():
    return json.loads(GOLDEN.read_text())


def test_oracle_reproduces_golden(golden):
    from tests.golden.make_golden import generate

    now = generate()
    assert now["prompt"] == golden["prompt"]
    for i, (a, b) in enumerate(zip(now["steps"], golden["steps"])):
        assert a["input"] == b["input"] and a["argmax"] == b["argmax"] and a["top5"] == b["top5"], f"pos {i}"
        assert abs(a["sum"] - b["sum"]) <= 1e-5 * max(1.0, abs(b["sum"])), f"pos {i}"
        assert abs(a["sumsq"] - b["sumsq"]) <= 1e-5 * b["sumsq"], f"pos {i}"
        assert np.allclose(a["head"], b["head"], rtol=1e-5, atol=1e-6), f"pos {i}"


@pytest.mark.gpu
def test_engine_matches_golden(have_gpu, golden):
    from cherenkov_amd import presets
    from cherenkov_amd.engine import Engine

    eng = Engine(presets.tiny(), experts=4, drafts=0, max_t=128)
    try:
        for i, s in enumerate(golden["steps"]):
            out = eng.step_rows([s["input"]])
            logits = np.asarray(eng.logits_row(0), dtype=np.float64)
            eng.commit(1)
            if s["margin"] > 1e-3:
                assert out[0] == s["argmax"], f"pos {i}: {out[0]} vs {s['argmax']}"
            head = np.asarray(s["head"])
            scale = max(1.0, float(np.max(np.abs(logits))))
            assert np.max(np.abs(logits[:8] - head)) <= 2e-2 * scale, f"pos {i}"
            assert abs(np.sqrt(np.sum(logits ** 2)) - np.sqrt(s["sumsq"])) <= 1e-3 * np.sqrt(s["sumsq"]), f"pos {i}"
    finally:
        eng.close()
