"""The prefix cache's host rules without a GPU (native prefix_cache.cpp):
the reference's own unit tests (tests/unit/prefix_cache.rs:3-44)."""

from __future__ import annotations

import pytest

from cherenkov_amd import abi

pytestmark = pytest.mark.skipif(not abi.LIB_PATH.exists(), reason="libcherenkov.so not built")

from cherenkov_amd.abi import EngineError  # noqa: E402
from cherenkov_amd.prefix_cache import chunk_len, matches, pacing_sample  # noqa: E402


def test_matching_checks_mtp_lookahead_and_exact_prompt_state():
    assert matches([1, 2], 3, False, [1, 2, 3, 4])
    assert not matches([1, 2], 3, False, [1, 2, 9])
    assert not matches([1, 2], 3, False, [1, 2])
    assert matches([1, 2], 3, True, [1, 2])
    assert matches([1, 2], None, False, [1, 2, 9])
    assert not matches([1, 2], None, True, [1, 9, 2])
    assert not matches([1, 2], None, True, [1])


@pytest.mark.parametrize("remaining,capacity,quantum,expected", [
    (275, 4096, 128, 92), (25740, 4096, 128, 128), (25740, 4096, 1024, 990), (25740, 4096, 4096, 3678),
    (275, 64, 1024, 55), (17, 4096, 4096, 17),
])
def test_chunks_respect_quantum_capacity_and_prompt_boundaries(remaining, capacity, quantum, expected):
    assert chunk_len(remaining, capacity, quantum) == expected


@pytest.mark.parametrize("remaining,capacity,quantum", [(10, 0, 128), (10, 128, 0), (0, 128, 128)])
def test_chunk_len_rejects_empty_work(remaining, capacity, quantum):
    with pytest.raises(EngineError, match="prefill chunk requires tokens and capacity"):
        chunk_len(remaining, capacity, quantum)


@pytest.mark.parametrize("remaining,capacity,engine,eligible", [
    (4096, 4096, True, True), (25740, 4096, True, True), (4, 4096, True, False), (1000, 4096, True, False),
    (4096, 512, True, False), (4096, 4096, False, False),
])
def test_pacing_ignores_tails_memory_limits_and_the_small_row_path(remaining, capacity, engine, eligible):
    assert pacing_sample(remaining, capacity, 1024, engine) == eligible
