"""GPU tests of the packed-store loader (chk_engine_load_store; Gpu::load
over Packed::open, gpu/load.rs:8-19, packed.rs:66-231): an engine loaded
from a store written in the reference's format (tests/store_writer.py) from
the synthetic weights holds the same bytes in HBM as the engine that
generates them, and decodes identically (bit for bit), including a store
whose dense.bin order and record field order differ from the engine's own
layout; a store lacking a tensor is refused by name."""

from __future__ import annotations

import json

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import EngineError
from cherenkov_amd.engine import Engine
from tests.store_writer import write_store

pytestmark = pytest.mark.gpu


def decode_trace(eng, prompt, n):
    nxt, dr = eng.prefill_chunk(prompt)
    out = [(nxt, dr, eng.logits_row(0).copy())]
    tok = nxt
    for _ in range(n):
        r = eng.step_rows([tok])
        out.append((r[0], None, eng.logits_row(0).copy()))
        eng.commit(1)
        tok = r[0]
    return out


@pytest.mark.parametrize("layout", ["native", "permuted"])
def test_store_engine_equals_generated_engine(have_gpu, tmp_path, layout):
    cfg = presets.tiny(mtp=1)
    order = None if layout == "native" else ("down_w", "gate_w", "up_w", "down_b", "down_s", "up_b", "up_s",
                                             "gate_b", "gate_s")
    path = write_store(cfg, tmp_path / "packed", shuffle_dense=layout != "native", field_order=order)
    a = Engine.load_store(path, experts=4, drafts=2, max_t=128)
    b = Engine(cfg, experts=4, drafts=2, max_t=128)
    try:
        assert a.cfg.hidden_size == cfg.hidden_size
        for layer, e in [(0, 0), (2, 9), (3, 15), (cfg.num_hidden_layers, 4)]:
            np.testing.assert_array_equal(a.expert_record(layer, e, 4), b.expert_record(layer, e, 4))
        ma, mb = a.memory_stats(), b.memory_stats()
        assert ma["dense"] == mb["dense"] and ma["experts"] == mb["experts"]
        rng = np.random.default_rng(950)
        prompt = rng.integers(0, cfg.vocab_size, size=20).tolist()
        ta, tb = decode_trace(a, prompt, 6), decode_trace(b, prompt, 6)
        for i, ((na, da, la), (nb, db, lb)) in enumerate(zip(ta, tb)):
            assert (na, da) == (nb, db), f"step {i}"
            np.testing.assert_array_equal(la, lb, err_msg=f"step {i} logits")
    finally:
        a.close()
        b.close()


def test_store_lowbit_experts_repacked_from_store(have_gpu, tmp_path):
    cfg = presets.tiny(mtp=0)
    path = write_store(cfg, tmp_path / "packed")
    a = Engine.load_store(path, experts=3, drafts=0, max_t=64)
    b = Engine(cfg, experts=3, drafts=0, max_t=64)
    try:
        for layer, e in [(0, 1), (3, 14)]:
            np.testing.assert_array_equal(a.expert_record(layer, e, 3), b.expert_record(layer, e, 3))
        assert a.step(5) == b.step(5)
        np.testing.assert_array_equal(a.logits_row(0), b.logits_row(0))
    finally:
        a.close()
        b.close()


def test_store_missing_tensor_is_named(have_gpu, tmp_path):
    cfg = presets.tiny(mtp=0)
    path = write_store(cfg, tmp_path / "packed")
    m = json.loads((path / "manifest.json").read_text())
    gone = "language_model.model.layers.1.linear_attn.in_proj_z.scales"
    m["dense"] = [d for d in m["dense"] if d["name"] != gone]
    (path / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(EngineError, match=f'dense tensor "{gone}" not in manifest'):
        Engine.load_store(path, experts=4, drafts=0, max_t=64)


def test_store_negative_ngram_offset_is_refused(have_gpu, tmp_path):
    """A store whose n-gram head offsets hold -1 (an I64 tensor) is refused
    with the loader's message before any kernel reads the table: the
    offset is not wrapped into a huge unsigned row."""
    cfg = presets.with_ple(presets.tiny(mtp=0), layer=2)
    path = write_store(cfg, tmp_path / "packed")
    m = json.loads((path / "manifest.json").read_text())
    ent = [d for d in m["dense"] if d["name"].endswith(".ngram_heads_offsets")]
    assert len(ent) == 1
    with open(path / "dense.bin", "r+b") as fh:
        fh.seek(ent[0]["offset"])
        fh.write(np.array([-1], np.int64).tobytes())
    with pytest.raises(EngineError, match="n-gram heads exceed the table"):
        Engine.load_store(path, experts=4, drafts=0, max_t=64)
