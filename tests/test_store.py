"""The packed-store reader without a GPU: a store written in the
reference's format (tests/store_writer.py: config.json, manifest.json,
dense.bin, experts.bin) yields the model's ChkConfig through
chk_store_config, and malformed stores are refused with the reference's
messages (manifest.rs:67-110, config.rs:93-122, packed.rs:75-90)."""

from __future__ import annotations

import ctypes as C
import json

import pytest

from cherenkov_amd import abi, presets
from tests.store_writer import write_store


def store_config(path):
    cfg = abi.ChkConfig()
    rc = abi.lib().chk_store_config(str(path).encode(), C.byref(cfg))
    return rc, cfg, abi.lib().chk_last_error().decode()


@pytest.fixture(scope="module")
def tiny_store(tmp_path_factory):
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built")
    cfg = presets.tiny(mtp=1)
    return cfg, write_store(cfg, tmp_path_factory.mktemp("store") / "packed")


def test_store_config_matches_the_model(tiny_store):
    cfg, path = tiny_store
    rc, got, err = store_config(path)
    assert rc == 0, err
    for k, _ in cfg._fields_:
        if k != "seed":
            assert getattr(got, k) == getattr(cfg, k), k
    # a model directory whose packed files sit in packed/ works the same
    rc, got2, err = store_config(path.parent)
    assert rc == 0, err
    assert got2.hidden_size == cfg.hidden_size


def test_store_config_with_a_ple_layer(tmp_path):
    """ple_layer_ids, the PLE widths and the manifest's n-gram row group
    reach the config (the synthetic table's head_rows is not a store
    field)."""
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built")
    cfg = presets.with_ple(presets.tiny(mtp=0), layer=2, group=8)
    path = write_store(cfg, tmp_path / "s")
    rc, got, err = store_config(path)
    assert rc == 0, err
    for k, _ in cfg._fields_:
        if k not in ("seed", "ngram_head_rows"):
            assert getattr(got, k) == getattr(cfg, k), k
    assert got.ngram_group == 8


@pytest.mark.parametrize("case,msg", [
    ("row_bytes", "n-gram row layout is inconsistent"),
    ("no_ngram", "manifest has no n-gram layout"),
    ("no_embed_dim", "ple_embed_dim"),
])
def test_malformed_ple_stores_are_refused(tmp_path, case, msg):
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built")
    cfg = presets.with_ple(presets.tiny(mtp=0), layer=2)
    path = write_store(cfg, tmp_path / "s")
    edits = {
        "row_bytes": ("manifest.json", lambda d: d["ngram"].update(row_bytes=d["ngram"]["row_bytes"] + 4)),
        "no_ngram": ("manifest.json", lambda d: d.pop("ngram")),
        "no_embed_dim": ("config.json", lambda d: d["text_config"].pop("ple_embed_dim")),
    }
    fname, fn = edits[case]
    _edit(path, fname, fn)
    rc, _, err = store_config(path)
    assert rc != 0 and msg in err, err


def _edit(path, fname, fn):
    p = path / fname
    d = json.loads(p.read_text())
    fn(d)
    p.write_text(json.dumps(d))


@pytest.mark.parametrize("case,msg", [
    ("version", "unsupported packed layout version 2"),
    ("group", "expert group size must be 64"),
    ("prefixes", "expert layer count does not match layer prefixes"),
    ("mtp_records", "no expert records for mtp.layers.0.mlp.switch_mlp"),
    ("model_type", "unsupported model_type llama"),
    ("layer_types", "layer_types length mismatch"),
    ("gate", "output_gate_type must be sigmoid"),
    ("huge", "integer above 2^53"),
    ("stride0", "expert record size must be nonzero"),
    ("field", "expert record field outside the record"),
])
def test_malformed_stores_are_refused(tmp_path, case, msg):
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built")
    cfg = presets.tiny(mtp=1, layers=4)
    path = write_store(cfg, tmp_path / "s")
    edits = {
        "version": ("manifest.json", lambda d: d.update(version=2)),
        "group": ("manifest.json", lambda d: d["experts"].update(group=32)),
        "prefixes": ("manifest.json", lambda d: d["experts"]["layer_prefixes"].pop()),
        "mtp_records": ("manifest.json", lambda d: (d["experts"]["layer_prefixes"].__setitem__(-1, "mtp.layers.1.x"))),
        "model_type": ("config.json", lambda d: d.update(model_type="llama")),
        "layer_types": ("config.json", lambda d: d["text_config"]["layer_types"].pop()),
        "gate": ("config.json", lambda d: d["text_config"].update(output_gate_type="silu")),
        "huge": ("manifest.json", lambda d: d["experts"].update(record_stride=2.0 ** 64)),
        "stride0": ("manifest.json", lambda d: d["experts"].update(record_bytes=0, record_stride=0)),
        # a field that starts inside the record and runs past its end
        "field": ("manifest.json", lambda d: d["experts"].update(down_b=d["experts"]["record_bytes"] - 2)),
    }
    fname, fn = edits[case]
    _edit(path, fname, fn)
    rc, _, err = store_config(path)
    assert rc != 0 and msg in err, err


def test_reference_fixture_config_is_parsed(tmp_path):
    """The reference's own qwen4_exp test checkpoint config (tests/fixtures/
    qwen4_exp/config.json, committed as tests/golden/qwen4_exp_fixture_config.json)
    in a store of its shape: chk_store_config reads every field the engine
    uses (config.rs:9-126: layer_types, the hyper-connection, indexer, MTP
    and PLE settings, rope_parameters.rope_theta, eos_token_id) to the
    values the fixture states, and the n-gram row group from the manifest."""
    import shutil
    from pathlib import Path

    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built")
    want = presets.qwen4_exp_fixture()
    path = write_store(want, tmp_path / "s")
    golden = Path(__file__).resolve().parent / "golden" / "qwen4_exp_fixture_config.json"
    shutil.copyfile(golden, path / "config.json")
    rc, got, err = store_config(path)
    assert rc == 0, err
    for k, _ in want._fields_:
        if k not in ("seed", "ngram_head_rows"):
            assert getattr(got, k) == getattr(want, k), k
    t = json.loads(golden.read_text())["text_config"]
    assert got.hidden_size == t["hidden_size"] == 256
    assert got.linear_num_value_heads == t["linear_num_value_heads"] == 48
    assert got.vocab_size == t["vocab_size"] == 248320
    assert got.ple_layer == t["ple_layer_ids"][0] == 2
    assert got.indexer_budget == t["indexer_budget"] == 2048
    assert got.rope_theta == t["rope_parameters"]["rope_theta"]
    assert got.eos_token_id == t["eos_token_id"]
    assert got.ngram_group == 16
