"""The drop-in boundary without a GPU: libcherenkov.so loads, exports
every function include/cherenkov/*.h declares, and the Python mirror's
ctypes signatures cover exactly those functions.  No compute calls."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from cherenkov_amd import abi

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^[A-Za-z_][\w \*]*?\b(chk_\w+)\s*\(", re.M)


def header_functions() -> set[str]:
    names = set()
    for h in sorted((ROOT / "include" / "cherenkov").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in DECL.finditer(text):
            if not m.group(0).lstrip().startswith(("static", "CHK_HD", "inline")):
                names.add(m.group(1))
    return names


def test_headers_declare_the_engine_api():
    names = header_functions()
    for n in ("chk_engine_load", "chk_step_rows", "chk_commit", "chk_mtp_draft", "chk_prefill_chunk",
              "chk_q4_matvec", "chk_moe_block", "chk_decode_step", "chk_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built (run __graft_entry__.build())")
    L = C.CDLL(str(abi.LIB_PATH))
    missing = [n for n in sorted(header_functions()) if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_signatures_match_headers():
    declared = header_functions()
    bound = {n for n, _, _ in abi.SIGNATURES}
    assert bound <= declared, f"bound but not declared: {sorted(bound - declared)}"
    assert declared <= bound, f"declared but not bound: {sorted(declared - bound)}"


def test_load_validates_before_touching_the_device():
    """Configs the kernels cannot run are refused by chk_engine_load before
    any device call (so this runs without a GPU): hidden sizes above 4096
    (two 32-input chunks per lane in the batch-1 kernels), hyper-connection
    low ranks past 16 lanes a stream, more than 3 drafts, PLE blocks the
    kernels cannot lay out."""
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built (run __graft_entry__.build())")
    from cherenkov_amd import presets

    L = abi.lib()
    cases = []
    c = presets.tiny()
    c.hidden_size = 4352
    cases.append((c, abi.ChkOptions(4, 0, 64, 0), "hidden size must be at most 4096"))
    c = presets.tiny()
    c.hc_lowrank = 544
    cases.append((c, abi.ChkOptions(4, 0, 64, 0), "hc_lowrank must be a multiple of 32 up to 512"))
    for si in (96, 1088):
        c = presets.tiny()
        c.shared_expert_intermediate_size = si
        cases.append((c, abi.ChkOptions(4, 0, 64, 0), "shared expert width must be a multiple of 64 up to 1024"))
    c = presets.tiny()
    cases.append((c, abi.ChkOptions(4, 4, 64, 0), "drafts must be 0..=3"))
    c = presets.tiny()
    cases.append((c, abi.ChkOptions(5, 0, 64, 0), "expert precision"))
    c = presets.with_ple(presets.tiny(), layer=5)
    cases.append((c, abi.ChkOptions(4, 0, 64, 0), "ple_layer_ids beyond the decoder layers"))
    c = presets.with_ple(presets.tiny(), heads_per_ngram=17)
    cases.append((c, abi.ChkOptions(4, 0, 64, 0), "at most 32 n-gram heads"))
    c = presets.with_ple(presets.tiny(), embed_dim=272)
    cases.append((c, abi.ChkOptions(4, 0, 64, 0), "ple_embed_dim must be a multiple of 64"))
    c = presets.with_ple(presets.tiny(), kernel=2, ngram_size=1)
    cases.append((c, abi.ChkOptions(4, 0, 64, 0), "n-gram orders"))
    for cfg, opt, msg in cases:
        h = C.c_void_p()
        rc = L.chk_engine_load(C.byref(cfg), C.byref(opt), C.byref(h))
        assert rc != 0 and not h.value
        assert msg in L.chk_last_error().decode()


def test_bounded_load_refuses_a_reserve_above_the_budget():
    """Gpu::load_bounded (gpu/load.rs:55-61): a reserve larger than the
    memory budget is refused before any device call."""
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built (run __graft_entry__.build())")
    from cherenkov_amd import presets

    L = abi.lib()
    cfg = presets.tiny()
    opt = abi.ChkOptions(4, 0, 64, 0)
    h = C.c_void_p()
    assert L.chk_engine_load_bounded(C.byref(cfg), C.byref(opt), 2 << 30, 1 << 30, 64, C.byref(h)) != 0
    assert not h.value
    assert "cache exceeds memory budget" in L.chk_last_error().decode()
