"""The prefill attention's work plan (pf_flash_plan, host code in
csrc/prefill.hip, through chk_pf_flash_plan; no device call): per kv head,
row block rb of a T-row chunk at pos0 needs tiles 0 .. (pos0 + min(16 rb +
15, T - 1)) / 32.  Every plan must cover each (row block, tile) step exactly
once, flag exactly the pieces of split row blocks as partials (whole blocks
write their output directly), list each split block's pieces in
consecutive slots with a merge entry, and bound its buffers (slots <= 2 W,
segments <= 6 per workgroup); where the blocks' work is uneven it must
deal it in near-equal shares."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cherenkov_amd import abi

MAXSEG = 6
NONE = 0xFFFFFFFF


def plan(T, pos0, max_wg):
    L = abi.lib()
    R = (T + 15) // 16
    cap = (R + 1) * MAXSEG * 4
    seg = np.zeros(cap, np.uint32)
    merge = np.zeros(4 * (R + 1), np.uint32)
    W, nslots, nmerge = C.c_uint32(), C.c_uint32(), C.c_uint32()
    abi.check(L.chk_pf_flash_plan(T, pos0, max_wg, C.byref(W), C.byref(nslots), seg.ctypes.data, seg.size,
                                  merge.ctypes.data, merge.size, C.byref(nmerge)))
    return W.value, nslots.value, seg[: W.value * MAXSEG * 4].reshape(W.value, MAXSEG, 4), merge[: 4 * nmerge.value].reshape(-1, 4)


def tiles(T, pos0):
    R = (T + 15) // 16
    return [(pos0 + min(16 * rb + 15, T - 1)) // 32 + 1 for rb in range(R)]


@pytest.mark.parametrize("T", [1, 5, 16, 17, 90, 128, 500, 2047, 2048, 4096])
@pytest.mark.parametrize("pos0", [0, 31, 2048, 30000])
@pytest.mark.parametrize("max_wg", [1, 3, 128])
def test_plan_covers_every_step_once(T, pos0, max_wg):
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built (run __graft_entry__.build())")
    W, nslots, seg, merge = plan(T, pos0, max_wg)
    tl = tiles(T, pos0)
    cover = [np.zeros(n, int) for n in tl]
    pieces = {}
    shares = []
    for k in range(W):
        share = 0
        for s in range(MAXSEG):
            rb, ta, tb, slot = (int(v) for v in seg[k, s])
            if rb == NONE:
                break
            assert rb < len(tl) and ta < tb <= tl[rb]
            cover[rb][ta:tb] += 1
            whole = ta == 0 and tb == tl[rb]
            assert whole == (slot == NONE), (rb, ta, tb, slot)
            if not whole:
                pieces.setdefault(rb, []).append(slot)
            share += tb - ta
        shares.append(share)
    assert all((c == 1).all() for c in cover)
    assert nslots <= 2 * max(1, min(len(tl), max_wg)) or not pieces
    assert {int(m[0]): (int(m[1]), int(m[2])) for m in merge} == {
        rb: (min(sl), len(sl)) for rb, sl in pieces.items()}
    for rb, sl in pieces.items():
        assert sorted(sl) == list(range(min(sl), min(sl) + len(sl)))
    if pieces:  # a split plan deals near-equal shares
        assert max(shares) <= sum(tl) / W + 2


def test_plan_halves_the_longest_share_at_the_bench_shape():
    """2048 rows at position 0, 128 workgroups per kv head: the last row
    block needs 64 tiles, the average is 32.5; the plan's longest share is
    33 tiles (the whole-block form's would be 64)."""
    if not abi.LIB_PATH.exists():
        pytest.skip("libcherenkov.so not built (run __graft_entry__.build())")
    W, _, seg, merge = plan(2048, 0, 128)
    assert W == 128 and len(merge) > 0
    share = [sum(int(g[2]) - int(g[1]) for g in seg[k] if g[0] != NONE) for k in range(W)]
    assert max(share) == 33 and sum(share) == sum(tiles(2048, 0))
