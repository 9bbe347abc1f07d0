"""The allocation-free LM head entry point (chk_lm_head_argmax_noalloc)
against chk_lm_head_argmax, through the C ABI: logits bit-identical and
greedy ids equal, on two calls in a row, the second with a smaller input
(fewer rows and a narrower head), so the shared scratch keeps nothing of
the first call that the second could read; and the same call captured into
a graph and replayed on new inputs."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd.abi import EngineError, check, lib
from tests.gpu_util import empty_dev, to_dev, to_host
from tests.numerics import bf16_bits

pytestmark = pytest.mark.gpu


def head(rng, out_dim, in_dim):
    w = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.normal(0, 0.02, size=(out_dim, in_dim // 64)))
    b = bf16_bits(rng.normal(0, 0.01, size=(out_dim, in_dim // 64)))
    return w, s, b


def run(fn, w, s, b, out_dim, in_dim, x):
    nb = x.shape[0]
    dw, ds, db, dx = to_dev(w), to_dev(s), to_dev(b), to_dev(x)
    logits = empty_dev((nb, out_dim))
    ids = empty_dev((nb,), np.uint32)
    check(fn(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), out_dim, in_dim, dx.data_ptr(), nb, logits.data_ptr(),
             ids.data_ptr(), None))
    return to_host(logits), to_host(ids).view(np.uint32)


def test_noalloc_lm_head_matches_allocating_entry_point(have_gpu):
    L = lib()
    rng = np.random.default_rng(4242)
    for out_dim, in_dim, nb in ((151936, 2048, 4), (4096, 512, 1)):
        w, s, b = head(rng, out_dim, in_dim)
        x = rng.normal(0, 1, size=(nb, in_dim)).astype(np.float32)
        lg_a, id_a = run(L.chk_lm_head_argmax, w, s, b, out_dim, in_dim, x)
        lg_n, id_n = run(L.chk_lm_head_argmax_noalloc, w, s, b, out_dim, in_dim, x)
        np.testing.assert_array_equal(lg_n, lg_a)
        np.testing.assert_array_equal(id_n, id_a)
        # the greedy rule: lowest index of the maximum
        np.testing.assert_array_equal(id_n, np.argmax(lg_a, axis=1).astype(np.uint32))


def test_noalloc_lm_head_rejects_oversized_batches(have_gpu):
    L = lib()
    rng = np.random.default_rng(1)
    w, s, b = head(rng, 64, 64)
    x = rng.normal(0, 1, size=(5, 64)).astype(np.float32)
    with pytest.raises(EngineError, match="nb must be 1..=4"):
        run(L.chk_lm_head_argmax_noalloc, w, s, b, 64, 64, x)


def test_noalloc_lm_head_under_graph_capture(have_gpu):
    """The entry point captured into a graph on a side stream (after one
    eager call, which resolves the scratch address), replayed twice on new
    inputs written into the captured input buffer, with eager work and
    synchronisations between the replays: every replay equals the
    allocating entry point on the same input, bit for bit."""
    import torch

    L = lib()
    rng = np.random.default_rng(77)
    out_dim, in_dim, nb = 151936, 2048, 2
    w, s, b = head(rng, out_dim, in_dim)
    dw, ds, db = to_dev(w), to_dev(s), to_dev(b)
    dx = to_dev(rng.normal(0, 1, size=(nb, in_dim)).astype(np.float32))
    logits = empty_dev((nb, out_dim))
    ids = empty_dev((nb,), np.uint32)

    def call(stream_ptr):
        return L.chk_lm_head_argmax_noalloc(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), out_dim, in_dim,
                                            dx.data_ptr(), nb, logits.data_ptr(), ids.data_ptr(), stream_ptr)

    check(call(None))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        check(call(torch.cuda.current_stream().cuda_stream))
    for replay in range(2):
        x = rng.normal(0, 1 + replay, size=(nb, in_dim)).astype(np.float32)
        dx.copy_(torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        lg_g, id_g = to_host(logits), to_host(ids).view(np.uint32)
        lg_a, id_a = run(L.chk_lm_head_argmax, w, s, b, out_dim, in_dim, x)
        np.testing.assert_array_equal(lg_g, lg_a, err_msg=f"replay {replay}")
        np.testing.assert_array_equal(id_g, id_a, err_msg=f"replay {replay}")
