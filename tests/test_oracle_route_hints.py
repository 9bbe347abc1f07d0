"""The oracle's near-tie route hints (test-side; no counterpart in the
reference).  Two f32 implementations of forward_token agree to rounding, so
where a layer's k-th and (k+1)-th router probabilities are within rounding
of each other they may route differently; the GPU parity tests hand the
engine's routing to the oracle as a hint, which the oracle takes only
where it departs from its own top-k (src/qwen4_exp/cpu.rs:509-525) by
experts within the tolerance of the k-th probability.  Pinned here: a hint
equal to the oracle's own set changes nothing, bit for bit; a swap of the
k-th for the (k+1)-th expert is taken exactly when the tolerance covers
their gap, and then changes the routing and the logits; a hint that moves a
far expert, or repeats an expert, is refused.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from oracle.oracle import OracleModel

TOKEN = 77


@pytest.fixture(scope="module")
def model():
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    st = m.new_state()
    logits = st.forward_token(TOKEN)
    routes = [st.last_routes(layer) for layer in range(cfg.num_hidden_layers)]
    return cfg, m, logits, routes


def rank(probs: np.ndarray) -> np.ndarray:
    """Experts by probability descending, index ascending on equal values."""
    return np.lexsort((np.arange(probs.size), -probs.astype(np.float64)))


def run(m, hints, tol):
    st = m.new_state()
    st.route_hints(np.asarray(hints, np.uint32), tol)
    logits = st.forward_token(TOKEN)
    return st, logits


def test_own_routing_records_top_k(model):
    cfg, _, _, routes = model
    k = cfg.num_experts_per_tok
    for ids, probs in routes:
        assert np.array_equal(ids, rank(probs)[:k])
        assert abs(float(probs.sum()) - 1.0) < 1e-5


def test_same_set_changes_nothing(model):
    cfg, m, logits, routes = model
    own = np.stack([ids for ids, _ in routes])
    st, got = run(m, own[:, ::-1], 1.0)  # same sets, other order
    assert st.route_swaps == 0
    assert np.array_equal(got, logits)


def test_boundary_swap_taken_only_within_tolerance(model):
    cfg, m, logits, routes = model
    k = cfg.num_experts_per_tok
    ids, probs = routes[0]
    order = rank(probs)
    pk, pk1 = float(probs[order[k - 1]]), float(probs[order[k]])
    gap = (pk - pk1) / pk
    assert gap > 0
    hint = np.array(ids)
    hint[list(ids).index(order[k - 1])] = order[k]
    # below the gap: refused, bit-exact
    st, got = run(m, hint[None, :], gap * 0.99)
    assert st.route_swaps == 0 and np.array_equal(got, logits)
    # covering the gap: taken, ranked by the oracle's own probabilities
    st, got = run(m, hint[None, :], gap * 1.01)
    assert st.route_swaps == 1
    taken, _ = st.last_routes(0)
    want = [e for e in order[: k + 1] if e != order[k - 1]]
    assert list(taken) == want
    assert not np.array_equal(got, logits)
    # later layers had no hint and ran their own top-k on the changed input
    for layer in range(1, cfg.num_hidden_layers):
        ids_l, probs_l = st.last_routes(layer)
        assert np.array_equal(ids_l, rank(probs_l)[:k])


def test_far_or_repeated_experts_refused(model):
    cfg, m, logits, routes = model
    k = cfg.num_experts_per_tok
    ids, probs = routes[0]
    order = rank(probs)
    pk = float(probs[order[k - 1]])
    gap = (pk - float(probs[order[k]])) / pk
    # the top expert (far above the k-th) out, the (k+1)-th in
    top_gap = (float(probs[order[0]]) - pk) / pk
    assert top_gap > gap * 1.01
    hint = np.array(ids)
    hint[list(ids).index(order[0])] = order[k]
    st, got = run(m, hint[None, :], gap * 1.01)
    assert st.route_swaps == 0 and np.array_equal(got, logits)
    # an expert twice
    hint = np.array(ids)
    hint[list(ids).index(order[k - 1])] = order[0]
    st, got = run(m, hint[None, :], 10.0)
    assert st.route_swaps == 0 and np.array_equal(got, logits)


def test_hints_are_used_once(model):
    cfg, m, logits, routes = model
    k = cfg.num_experts_per_tok
    ids, probs = routes[0]
    order = rank(probs)
    hint = np.array(ids)
    hint[list(ids).index(order[k - 1])] = order[k]
    st = m.new_state()
    st.route_hints(hint[None, :], 1.0)
    st.forward_token(TOKEN)
    assert st.route_swaps == 1
    st.forward_token(TOKEN)  # no hint for this pass
    assert st.route_swaps == 1
    with pytest.raises(Exception):
        st.route_hints(np.zeros((cfg.num_hidden_layers + 2, k), np.uint32), 1.0)
