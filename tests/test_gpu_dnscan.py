"""GPU parity of the prefill's gated delta rule (linear_attention's
recurrence, /root/reference/src/qwen4_exp/cpu.rs:745-812; the reference
prefill runs it row by row, src/qwen4_exp/gpu/prefill/deltanet.rs:80-95).

The chunked scan (64 rows per chunk, MFMA products) and the sequential
kernel are checked against the oracle's delta_head_step applied row by row
(ragged chunk counts, GQA, a non-zero starting state, decays that underflow
to 0), and the chunked scan against the sequential kernel at the 80B shape
(32 value heads, 2048 and 4096 rows).  There is no reference vector for the
chunked form (the reference has none); chunked == sequential is the
invariant the blueprint names for it.
"""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd.abi import check, lib
from oracle.oracle import delta_head_step
from tests.gpu_util import assert_close, empty_dev, to_dev, to_host

pytestmark = pytest.mark.gpu

DK = 128


def make_inputs(seed, T, nk, nv, dv=128, tiny_decay=False):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, nk, DK))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    q *= DK**-0.5
    k = rng.standard_normal((T, nk, DK))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, nv, dv))
    conv = np.concatenate([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], axis=1).astype(np.float32)
    decay = rng.uniform(0.3, 1.0, (T, nv)).astype(np.float32)
    if tiny_decay:
        decay[rng.random((T, nv)) < 0.05] = 1e-30
        decay[rng.random((T, nv)) < 0.02] = 0.0
    beta = rng.uniform(0.0, 1.0, (T, nv)).astype(np.float32)
    state = (0.5 * rng.standard_normal((nv, dv, DK))).astype(np.float32)
    return conv, decay, beta, state


def gpu_scan(conv, decay, beta, state, nk, nv, dv, chunked):
    T = conv.shape[0]
    dstate = to_dev(state.copy())
    dy = empty_dev((T, nv * dv))
    check(lib().chk_dn_scan(to_dev(conv).data_ptr(), to_dev(decay).data_ptr(), to_dev(beta).data_ptr(),
                            dstate.data_ptr(), dy.data_ptr(), T, nk, nv, DK, dv, int(chunked), None))
    return to_host(dy), to_host(dstate)


def oracle_scan(conv, decay, beta, state, nk, nv, dv, heads=None):
    """Row-by-row recurrence with the oracle's delta_head_step; the
    oracle's state is [dk][dv], the engine's [dv][dk]."""
    T = conv.shape[0]
    qk = nk * DK
    heads = range(nv) if heads is None else heads
    y = np.zeros((T, nv * dv), np.float32)
    out_state = state.copy()
    for h in heads:
        hk = h // (nv // nk)
        s = state[h].T.copy()
        for t in range(T):
            q = conv[t, hk * DK:(hk + 1) * DK]
            k = conv[t, qk + hk * DK:qk + (hk + 1) * DK]
            v = conv[t, 2 * qk + h * dv:2 * qk + (h + 1) * dv]
            s, y[t, h * dv:(h + 1) * dv] = delta_head_step(s, q, k, v, float(decay[t, h]), float(beta[t, h]))
        out_state[h] = s.T
    return y, out_state


def tight(got, ref, label, frac=1e-3):
    """A bar well inside the north star's: both scans compute the same f32
    recurrence, so a wrong index or decay shows as an error far above it."""
    err = float(np.abs(got.astype(np.float64) - ref).max())
    bound = frac * max(1.0, float(np.abs(ref).max()))
    assert err <= bound, f"{label}: max-abs {err:.3e} > {bound:.3e}"


@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 130, 257])
@pytest.mark.parametrize("chunked", [0, 1])
def test_scan_matches_oracle(have_gpu, T, chunked):
    nk, nv, dv = 2, 4, 128
    conv, decay, beta, state = make_inputs(100 + T, T, nk, nv, dv, tiny_decay=T > 64)
    y, s = gpu_scan(conv, decay, beta, state, nk, nv, dv, chunked)
    ry, rs = oracle_scan(conv, decay, beta, state, nk, nv, dv)
    assert_close(y, ry, f"y T={T} chunked={chunked}")
    assert_close(s, rs, f"state T={T} chunked={chunked}")
    tight(y, ry, f"y T={T} chunked={chunked}")
    tight(s, rs, f"state T={T} chunked={chunked}")


def test_scan_zero_state_closed_form(have_gpu):
    """From a zero state the first row's output is beta (k . q) v (the
    delta rule's textbook first step), whatever the decay."""
    nk, nv, dv = 1, 2, 128
    conv, decay, beta, _ = make_inputs(7, 64, nk, nv, dv)
    state = np.zeros((nv, dv, DK), np.float32)
    y, _ = gpu_scan(conv, decay, beta, state, nk, nv, dv, 1)
    q, k = conv[0, :DK].astype(np.float64), conv[0, DK:2 * DK].astype(np.float64)
    for h in range(nv):
        v = conv[0, 2 * DK + h * dv:2 * DK + (h + 1) * dv].astype(np.float64)
        ref = beta[0, h] * (k @ q) * v
        tight(y[0, h * dv:(h + 1) * dv], ref, f"row 0 head {h}", 1e-5)


@pytest.mark.parametrize("T", [2048, 4096])
def test_chunked_equals_sequential_full_shape(have_gpu, T):
    """The 80B shape's DeltaNet (16 key / 32 value heads of 128): chunked
    against the sequential kernel over every head, and heads 0 and 31
    against the oracle."""
    nk, nv, dv = 16, 32, 128
    conv, decay, beta, state = make_inputs(2026 + T, T, nk, nv, dv, tiny_decay=True)
    y1, s1 = gpu_scan(conv, decay, beta, state, nk, nv, dv, 1)
    y0, s0 = gpu_scan(conv, decay, beta, state, nk, nv, dv, 0)
    assert_close(y1, y0, f"y T={T}")
    assert_close(s1, s0, f"state T={T}")
    tight(y1, y0, f"y T={T}")
    tight(s1, s0, f"state T={T}")
    if T == 2048:
        heads = [0, nv - 1]
        ry, rs = oracle_scan(conv, decay, beta, state, nk, nv, dv, heads=heads)
        for h in heads:
            cols = slice(h * dv, (h + 1) * dv)
            tight(y1[:, cols], ry[:, cols], f"y head {h}")
            tight(s1[h], rs[h], f"state head {h}")
