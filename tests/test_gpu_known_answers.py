"""GPU runs of the reference's own known-answer cases through the product
kernels (C ABI of include/cherenkov/kernels.h):

  the LM head's greedy argmax — ties resolve to the lowest index across
  the grid stride, a winner in the final partial block, all -inf -> 0
  (tests/unit/qwen4_exp/gpu/sampling.rs:5-40);

  q8 flash-decode attention over the reference test's LCG-23 cache,
  24 q / 2 kv heads x 256, 300 and 2300 tokens, against that test's CPU
  formula with fp16-rounded scales (tests/unit/qwen4_exp/gpu/attention.rs:
  115-200), plus the model's 16/2 shape across chunk boundaries.
"""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd.abi import check, lib
from tests.gpu_util import assert_close, empty_dev, to_dev, to_host
from tests.numerics import bf16_bits
from tests.test_oracle import reference_attention_case

pytestmark = pytest.mark.gpu

NEG_INF_BF16 = 0xFF80


def _head(bias_per_row: np.ndarray, in_dim: int):
    """Q4 rows whose output is exactly bias * sum(x): codes 0, scale 0."""
    out = bias_per_row.size
    w = np.zeros((out, in_dim // 8), np.uint32)
    s = np.zeros((out, in_dim // 64), np.uint16)
    b = np.repeat(bias_per_row.astype(np.uint16)[:, None], in_dim // 64, axis=1)
    return w, s, b


@pytest.mark.parametrize("nb", [1, 2])
def test_lm_head_argmax_ties_partial_blocks(have_gpu, nb):
    # rows per grid stride of the head kernel: 1024 workgroups x 4 waves x 8 rows
    stride = 1024 * 4 * 8
    n = stride + 40
    in_dim = 2048  # every lane holds a chunk: -inf biases never meet a zero x sum
    x = np.ones((nb, in_dim), np.float32)
    x[1:] *= 2.0
    lo, hi = int(bf16_bits(np.float32(-10.0 / in_dim))[0]), int(bf16_bits(np.float32(3.5 / in_dim))[0])
    cases = []
    bias = np.full(n, lo, np.uint16)
    bias[[5, 36, 4097, stride + 5]] = hi
    cases.append((bias, 5))
    bias = np.full(n, NEG_INF_BF16, np.uint16)
    bias[n - 1] = int(bf16_bits(np.float32(-1.0 / in_dim))[0])
    cases.append((bias, n - 1))
    cases.append((np.full(n, NEG_INF_BF16, np.uint16), 0))
    for bias, want in cases:
        w, s, b = _head(bias, in_dim)
        dw, ds, db, dx = to_dev(w), to_dev(s), to_dev(b), to_dev(x)
        logits = empty_dev((nb, n))
        ids = empty_dev((nb,), np.uint32)
        check(lib().chk_lm_head_argmax(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), n, in_dim, dx.data_ptr(), nb,
                                       logits.data_ptr(), ids.data_ptr(), None))
        got = to_host(ids).view(np.uint32)
        assert got.tolist() == [want] * nb
        lg = to_host(logits)
        assert lg[0, want] == (np.float32(-1.0) if want == n - 1 else (np.float32(3.5) if want == 5 else -np.inf))


@pytest.mark.parametrize("t_len", [300, 2300])
def test_attention_q8_reference_case(have_gpu, t_len):
    q, kc, vc, ks, vs, _, _, want = reference_attention_case(t_len)
    out = empty_dev((24, 256))
    dq, dk, dv, dks, dvs = to_dev(q), to_dev(kc), to_dev(vc), to_dev(ks), to_dev(vs)
    check(lib().chk_attn_decode_q8(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dks.data_ptr(), dvs.data_ptr(),
                                   t_len, 24, 2, 256, out.data_ptr(), None))
    assert_close(to_host(out), want, f"attention T={t_len}")


@pytest.mark.parametrize("nh,nkv,hd,t_len", [(16, 2, 256, 1), (16, 2, 256, 64), (16, 2, 256, 65),
                                            (16, 2, 256, 2049), (4, 2, 256, 129), (8, 2, 128, 200),
                                            (2, 2, 128, 63)])
def test_attention_q8_shapes(have_gpu, nh, nkv, hd, t_len):
    rng = np.random.default_rng(nh * 1000 + t_len)
    q = rng.normal(0, 1, (nh, 2 * hd)).astype(np.float32)
    kv_row = nkv * hd
    kc = rng.integers(-127, 128, (t_len, kv_row), dtype=np.int8)
    vc = rng.integers(-127, 128, (t_len, kv_row), dtype=np.int8)
    ksf = rng.uniform(0.001, 0.02, (t_len, kv_row // 32)).astype(np.float32)
    vsf = rng.uniform(0.001, 0.02, (t_len, kv_row // 32)).astype(np.float32)
    ks, vs = ksf.astype(np.float16), vsf.astype(np.float16)
    kd = kc.reshape(t_len, -1, 32).astype(np.float64) * ks.astype(np.float64)[:, :, None]
    vd = vc.reshape(t_len, -1, 32).astype(np.float64) * vs.astype(np.float64)[:, :, None]
    kd, vd = kd.reshape(t_len, kv_row), vd.reshape(t_len, kv_row)
    g = nh // nkv
    want = np.empty((nh, hd))
    for h in range(nh):
        hk = h // g
        sc = kd[:, hk * hd:(hk + 1) * hd] @ q[h, :hd] * hd ** -0.5
        p = np.exp(sc - sc.max())
        want[h] = (p @ vd[:, hk * hd:(hk + 1) * hd]) / p.sum() / (1.0 + np.exp(-q[h, hd:]))
    out = empty_dev((nh, hd))
    dq, dk, dv = to_dev(q), to_dev(kc), to_dev(vc)
    dks, dvs = to_dev(ks.view(np.uint16)), to_dev(vs.view(np.uint16))
    check(lib().chk_attn_decode_q8(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dks.data_ptr(), dvs.data_ptr(),
                                   t_len, nh, nkv, hd, out.data_ptr(), None))
    assert_close(to_host(out), want, f"attention {nh}/{nkv}x{hd} T={t_len}")
