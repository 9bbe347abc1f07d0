"""GPU parity of the prefill path: the MFMA Q4 GEMM against the oracle's
row-by-row Q4 matvec (quant.rs:49-88 semantics), through the C ABI."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd.abi import check, lib
from oracle.oracle import q4_matvec
from tests.gpu_util import assert_close, empty_dev, to_dev, to_host
from tests.numerics import bf16_bits

pytestmark = pytest.mark.gpu


def rand_q4(rng, out_dim, in_dim):
    w = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.normal(0, 0.02, size=(out_dim, in_dim // 64)))
    b = bf16_bits(rng.normal(0, 0.01, size=(out_dim, in_dim // 64)))
    return w, s, b


@pytest.mark.parametrize("out_dim,in_dim,T", [(256, 2048, 64), (333, 512, 100), (1296, 2048, 37), (2048, 4096, 130),
                                              (16, 64, 1)])
def test_q4_gemm_matches_rowwise_oracle(have_gpu, out_dim, in_dim, T):
    rng = np.random.default_rng(out_dim * 7 + T)
    w, s, b = rand_q4(rng, out_dim, in_dim)
    x = rng.normal(0, 1, (T, in_dim)).astype(np.float32)
    dw, ds, db, dx = to_dev(w), to_dev(s), to_dev(b), to_dev(x)
    y = empty_dev((T, out_dim))
    check(lib().chk_q4_gemm(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), out_dim, in_dim, dx.data_ptr(), T,
                            y.data_ptr(), None))
    got = to_host(y)
    ref = np.stack([q4_matvec(w, s, b, out_dim, in_dim, x[t]) for t in range(T)])
    # f32-grade: exact weights, activations carried to ~22 bits, f32 accumulation
    assert_close(got, ref, f"gemm {out_dim}x{in_dim} T={T}", abs_frac=1e-4, min_cos=0.999999)
