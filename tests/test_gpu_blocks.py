"""GPU parity of the engine's primitives and blocks against the CPU oracle
(the restatement of /root/reference/src/qwen4_exp/cpu.rs), through the
C ABI of include/cherenkov/{engine,kernels}.h.

Covers: the device weight generator (bit-exact with the oracle's), the
Q3/Q2 repack (bit-exact with lowbit.rs pack_matrix), the Q4 matvec, the
hyper-connection read, the MoE block at full shape in Q4/Q3/Q2 (config 2),
the DeltaNet layer decode and 3-row verify with rollback (config 3), and
gated attention over a q8 KV cache at 1k/8k/32k tokens, batch 1 and 2
(config 4).
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.abi import check, lib
from cherenkov_amd.engine import Engine
from oracle.oracle import OracleModel, pack_matrix, q4_matvec
from tests.gpu_util import assert_close, empty_dev, to_dev, to_host, topk_margin

pytestmark = pytest.mark.gpu


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def rand_q4(rng, out_dim, in_dim):
    w = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.normal(0, 0.02, size=(out_dim, in_dim // 64)))
    b = bf16_bits(rng.normal(0, 0.01, size=(out_dim, in_dim // 64)))
    return w, s, b


# ------------------------------------------------------------------ engines

@pytest.fixture(scope="module")
def tiny_pair(have_gpu):
    cfg = presets.tiny()
    eng = Engine(cfg, experts=4, drafts=2, max_t=512)
    orc = OracleModel(cfg)
    yield cfg, eng, orc
    eng.close()


@pytest.fixture(scope="module")
def big4(have_gpu):
    """Full-width blocks (hidden 2048, 512 experts top-10): a 4-layer model of
    the 80B-A3B shape, context up to 33k tokens."""
    cfg = presets.qwen3next_80b_shape(layers=4, mtp=0)
    eng = Engine(cfg, experts=4, drafts=0, max_t=33 * 1024)
    orc = OracleModel(cfg)
    yield cfg, eng, orc
    eng.close()


# ------------------------------------------------------- weights and repack

def test_device_generator_matches_oracle(tiny_pair):
    cfg, eng, orc = tiny_pair
    for layer, e in [(0, 0), (1, 7), (3, 15), (4, 3)]:  # 4 = MTP record layer
        got = eng.expert_record(layer, e, 4)
        ref = orc.expert_record(layer, e)
        assert np.array_equal(got, ref), f"record ({layer}, {e}) differs"


@pytest.mark.parametrize("bits", [3, 2])
def test_lowbit_repack_matches_pack_matrix(have_gpu, bits):
    cfg = presets.tiny(layers=4, mtp=0)
    eng = Engine(cfg, experts=bits, drafts=0, max_t=64)
    try:
        I, H = cfg.moe_intermediate_size, cfg.hidden_size
        codes = I * H
        mat = codes * bits // 8
        sb = I * (H // 64) * 2
        for layer, e in [(0, 0), (2, 9)]:
            q4 = eng.expert_record(layer, e, 4)
            lo = eng.expert_record(layer, e, bits)
            for m in range(3):
                src = q4[m * codes // 2:(m + 1) * codes // 2]
                ref = pack_matrix(src, codes, bits)
                assert np.array_equal(lo[m * mat:(m + 1) * mat], ref), f"matrix {m} of ({layer},{e})"
            # six scale/bias blocks copied verbatim, in lowbit.rs order
            q4_scales = q4[3 * codes // 2:3 * codes // 2 + 6 * sb]
            assert np.array_equal(lo[3 * mat:3 * mat + 6 * sb], q4_scales)
    finally:
        eng.close()


# ------------------------------------------------------------ Q4 matvec

@pytest.mark.parametrize("in_dim", [64, 320, 512, 2048, 4096, 8192])
@pytest.mark.parametrize("nb", [1, 2, 3, 4])
def test_q4_matvec(have_gpu, in_dim, nb):
    rng = np.random.default_rng(in_dim * 10 + nb)
    out_dim = 333
    w, s, b = rand_q4(rng, out_dim, in_dim)
    x = rng.normal(0, 1, size=(nb, in_dim)).astype(np.float32)
    dw, ds, db, dx = to_dev(w), to_dev(s), to_dev(b), to_dev(x)
    dy = empty_dev((nb, out_dim))
    check(lib().chk_q4_matvec(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), out_dim, in_dim, dx.data_ptr(),
                              dy.data_ptr(), nb, None))
    y = to_host(dy)
    for r in range(nb):
        ref = q4_matvec(w, s, b, out_dim, in_dim, x[r])
        # same math, different summation order: fp32 rounding only
        np.testing.assert_allclose(y[r], ref, rtol=2e-4, atol=2e-4 * max(1.0, np.abs(ref).max()))


# ---------------------------------------------------- hyper-connection read

@pytest.mark.parametrize("which", [0, 1, 2, 3])
def test_hc_read(tiny_pair, which):
    cfg, eng, orc = tiny_pair
    rng = np.random.default_rng(100 + which)
    hh = cfg.hidden_size * cfg.hc_count
    nb = 3
    hyper = rng.normal(0, 3, size=(nb, hh)).astype(np.float32)
    dmix = empty_dev((nb, cfg.hidden_size))
    dinj = empty_dev((nb, cfg.hc_count))
    check(lib().chk_hc_read(eng.handle, 1, which, to_dev(hyper).data_ptr(), nb, dmix.data_ptr(), dinj.data_ptr()))
    mix, inj = to_host(dmix), to_host(dinj)
    for r in range(nb):
        m_ref, i_ref = orc.gated_residual(1 if which < 2 else 0, which, hyper[r])
        assert_close(mix[r], m_ref, f"hc{which} mixed row {r}")
        if which < 2:
            assert_close(inj[r], i_ref, f"hc{which} inj row {r}", abs_frac=1e-4)


def test_hc_read_full_width(big4):
    cfg, eng, orc = big4
    rng = np.random.default_rng(7)
    hh = cfg.hidden_size * cfg.hc_count
    hyper = rng.normal(0, 5, size=(2, hh)).astype(np.float32)
    dmix = empty_dev((2, cfg.hidden_size))
    dinj = empty_dev((2, cfg.hc_count))
    check(lib().chk_hc_read(eng.handle, 2, 1, to_dev(hyper).data_ptr(), 2, dmix.data_ptr(), dinj.data_ptr()))
    mix = to_host(dmix)
    for r in range(2):
        m_ref, _ = orc.gated_residual(2, 1, hyper[r])
        assert_close(mix[r], m_ref, f"hc full row {r}")


# ------------------------------------------------------------ MoE (config 2)

def rms_norm_unit(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = x.astype(np.float32)
    return (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def check_moe(cfg, eng, orc, layer, x, label):
    nb = x.shape[0]
    k, E = cfg.num_experts_per_tok, cfg.num_experts
    dout = empty_dev((nb, cfg.hidden_size))
    dids = empty_dev((nb, k), np.uint32)
    dw = empty_dev((nb, k))
    dp = empty_dev((nb, E))
    check(lib().chk_moe_block(eng.handle, layer, to_dev(x).data_ptr(), nb, dout.data_ptr(), dids.data_ptr(),
                              dw.data_ptr(), dp.data_ptr()))
    out, ids, w, probs = to_host(dout), to_host(dids).view(np.uint32), to_host(dw), to_host(dp)
    exempt = 0
    for r in range(nb):
        o_ref, i_ref, w_ref, p_ref = orc.moe(layer, x[r])
        margin = topk_margin(p_ref, k)
        assert_close(probs[r], p_ref, f"{label} router probs row {r}", abs_frac=1e-4)
        if margin > 1e-3:
            assert list(ids[r]) == list(i_ref), f"{label} row {r}: top-k {ids[r]} vs {i_ref} (margin {margin:.2e})"
            np.testing.assert_allclose(w[r], w_ref, rtol=1e-4, atol=1e-6)
            assert_close(out[r], o_ref, f"{label} out row {r}")
        else:
            exempt += 1
    return exempt


@pytest.mark.parametrize("nb", [1, 3])
def test_moe_block_q4(big4, nb):
    cfg, eng, orc = big4
    rng = np.random.default_rng(2000 + nb)
    exempt = 0
    for it in range(4):
        x = rms_norm_unit(bf16_round(rng.normal(0, 1, size=(nb, cfg.hidden_size))))
        exempt += check_moe(cfg, eng, orc, it % 4, x, f"moe q4 it{it}")
    assert exempt <= 1


@pytest.mark.parametrize("bits", [3, 2])
def test_moe_block_lowbit(have_gpu, bits):
    cfg = presets.qwen3next_80b_shape(layers=1, mtp=0)
    eng = Engine(cfg, experts=bits, drafts=0, max_t=64)
    orc = OracleModel(cfg, expert_bits=bits)
    try:
        rng = np.random.default_rng(3000 + bits)
        x = rms_norm_unit(bf16_round(rng.normal(0, 1, size=(2, cfg.hidden_size))))
        assert check_moe(cfg, eng, orc, 0, x, f"moe q{bits}") <= 1
    finally:
        eng.close()


# ------------------------------------------------------- DeltaNet (config 3)

def test_deltanet_decode_and_verify_rollback(big4):
    cfg, eng, orc = big4
    layer = 1
    eng.reset()
    st = orc.new_state()
    rng = np.random.default_rng(31)
    H = cfg.hidden_size
    dout = empty_dev((3, H))
    # single decode steps from zero state
    for t in range(3):
        x = rng.normal(0, 1, size=(1, H)).astype(np.float32)
        check(lib().chk_deltanet_block(eng.handle, layer, to_dev(x).data_ptr(), 1, 0, dout.data_ptr()))
        ref = st.deltanet(layer, x[0])
        assert_close(to_host(dout)[0], ref, f"deltanet decode step {t}")
    s_gpu = np.empty(cfg.linear_num_value_heads * 128 * 128, np.float32)
    conv_dim = 2 * 16 * 128 + 32 * 128
    c_gpu = np.empty(conv_dim * 3, np.float32)
    check(lib().chk_deltanet_state(eng.handle, layer, s_gpu.ctypes.data, c_gpu.ctypes.data))
    s_ref, c_ref = st.delta_state(layer)
    assert_close(s_gpu, s_ref, "deltanet state")
    assert_close(c_gpu, c_ref, "conv history")
    # a 3-row verify batch == three sequential rows
    x3 = rng.normal(0, 1, size=(3, H)).astype(np.float32)
    check(lib().chk_deltanet_block(eng.handle, layer, to_dev(x3).data_ptr(), 3, 1, dout.data_ptr()))
    o3 = to_host(dout)
    snap_ref = []
    for r in range(3):
        ref = st.deltanet(layer, x3[r])
        assert_close(o3[r], ref, f"deltanet verify row {r}")
        snap_ref.append(st.delta_state(layer))
    # rollback to plane 0 (commit 1 of 3) restores the state after row 0
    check(lib().chk_deltanet_rollback(eng.handle, layer, 0))
    check(lib().chk_deltanet_state(eng.handle, layer, s_gpu.ctypes.data, c_gpu.ctypes.data))
    assert_close(s_gpu, snap_ref[0][0], "state after rollback to row 0")
    assert_close(c_gpu, snap_ref[0][1], "conv history after rollback to row 0")


# ------------------------------------------------------ attention (config 4)

@pytest.mark.parametrize("T", [1024, 8192, 32768])
def test_attention_q8_decode(big4, T):
    cfg, eng, orc = big4
    layer = 3
    kv_row = cfg.num_key_value_heads * cfg.head_dim
    rng = np.random.default_rng(40 + T)
    k = rng.normal(0, 1, size=(T, kv_row)).astype(np.float32)
    v = rng.normal(0, 1, size=(T, kv_row)).astype(np.float32)
    check(lib().chk_kv_fill(eng.handle, layer, 0, to_dev(k).data_ptr(), to_dev(v).data_ptr(), T))
    x = rng.normal(0, 1, size=(1, cfg.hidden_size)).astype(np.float32)
    dout = empty_dev((1, cfg.hidden_size))
    check(lib().chk_attention_block(eng.handle, layer, to_dev(x).data_ptr(), 1, T, dout.data_ptr()))
    ref = orc.attention_kv(layer, x[0], k, v, kv_q8=True)
    assert_close(to_host(dout)[0], ref, f"attention q8 T={T}")
    # the f32-KV formula of cpu.rs agrees within the end-to-end tolerance
    ref32 = orc.attention_kv(layer, x[0], k, v, kv_q8=False)
    assert_close(to_host(dout)[0], ref32, f"attention vs f32 KV T={T}", abs_frac=5e-2, min_cos=0.995)


@pytest.mark.parametrize("T", [1024, 8192, 32768])
def test_attention_q8_batch2(big4, T):
    cfg, eng, orc = big4
    layer = 3
    kv_row = cfg.num_key_value_heads * cfg.head_dim
    rng = np.random.default_rng(50 + T)
    Ts = [T, T // 2 + 17]
    ks = [rng.normal(0, 1, size=(t, kv_row)).astype(np.float32) for t in Ts]
    vs = [rng.normal(0, 1, size=(t, kv_row)).astype(np.float32) for t in Ts]
    for seq in range(2):
        check(lib().chk_kv_fill(eng.handle, layer, seq, to_dev(ks[seq]).data_ptr(), to_dev(vs[seq]).data_ptr(), Ts[seq]))
    x = rng.normal(0, 1, size=(2, cfg.hidden_size)).astype(np.float32)
    dout = empty_dev((2, cfg.hidden_size))
    pos = (C.c_uint32 * 2)(*Ts)
    check(lib().chk_attention_block2(eng.handle, layer, to_dev(x).data_ptr(), pos, dout.data_ptr()))
    out = to_host(dout)
    for r in range(2):
        ref = orc.attention_kv(layer, x[r], ks[r], vs[r], kv_q8=True)
        assert_close(out[r], ref, f"attention batch2 row {r}")


def test_attention_verify_rows_are_causal(big4):
    """Three rows at positions T, T+1, T+2 of one sequence: row r sees its own
    and earlier rows' keys only (the verify batch of speculative decode)."""
    cfg, eng, orc = big4
    layer = 3
    kv_row = cfg.num_key_value_heads * cfg.head_dim
    T = 300
    rng = np.random.default_rng(77)
    k = rng.normal(0, 1, size=(T, kv_row)).astype(np.float32)
    v = rng.normal(0, 1, size=(T, kv_row)).astype(np.float32)
    check(lib().chk_kv_fill(eng.handle, layer, 0, to_dev(k).data_ptr(), to_dev(v).data_ptr(), T))
    x = rng.normal(0, 1, size=(3, cfg.hidden_size)).astype(np.float32)
    dout = empty_dev((3, cfg.hidden_size))
    check(lib().chk_attention_block(eng.handle, layer, to_dev(x).data_ptr(), 3, T, dout.data_ptr()))
    out = to_host(dout)
    ref = orc.attention_kv(layer, x, k, v, kv_q8=True)
    for r in range(3):
        assert_close(out[r], ref[r], f"verify attention row {r}")
