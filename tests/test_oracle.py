"""CPU pins of the oracle (oracle/oracle.cpp, the C++ restatement of the
reference's CPU path): the reference's own known-answer tests for this
path, restated, plus closed forms and brute force where the reference has
no vector.  A plausible slip in the oracle (a transposed operand, a
dropped term, a wrong tie order or rounding mode) fails one of these.

Reference tests followed:
  tests/unit/quant.rs:42-92                    Q4 grouped matvec == dequant then dot
  tests/unit/qwen4_exp/lowbit.rs:154-278       Q2/Q3 slot permutation, pack round trip
  tests/unit/qwen4_exp/gpu/prefill.rs:177-260  low-bit midpoint rule vs an f64 dot
  tests/unit/qwen4_exp/gpu/attention.rs:115-200  q8 attention vs the CPU formula (LCG 23)
  src/qwen4_exp/cpu.rs:514                     routing order (index ascending on ties)
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests.numerics import (
    Lcg,
    bf16_bits,
    bf16_to_f32,
    f16_round,
    mlx_quantize,
    q4_codes,
    unpack_q2,
    unpack_q3,
)


# ------------------------------------------------------------- Q4 affine

def test_q4_matvec_matches_dequant_reference():
    """tests/unit/quant.rs:42-92: rows ((r*31 + i*7) % 97)/43 - 1, x
    ((i*13) % 29)/17 - 0.8; dequantised rows within 0.2 of the source,
    grouped matvec within 1e-3 (relative, floor 1) of dequant-then-dot."""
    out_dim, in_dim = 8, 128
    r = np.arange(out_dim)[:, None]
    i = np.arange(in_dim)[None, :]
    rows = (((r * 31 + i * 7) % 97).astype(np.float32) / np.float32(43.0) - np.float32(1.0)).astype(np.float32)
    w, s, b = mlx_quantize(rows)
    x = (((np.arange(in_dim) * 13) % 29).astype(np.float32) / np.float32(17.0) - np.float32(0.8)).astype(np.float32)
    y_ref = np.zeros(out_dim, np.float32)
    for row in range(out_dim):
        dense = O.q4_dequant_row(w, s, b, out_dim, in_dim, row)
        assert np.all(np.abs(dense - rows[row]) < 0.2), f"row {row}"
        y_ref[row] = np.float32(np.sum(dense * x, dtype=np.float32))
    y = O.q4_matvec(w, s, b, out_dim, in_dim, x)
    assert np.all(np.abs(y - y_ref) < 1e-3 * np.maximum(np.abs(y_ref), 1.0))


def test_q4_dequant_is_scale_times_code_plus_bias():
    """quant.rs:24-45: x = scale * q + bias in f32 (two roundings, no fma),
    nibbles LSB-first along the input dim; bit-exact."""
    rng = np.random.default_rng(5)
    out_dim, in_dim = 6, 256
    w = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.normal(0, 0.02, size=(out_dim, in_dim // 64)))
    b = bf16_bits(rng.normal(0, 0.01, size=(out_dim, in_dim // 64)))
    codes = q4_codes(w).astype(np.float32)
    sf = np.repeat(bf16_to_f32(s), 64, axis=1)
    bf = np.repeat(bf16_to_f32(b), 64, axis=1)
    want = (sf * codes).astype(np.float32) + bf
    for row in range(out_dim):
        got = O.q4_dequant_row(w, s, b, out_dim, in_dim, row)
        assert np.array_equal(got.view(np.uint32), want[row].astype(np.float32).view(np.uint32))


def test_q4_grouped_matvec_equals_dense_f64():
    """Closed form: sum_g s (q . x_g) + b sum(x_g) == (s q + b) . x."""
    rng = np.random.default_rng(7)
    out_dim, in_dim = 64, 2048
    w = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.normal(0, 0.02, size=(out_dim, in_dim // 64)))
    b = bf16_bits(rng.normal(0, 0.01, size=(out_dim, in_dim // 64)))
    x = rng.normal(0, 1, size=in_dim).astype(np.float32)
    dense = np.repeat(bf16_to_f32(s), 64, 1).astype(np.float64) * q4_codes(w) + np.repeat(bf16_to_f32(b), 64, 1)
    want = dense @ x.astype(np.float64)
    got = O.q4_matvec(w, s, b, out_dim, in_dim, x)
    assert np.max(np.abs(got - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))


# --------------------------------------------------------------- Q3 / Q2

def test_lowbit_slots_are_a_permutation():
    """tests/unit/qwen4_exp/lowbit.rs:154-173."""
    seen = set()
    for t, off in O.q2_slots():
        assert off <= 30 and off % 2 == 0
        assert (t, off) not in seen
        seen.add((t, off))
    assert len(seen) == 32
    up_seen, lo_seen = set(), set()
    for t, up, lo in O.q3_slots():
        assert up <= 30 and lo <= 31
        assert (t, up) not in up_seen
        assert lo not in lo_seen
        up_seen.add((t, up))
        lo_seen.add(lo)
    assert len(up_seen) == 32 and len(lo_seen) == 32


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("inter,hidden", [(2, 64), (512, 2048)])
def test_lowbit_packing_round_trips(bits, inter, hidden):
    """tests/unit/qwen4_exp/lowbit.rs:175-278: source bytes (i*37 + 11) % 256,
    unpacked as the kernels read them == Q4 code >> (4 - bits)."""
    codes = inter * hidden
    src = ((np.arange(codes // 2) * 37 + 11) % 256).astype(np.uint8)
    dst = O.pack_matrix(src, codes, bits)
    assert dst.size == codes * bits // 8
    chunks = codes // 32
    want = (q4_codes(src.view("<u4").reshape(chunks, 4)) >> (4 - bits)).astype(np.uint8)
    got = unpack_q2(dst, chunks) if bits == 2 else unpack_q3(dst, chunks)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512)])
def test_lowbit_matvec_midpoint_rule(bits, shape):
    """tests/unit/qwen4_exp/gpu/prefill.rs:177-260: weights
    fma(s, (code/step)*step + (step-1)/2, b) with step = 2^(4-bits), dotted
    in f64; x = (((i*37 + i/in*19) % 257) - 128)/129; max error within
    0.002 * max(1, max|ref|) at the reference's channels."""
    out_dim, in_dim = shape
    rng = np.random.default_rng(11 + bits)
    w = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.normal(0, 0.02, size=(out_dim, in_dim // 64)))
    b = bf16_bits(rng.normal(0, 0.01, size=(out_dim, in_dim // 64)))
    channels = [0, 1, 7, 8, 31, 32, 63, 64, 127, 128, out_dim - 1]
    step = 1 << (4 - bits)
    worst, scale = 0.0, 0.0
    for row in range(3):
        i = np.arange(in_dim) + row * in_dim
        x = ((((i * 37 + i // in_dim * 19) % 257).astype(np.float32) - 128.0) / np.float32(129.0)).astype(np.float32)
        y = O.lowbit_matvec(w, s, b, out_dim, in_dim, bits, x)
        for ch in channels:
            code = q4_codes(w[ch])
            mid = (code // step * step).astype(np.float64) + (step - 1) * 0.5
            sf = np.repeat(bf16_to_f32(s[ch]), 64).astype(np.float64)
            bf = np.repeat(bf16_to_f32(b[ch]), 64).astype(np.float64)
            wt = (sf * mid + bf).astype(np.float32)  # one rounding: f32 fma
            ref = float(np.dot(x.astype(np.float64), wt.astype(np.float64)))
            worst = max(worst, abs(float(y[ch]) - ref))
            scale = max(scale, abs(ref))
    assert worst <= 0.002 * max(1.0, scale)


# ----------------------------------------------------------- q8 and fp16

def test_f32_to_f16_is_ieee_round_nearest_even():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.normal(0, 1, 4000).astype(np.float32),
        rng.normal(0, 1e-5, 2000).astype(np.float32),   # subnormal halves
        (rng.normal(0, 1, 1000) * 7e4).astype(np.float32),  # overflow edge
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                  1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf], np.float32),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_q8_rule():
    """kv_append_q8 (kernels/common/attention.metal:225-233): per 32 block
    d = amax/127, q = rint(v/d) clamped to +-127 (0 when d = 0), stored as
    q * fp16(d)."""
    rng = np.random.default_rng(9)
    x = rng.normal(0, 2, 32 * 40).astype(np.float32)
    x[32:64] = 0.0                      # an all-zero block
    x[64:96] = np.linspace(-1, 1, 32)   # exact amax
    x[100] = 1e-30                      # tiny values
    got = O.q8_roundtrip(x)
    blk = x.reshape(-1, 32)
    d = (np.max(np.abs(blk), axis=1) / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(d[:, None] > 0, np.rint(blk / d[:, None]), 0.0)
    q = np.clip(q, -127, 127).astype(np.float32)
    want = (q * f16_round(d)[:, None]).astype(np.float32).ravel()
    assert np.array_equal(got, want)


# -------------------------------------------------------------- routing

def test_route_topk_brute_force_and_ties():
    rng = np.random.default_rng(13)
    for trial in range(50):
        E, k = 16, 4
        p = rng.random(E).astype(np.float32)
        if trial % 3 == 0:  # exact ties: equal probabilities must rank by index
            p[rng.choice(E, 6, replace=False)] = p[0]
        p = p / p.sum(dtype=np.float32)
        for norm in (True, False):
            ids, w = O.route_topk(p, k, norm)
            order = sorted(range(E), key=lambda e: (-float(p[e]), e))[:k]
            assert ids.tolist() == order
            sel = p[order]
            want = sel / np.float32(np.sum(sel, dtype=np.float32)) if norm else sel
            assert np.allclose(w, want, rtol=1e-6, atol=0)
    ids, _ = O.route_topk(np.full(8, 0.125, np.float32), 3, True)
    assert ids.tolist() == [0, 1, 2]


def test_softmax_matches_f64():
    rng = np.random.default_rng(17)
    x = (rng.normal(0, 3, 512)).astype(np.float32)
    got = O.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.max(np.abs(got - e / e.sum())) < 1e-7
    assert abs(float(got.sum(dtype=np.float64)) - 1.0) < 1e-5


# -------------------------------------------------------------- DeltaNet

def _unit(rng, n):
    v = rng.normal(0, 1, n)
    return (v / np.linalg.norm(v)).astype(np.float32)


def test_delta_rule_zero_state():
    """From S = 0: delta = beta v, S = k delta^T, y = S^T q = beta (k.q) v."""
    rng = np.random.default_rng(19)
    dk, dv = 128, 128
    q, k, v = _unit(rng, dk), _unit(rng, dk), rng.normal(0, 1, dv).astype(np.float32)
    for decay, beta in [(0.3, 0.7), (1.0, 1.0), (0.9, 0.05)]:
        s, y = O.delta_head_step(np.zeros((dk, dv), np.float32), q, k, v, decay, beta)
        want_y = beta * float(np.dot(k.astype(np.float64), q)) * v.astype(np.float64)
        assert np.max(np.abs(y - want_y)) < 1e-5
        assert np.max(np.abs(s - beta * np.outer(k, v))) < 1e-6


def test_delta_rule_orthonormal_keys_store_and_recall():
    """decay = 1, beta = 1, orthonormal keys: each step writes v_i at k_i
    exactly (the classic delta-rule projection), so S = sum k_i v_i^T and
    querying k_j returns v_j; re-writing a stored pair leaves S unchanged."""
    rng = np.random.default_rng(23)
    dk, dv, n = 64, 32, 8
    keys = np.linalg.qr(rng.normal(0, 1, (dk, n)))[0].T.astype(np.float32)
    vals = rng.normal(0, 1, (n, dv)).astype(np.float32)
    s = np.zeros((dk, dv), np.float32)
    for i in range(n):
        s, _ = O.delta_head_step(s, keys[i], keys[i], vals[i], 1.0, 1.0)
    assert np.max(np.abs(s - keys.T.astype(np.float64) @ vals)) < 1e-5
    for j in range(n):
        _, y = O.delta_head_step(s, keys[j], keys[j], vals[j], 1.0, 1.0)
        assert np.max(np.abs(y - vals[j])) < 1e-5
        s2, _ = O.delta_head_step(s, keys[j], keys[j], vals[j], 1.0, 1.0)
        assert np.max(np.abs(s2 - s)) < 1e-5


def test_delta_rule_decay_scales_state():
    """beta = 0: S <- decay S and y = decay S^T q."""
    rng = np.random.default_rng(29)
    dk, dv = 32, 16
    s0 = rng.normal(0, 1, (dk, dv)).astype(np.float32)
    q, k, v = _unit(rng, dk), _unit(rng, dk), rng.normal(0, 1, dv).astype(np.float32)
    s, y = O.delta_head_step(s0, q, k, v, 0.25, 0.0)
    assert np.max(np.abs(s - 0.25 * s0)) < 1e-6
    assert np.max(np.abs(y - 0.25 * s0.T.astype(np.float64) @ q)) < 1e-5


def test_causal_conv_equals_full_convolution():
    """causal_conv (cpu.rs:1067-1085) stepped over a sequence == silu of
    the causal convolution sum_j w[j] x[t - (k-1) + j] with zero history."""
    rng = np.random.default_rng(31)
    n, ck, T = 24, 4, 9
    w_bits = bf16_bits(rng.uniform(-0.5, 0.5, (n, ck)))
    w = bf16_to_f32(w_bits).astype(np.float64)
    xs = rng.normal(0, 1, (T, n)).astype(np.float32)
    hist = np.zeros(n * (ck - 1), np.float32)
    pad = np.vstack([np.zeros((ck - 1, n)), xs.astype(np.float64)])
    for t in range(T):
        out, hist = O.causal_conv(xs[t], w_bits, hist, ck)
        pre = sum(w[:, j] * pad[t + j] for j in range(ck))
        want = pre / (1.0 + np.exp(-pre))
        assert np.max(np.abs(out - want)) < 1e-5


# ----------------------------------------------------- norms, rope, misc

def test_norms_and_softplus():
    rng = np.random.default_rng(37)
    x = rng.normal(0, 3, 256).astype(np.float32)
    ones = bf16_bits(np.ones(256, np.float32))
    y = O.rms_norm(x, ones, 1e-6)
    x64 = x.astype(np.float64)
    assert np.max(np.abs(y - x64 / np.sqrt(np.mean(x64 * x64) + 1e-6))) < 1e-5
    w = bf16_bits(rng.uniform(0.5, 1.5, 256))
    y2 = O.rms_norm(x, w, 1e-6)
    assert np.max(np.abs(y2 - y * bf16_to_f32(w))) < 1e-5
    z = O.l2_norm(x, 1e-6)
    assert abs(np.linalg.norm(z.astype(np.float64)) - 1.0) < 1e-6
    for v in (-30.0, -3.0, 0.0, 0.5, 19.0, 20.0, 25.0):
        want = v if v > 20.0 else float(np.log1p(np.exp(v)))
        assert abs(O.softplus(v) - want) <= 1e-6 * max(1.0, abs(want))


def test_rope_partial_is_a_rotation():
    """rope_partial (cpu.rs:1051-1063): rotate-half pairs (j, j + rot/2),
    angle pos * theta^(-2j/rot); identity at pos 0; dims >= rot untouched;
    rotations compose additively."""
    rng = np.random.default_rng(41)
    hd, rot, theta = 256, 64, 1e7
    x = rng.normal(0, 1, hd).astype(np.float32)
    assert np.array_equal(O.rope_partial(x, 0, rot, theta), x)
    for pos in (1, 17, 2047):
        y = O.rope_partial(x, pos, rot, theta)
        assert np.array_equal(y[rot:], x[rot:])
        half = rot // 2
        j = np.arange(half)
        ang = pos * theta ** (-2.0 * j / rot)
        z = (x[:half] + 1j * x[half:rot].astype(np.float64)) * np.exp(1j * ang)
        assert np.max(np.abs(y[:half] - z.real)) < 2e-4
        assert np.max(np.abs(y[half:rot] - z.imag)) < 2e-4
    a = O.rope_partial(O.rope_partial(x, 5, rot, theta), 7, rot, theta)
    assert np.max(np.abs(a - O.rope_partial(x, 12, rot, theta))) < 1e-4


# --------------------------------------------------------------- attention

def _q8_cache(rng: Lcg, t_len: int, kv_row: int):
    """The cache of tests/unit/qwen4_exp/gpu/attention.rs:123-147: int8
    values (f * 100) truncated, fp16 scales 0.01 + 0.02 |f|."""
    n = t_len * kv_row
    kv = rng.fill(2 * n).reshape(n, 2)  # drawn k, v, k, v, ...
    kc = np.trunc(kv[:, 0] * np.float32(100.0)).astype(np.int8)
    vc = np.trunc(kv[:, 1] * np.float32(100.0)).astype(np.int8)
    ns = t_len * (kv_row // 32)
    sc = np.abs(rng.fill(2 * ns).reshape(ns, 2))
    ks = (np.float32(0.01) + np.float32(0.02) * sc[:, 0]).astype(np.float32)
    vs = (np.float32(0.01) + np.float32(0.02) * sc[:, 1]).astype(np.float32)
    return kc, vc, ks, vs


def reference_attention_case(t_len: int, nh: int = 24, nkv: int = 2, hd: int = 256):
    """Inputs and the expected output of the reference's q8 attention test
    (LCG seed 23), every token visible: returns q [nh][2 hd], int8 k/v, fp16
    scale bits, and the expected [nh][hd] from the test's CPU formula."""
    rng = Lcg(23)
    q = rng.fill(nh * 2 * hd).reshape(nh, 2 * hd)
    kv_row = nkv * hd
    kc, vc, ks, vs = _q8_cache(rng, t_len, kv_row)
    ksh, vsh = f16_round(ks), f16_round(vs)
    kd = (kc.reshape(t_len, kv_row // 32, 32).astype(np.float64) * ksh.reshape(t_len, -1, 1)).reshape(t_len, kv_row)
    vd = (vc.reshape(t_len, kv_row // 32, 32).astype(np.float64) * vsh.reshape(t_len, -1, 1)).reshape(t_len, kv_row)
    g = nh // nkv
    out = np.empty((nh, hd))
    for h in range(nh):
        hk = h // g
        sc = kd[:, hk * hd:(hk + 1) * hd] @ q[h, :hd].astype(np.float64) * hd ** -0.5
        p = np.exp(sc - sc.max())
        o = p @ vd[:, hk * hd:(hk + 1) * hd] / p.sum()
        out[h] = o / (1.0 + np.exp(-q[h, hd:].astype(np.float64)))
    return q, kc, vc, ks.astype(np.float16).view(np.uint16), vs.astype(np.float16).view(np.uint16), kd, vd, out


def test_attention_core_reference_case():
    """The oracle's attention core on the dequantised cache of the
    reference's LCG-23 case (t_len 300) == the test's CPU formula."""
    q, _, _, _, _, kd, vd, want = reference_attention_case(300)
    got = O.attend(q, kd.astype(np.float32), vd.astype(np.float32), 24, 2, 256)
    assert np.max(np.abs(got - want)) < 1e-5 * max(1.0, np.max(np.abs(want)))


# ------------------------------------------------------------ QSA selection

def _qsa_expect(scores, t_len, k, ratio):
    """The reference test's construction (tests/unit/qwen4_exp/gpu/qsa.rs:
    318-330): blocks ordered by (score desc, block asc), the first k as token
    runs, the incomplete tail appended, ascending."""
    n = t_len // ratio
    order = sorted(range(n), key=lambda b: (-float(scores[b]), b))
    vis = [t for b in order[:k] for t in range(b * ratio, (b + 1) * ratio)]
    vis += list(range(n * ratio, t_len))
    return sorted(vis)


def test_qsa_pick_reference_ties():
    """index_select_handles_ties (tests/unit/qwen4_exp/gpu/qsa.rs:300-372):
    600 complete blocks + 2 tail tokens, five distinct values and many
    zeros; ties go to the lowest block."""
    ratio, k, base_pos = 4, 512, 2401
    t_len = base_pos + 1
    n = t_len // ratio
    scores = np.array([0.0 if i % 3 == 0 else ((i * 7) % 5) * 0.5 for i in range(n + 8)], np.float32)
    got = O.qsa_pick(scores[:n], t_len, k, ratio)
    assert got.tolist() == _qsa_expect(scores, t_len, k, ratio)
    assert got.size == k * ratio + 2


@pytest.mark.parametrize("seed", range(4))
def test_qsa_pick_random_with_duplicates(seed):
    rng = np.random.default_rng(seed)
    ratio = int(rng.choice([2, 4, 8]))
    t_len = int(rng.integers(40, 3000))
    n = t_len // ratio
    k = int(rng.integers(1, n))
    scores = rng.choice(np.float32([0.0, 0.25, 0.5, 1.5, 2.0]), size=n) + (rng.random(n) < 0.3) * rng.random(n).astype(np.float32)
    got = O.qsa_pick(scores.astype(np.float32), t_len, k, ratio)
    assert got.tolist() == _qsa_expect(scores.astype(np.float32), t_len, k, ratio)


@pytest.mark.parametrize("base,override", [(2, 4), (4, 3), (4, 2)])
def test_per_record_bits_select_each_records_reconstruction(base, override):
    """The oracle's per-record precision (Pool::set_kind, residency.rs:
    298-306): a model of expert_bits `base` whose every record is set to
    `override` gives exactly the MoE output of a model of expert_bits
    `override`; one chosen record set alone changes the output, and 0
    restores the model's own precision exactly."""
    from cherenkov_amd import presets

    cfg = presets.tiny(mtp=0)
    E, k = cfg.num_experts, cfg.num_experts_per_tok
    x = np.random.default_rng(5).normal(0, 1, cfg.hidden_size).astype(np.float32)
    x /= np.sqrt(np.mean(x * x))
    m = O.OracleModel(cfg, expert_bits=base)
    ref_o = O.OracleModel(cfg, expert_bits=override)
    out_base, ids, w, _ = m.moe(1, x)
    out_ref, ids_r, _, _ = ref_o.moe(1, x)
    assert list(ids) == list(ids_r)
    # one chosen expert switched: only its term changes
    m.set_record_bits(1, int(ids[0]), override)
    one, _, _, _ = m.moe(1, x)
    assert not np.array_equal(one, out_base)
    for e in range(E):
        m.set_record_bits(1, e, override)
    np.testing.assert_array_equal(m.moe(1, x)[0], out_ref)
    # 0 restores the model's own precision
    for e in range(E):
        m.set_record_bits(1, e, 0)
    np.testing.assert_array_equal(m.moe(1, x)[0], out_base)
    assert len(ids) == k
