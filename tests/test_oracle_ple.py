"""Pins of the oracle's PLE n-gram block (oracle/oracle.cpp: ngram_ids_from,
ngram_row, ple, and its place in forward_token), CPU only.

The reference holds no test of this block, so each check is a hand-worked
case or a closed form on special weights, chosen so that a plausible slip
(a wrong shift or window, a missing EOS reset, i64 wrap or Euclidean
remainder, a wrong tap distance, ring slot or `back <= filled` rule, the
gate's sign or root, the block after instead of before its layer) fails:
  - ids: Python integers restate the documented hash (cpu.rs:848-887) on
    multipliers that isolate one shifted token at a time;
  - rows: table bytes with known codes, scales and biases (packed.rs:233-256);
  - ple (cpu.rs:889-967): constant projections give key, value and the
    gate in closed form; the conv taps are read back through a twin model
    whose conv weights are zero;
  - forward_token (cpu.rs:414-421): the block's addend lands in hyper
    before its layer's own read.
"""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from oracle.oracle import OracleModel
from tests.numerics import bf16_bits, bf16_to_f32
from tests.test_oracle_compositions import EPS, bf, close, expert_record, f, grouped_norm, q4_bias, sig, silu, \
    zero_layer_outputs

PLE_LAYER = 2  # 1-based, as ple_layer_ids writes it


def ple_cfg(**kw):
    cfg = presets.with_ple(presets.tiny(mtp=0), layer=PLE_LAYER, **kw)
    return cfg


def wrap_i64(v: int) -> int:
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >> 63 else v


def expected_ids(tokens, mult, offs, sizes, eos, ngram=3, heads=8):
    """The documented hash with Python integers."""
    t = len(tokens) - 1
    shifted = [tokens[t]]
    for k in range(1, ngram):
        before = t < k or eos in tokens[t - k:t]
        shifted.append(eos if before else tokens[t - k])
    ids = []
    for n in range(2, ngram + 1):
        mixed = 0
        for p in range(n):
            mixed ^= wrap_i64(shifted[p] * int(mult[p])) & ((1 << 64) - 1)
        mixed = wrap_i64(mixed)
        for h in range((n - 2) * heads, (n - 1) * heads):
            ids.append(mixed % int(sizes[h]) + int(offs[h]))  # Python %: Euclidean for size > 0
    return ids


@pytest.fixture(scope="module")
def model():
    return OracleModel(ple_cfg())


# ------------------------------------------------------------------ ids

@pytest.mark.parametrize("mult", [(1, 0, 0), (0, 1, 0), (0, 0, 1), (3, 5, 7)])
@pytest.mark.parametrize("tokens", [[5], [5, 7], [5, 7, 9], [5, 4095, 9], [4095, 7, 9], [5, 7, 4095],
                                    [11, 4095, 13, 17, 19]])
def test_ngram_ids_isolate_each_shift(model, mult, tokens):
    """Multipliers (1,0,0), (0,1,0), (0,0,1) make every bigram / trigram head
    hash one shifted token: the current one, the previous one or EOS, the
    one two back or EOS (an EOS in [t-k, t), or t < k, reads as EOS; the
    current token being EOS does not)."""
    m = model
    _, offs, sizes = m.ngram_meta()
    m.set_ngram_meta(np.array(mult, np.int64), offs, sizes)
    got = m.ngram_ids(tokens).tolist()
    assert got == expected_ids(tokens, mult, offs, sizes, eos=4095)
    if mult == (0, 0, 1):
        # bigram heads hash 0: their ids are the head offsets
        assert got[:8] == [int(o) for o in offs[:8]]


def test_ngram_ids_wrap_and_euclidean_remainder(model):
    """Products wrap like i64 (2^62 + 1 times 4 is 4 after the wrap) and a
    negative hash takes the Euclidean remainder (-15 mod 97 = 82)."""
    m = model
    _, offs, sizes = m.ngram_meta()
    sizes = np.array([97] * 16, np.uint64)
    offs = np.arange(16, dtype=np.uint64) * 1000
    m.set_ngram_meta(np.array([-3, 0, 0], np.int64), offs, sizes)
    assert m.ngram_ids([5]).tolist() == [82 + 1000 * h for h in range(16)]
    m.set_ngram_meta(np.array([2 ** 62 + 1, 0, 0], np.int64), offs, sizes)
    assert m.ngram_ids([4]).tolist() == [4 + 1000 * h for h in range(16)]
    m.set_ngram_meta(np.array([3, 5, 0], np.int64), offs, sizes)
    # bigram: 9*3 ^ 2*5 = 27 ^ 10 = 17; trigram adds 0 * EOS
    assert m.ngram_ids([2, 9]).tolist() == [17 + 1000 * h for h in range(16)]


def test_synthetic_metadata_is_the_documented_layout(model):
    m = OracleModel(ple_cfg())
    mult, offs, sizes = m.ngram_meta()
    assert sizes.tolist() == [1021 - h for h in range(16)]
    assert offs.tolist() == np.concatenate([[0], np.cumsum(sizes)[:-1]]).tolist()
    assert all(v > 0 and v % 2 == 1 for v in mult.tolist())
    assert m.ngram_table().size == int(sizes.sum()) * (16 // 2 + 4 * (16 // 16))


# ------------------------------------------------------------------ rows

@pytest.mark.parametrize("group", [16, 8])
def test_ngram_row_dequantises_codes_scales_biases(group):
    """Row r: codes q_i = (i + r) % 16, scale 0.5 (group g: 0.5 + g), bias
    0.25, so value_i = s_g q_i + 0.25 exactly."""
    m = OracleModel(ple_cfg(group=group))
    t = m.ngram_table()
    dim, gpr = 16, 16 // group
    rb = dim // 2 + 4 * gpr
    rows = t.size // rb
    for r in (0, 1, rows - 1):
        q = [(i + r) % 16 for i in range(dim)]
        words = [sum(q[w * 8 + j] << (4 * j) for j in range(8)) for w in range(dim // 8)]
        rec = np.frombuffer(np.array(words, np.uint32).tobytes(), np.uint8).tolist()
        scales = [0.5 + g for g in range(gpr)]
        rec += np.frombuffer(bf16_bits(np.array(scales, np.float32)).tobytes(), np.uint8).tolist()
        rec += np.frombuffer(bf16_bits(np.full(gpr, 0.25, np.float32)).tobytes(), np.uint8).tolist()
        t[r * rb:(r + 1) * rb] = rec
    m.set_ngram_table(t)
    for r in (0, 1, rows - 1):
        want = [scales[i // group] * ((i + r) % 16) + 0.25 for i in range(dim)]
        assert m.ngram_row(r).tolist() == want
    with pytest.raises(RuntimeError):
        m.ngram_row(rows)


# ------------------------------------------------------------------ block

def constant_table(m, value_code=3, scale=0.5, bias=0.25):
    """Every table row the same: e_i = scale * value_code + bias."""
    t = m.ngram_table()
    dim, gpr = 16, 1
    rb = dim // 2 + 4 * gpr
    word = sum(value_code << (4 * j) for j in range(8))
    rec = np.frombuffer(np.array([word] * (dim // 8), np.uint32).tobytes(), np.uint8).tolist()
    rec += np.frombuffer(bf16_bits(np.array([scale], np.float32)).tobytes(), np.uint8).tolist()
    rec += np.frombuffer(bf16_bits(np.array([bias], np.float32)).tobytes(), np.uint8).tolist()
    t[:] = np.tile(np.array(rec, np.uint8), t.size // rb)
    m.set_ngram_table(t)
    return scale * value_code + bias


def test_gate_sign_and_root_closed_form():
    """Constant key / value projections (every weight its group's bias):
    key_i = kb * sum(e), value_i = vb * sum(e).  With unit norms, stream g of
    hyper a constant c_g: dot_g = h * sign(K c_g) a_g / sqrt(h), a_g the two
    eps factors, gate = sign(dot) sqrt(|dot|), gated_g = sigmoid(gate) V;
    conv: last tap 1, so the addend is gated + silu(gvn)."""
    cfg = ple_cfg()
    m = OracleModel(cfg)
    st = m.new_state()
    H, hc, E = cfg.hidden_size, cfg.hc_count, cfg.ple_embed_dim
    hh = H * hc
    l = PLE_LAYER - 1
    ev = constant_table(m)
    S = E * ev  # sum(e)
    kb, vb = 0.125, -0.5
    m.set_q4(l, "ple.key", *q4_bias(hh, E, kb))
    m.set_q4(l, "ple.value", *q4_bias(H, E, vb))
    for n in ("ple.norm_key", "ple.norm_query", "ple.norm_conv"):
        m.set_bf16(l, n, bf(np.ones(hh)))
    conv = np.zeros((hh, cfg.ple_conv_kernel_size))
    conv[:, -1] = 1.0
    m.set_bf16(l, "ple.conv", bf(conv.ravel()))
    c = np.array([0.75, -2.0, 1e-3, -0.5])
    hyper = np.repeat(c, H).astype(np.float32)
    add, gvn = st.ple(17, hyper)
    K, V = kb * S, vb * S
    a = (1 / np.sqrt(1 + EPS / K ** 2)) * (1 / np.sqrt(1 + EPS / c ** 2))
    dot = H * np.sign(K * c) * a / np.sqrt(H)
    gate = np.sign(dot) * np.sqrt(np.maximum(np.abs(dot), 1e-6))
    gated = np.repeat(sig(gate) * V, H)
    gv = grouped_norm(gated, np.ones(hh), H)
    close(gvn, gv, "gvn", rtol=1e-5)
    close(add, gated + silu(gv), "addend", rtol=1e-5)


def test_zero_key_gate_is_sigmoid_of_a_thousandth():
    """key = 0 gives dot = +0 (some query products +0), gate = sqrt(1e-6)."""
    cfg = ple_cfg()
    m = OracleModel(cfg)
    st = m.new_state()
    H, hc, E = cfg.hidden_size, cfg.hc_count, cfg.ple_embed_dim
    hh = H * hc
    l = PLE_LAYER - 1
    ev = constant_table(m)
    m.set_q4(l, "ple.key", *q4_bias(hh, E, 0.0))
    m.set_q4(l, "ple.value", *q4_bias(H, E, 1.0))
    m.set_bf16(l, "ple.conv", bf(np.zeros(hh * cfg.ple_conv_kernel_size)))
    hyper = np.random.default_rng(3).normal(0, 1, hh).astype(np.float32)
    add, _ = st.ple(5, hyper)
    close(add, np.full(hh, sig(1e-3) * E * ev), "addend", rtol=1e-6)


@pytest.mark.parametrize("tap", [0, 1, 2, 3])
def test_conv_taps_read_the_dilated_ring(tap):
    """Only tap k non-zero (weight 0.5): the addend at position p is gated_p
    + silu(0.5 gvn_{p - 3 (3 - k)}) when that position exists (back <=
    filled), else gated_p + silu(0).  gated_p and the gvn sequence come
    from a twin model with every tap zero; 14 positions wrap the 9-slot
    ring."""
    cfg = ple_cfg()
    H, hc = cfg.hidden_size, cfg.hc_count
    hh = H * hc
    K = cfg.ple_conv_kernel_size
    l = PLE_LAYER - 1
    w = np.zeros((hh, K))
    w[:, tap] = 0.5
    a, b = OracleModel(cfg), OracleModel(cfg)
    a.set_bf16(l, "ple.conv", bf(w.ravel()))
    b.set_bf16(l, "ple.conv", bf(np.zeros(hh * K)))
    sa, sb = a.new_state(), b.new_state()
    rng = np.random.default_rng(11)
    gvns = []
    back = cfg.ngram_size * (K - 1 - tap)
    for p, tok in enumerate(rng.integers(0, cfg.vocab_size, 14)):
        hyper = rng.normal(0, 1, hh).astype(np.float32)
        add, gvn = sa.ple(int(tok), hyper)
        gated, gvn_b = sb.ple(int(tok), hyper)
        close(gvn, gvn_b, f"gvn {p}", rtol=0)
        gvns.append(gvn.astype(np.float64))
        src = gvns[p - back] if back <= p else np.zeros(hh)
        close(add, gated + silu(0.5 * src), f"addend at {p}", rtol=1e-5)


def test_forward_token_adds_the_block_before_its_layer():
    """Layer outputs zeroed except the PLE layer's shared expert behind its
    mlp_hc read (as the forward_token pin of the compositions test): the
    stack then leaves hyper = e + add + 1/2 y inj with y and inj computed
    from e + add, where add is the block's addend on the embedding (from a
    twin model).  Applying the block after the layer, or not at all, moves
    both terms."""
    cfg = ple_cfg()
    m = OracleModel(cfg)
    twin = OracleModel(cfg)
    st = m.new_state()
    H, hc, V = cfg.hidden_size, cfg.hc_count, cfg.vocab_size
    hh = H * hc
    SI = cfg.shared_expert_intermediate_size
    layer = PLE_LAYER - 1
    rng = np.random.default_rng(41)
    eb = rng.normal(0, 1, (V, H // 64))
    m.set_q4(0, "embed", *q4_bias(V, H, eb))
    for ly in range(cfg.num_hidden_layers):
        zero_layer_outputs(cfg, m, ly)
    bg, bu, bd = 0.25, -0.5, 0.125
    m.set_q4(layer, "moe.sh_gate", *q4_bias(SI, H, bg))
    m.set_q4(layer, "moe.sh_up", *q4_bias(SI, H, bu))
    m.set_q4(layer, "moe.sh_down", *q4_bias(H, SI, bd))
    m.set_bf16(layer, "moe.shared_gate", bf(np.zeros(H)))
    m.set_q4(layer, "mlp_hc.up", *q4_bias(hh, cfg.hc_lowrank, 0.0))
    gamma = np.array([0.5, -1.0, 0.25, 2.0])
    m.set_q4(layer, "mlp_hc.inject", *q4_bias(hc, hh, gamma[:, None]))
    wm = rng.normal(1, 0.3, hh)
    m.set_bf16(layer, "mlp_hc.norm", bf(wm))
    token = 321
    st.forward_token(token)
    e = np.repeat(f(eb[token]), 64)
    add, _ = twin.new_state().ple(token, np.tile(e, hc).astype(np.float32))
    hyper = np.tile(e, hc) + add.astype(np.float64)
    normed = grouped_norm(hyper, f(wm), H)
    mixed = 0.5 * normed.reshape(hc, H).mean(0)
    X = mixed.sum()
    y = bd * SI * silu(bg * X) * (bu * X)
    inj = 2 * sig(gamma * normed.sum() / hc)
    close(st.last_hyper(), hyper + np.repeat(0.5 * y * inj, H), "hyper after the stack", rtol=1e-5)


def test_ple_state_survives_across_tokens_in_forward_token():
    """forward_token keeps the ring: the second token's logits differ from
    a fresh state's for the same token (the first token's gvn feeds its
    taps only from position 3 on, so run past it)."""
    cfg = ple_cfg()
    m = OracleModel(cfg)
    st = m.new_state()
    toks = [7, 8, 9, 10, 11]
    for t in toks:
        last = st.forward_token(t)
    fresh = m.new_state()
    assert not np.allclose(last, fresh.forward_token(toks[-1]))
