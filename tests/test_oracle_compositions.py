"""Closed-form pins of the oracle's composed functions (oracle/oracle.cpp):
gated_residual, moe, deltanet, attention (with select_tokens' block
scoring), mtp_forward and forward_token, each run on special weights whose
result is known in closed form, chosen so that a plausible slip (a swapped
operand, a dropped or misplaced term, a wrong head mapping or tie order)
changes the result.  The special weights are Q4 matrices with zero scales,
so that every weight equals its group's bias (quant.rs:24-45: w = s q + b),
and bf16 vectors of exactly representable values.  Expected values are
computed in float64 from the reference formulas' closed forms
(src/qwen4_exp/cpu.rs:328-1085, src/nn.rs:6-56).  CPU only."""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from oracle.oracle import OracleModel
from tests.numerics import bf16_bits, bf16_to_f32

EPS = 1e-6


def sig(v):
    return 1.0 / (1.0 + np.exp(-np.asarray(v, np.float64)))


def silu(v):
    v = np.asarray(v, np.float64)
    return v * sig(v)


def softplus(v):
    return v if v > 20 else np.log1p(np.exp(v))


def q4_bias(out_dim: int, in_dim: int, bias) -> tuple:
    """A Q4 matrix whose every weight in (row, group) is bias[row, group]
    (codes and scales zero)."""
    b = np.broadcast_to(np.asarray(bias, np.float32), (out_dim, in_dim // 64))
    return (np.zeros((out_dim, in_dim // 8), np.uint32), np.zeros((out_dim, in_dim // 64), np.uint16),
            bf16_bits(np.ascontiguousarray(b)))


def bf(v) -> np.ndarray:
    return bf16_bits(np.asarray(v, np.float32))


def f(v) -> np.ndarray:
    """The f64 value of a bf16-representable input."""
    return bf16_to_f32(bf(v)).astype(np.float64)


def grouped_norm(hyper, w, h):
    """grouped_rms_norm (cpu.rs:1012-1027) in f64."""
    out = np.empty_like(hyper, dtype=np.float64)
    for g in range(hyper.size // h):
        x = hyper[g * h:(g + 1) * h].astype(np.float64)
        out[g * h:(g + 1) * h] = x / np.sqrt(np.mean(x * x) + EPS) * w[g * h:(g + 1) * h]
    return out


def close(got, want, label, rtol=2e-5):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(1e-6, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(got - want)))
    assert err <= rtol * scale, f"{label}: max-abs {err:.3e} vs scale {scale:.3e}"


# ------------------------------------------------------------ gated_residual

@pytest.mark.parametrize("which", [0, 2])
def test_gated_residual_closed_form(which):
    """gated_residual (cpu.rs:459-500) with down = beta, up = c, inject row g
    = gamma_g everywhere: d_j = silu(beta N / hc) for N = sum(normed), u =
    c * lowrank * d, mixed = sigmoid(u) * mean over streams of normed,
    inj_g = 2 sigmoid(gamma_g N / hc).  Streams at very different scales
    make `normed` differ from `hyper`."""
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    H, hc, lr = cfg.hidden_size, cfg.hc_count, cfg.hc_lowrank
    hh = H * hc
    layer = 1
    grp = "attn_hc" if which == 0 else "final"
    beta, c = 0.125, 0.25
    gamma = np.array([0.5, -0.5, 1.0, -1.0])
    m.set_q4(layer, f"{grp}.down", *q4_bias(lr, hh, beta))
    m.set_q4(layer, f"{grp}.up", *q4_bias(hh, lr, c))
    if which == 0:
        m.set_q4(layer, f"{grp}.inject", *q4_bias(hc, hh, gamma[:, None]))
    rng = np.random.default_rng(31)
    norm_w = rng.normal(1.0, 0.3, hh)
    m.set_bf16(layer, f"{grp}.norm", bf(norm_w))
    w = f(norm_w)
    scales = np.repeat([0.1, 1.0, 10.0, 3.0], H)
    hyper = (rng.normal(0, 1, hh) * scales).astype(np.float32)
    mixed, inj = m.gated_residual(layer, which, hyper)
    normed = grouped_norm(hyper, w, H)
    N = normed.sum()
    d = silu(beta * N / hc)
    u = c * lr * d
    want = sig(u) * normed.reshape(hc, H).mean(axis=0)
    close(mixed, want, "mixed")
    if which == 0:
        close(inj, 2 * sig(gamma * N / hc), "inj")


# ---------------------------------------------------------------------- moe

def expert_record(cfg, rec_len, bg, bu, bd) -> np.ndarray:
    """A Q4 expert record (pack.rs:351-393 field order) whose gate, up and
    down weights are the constants bg, bu, bd."""
    I, H = cfg.moe_intermediate_size, cfg.hidden_size
    codes = I * H
    rec = np.zeros(rec_len, np.uint8)
    off = 3 * codes // 2
    sb = I * (H // 64) * 2
    sd = H * (I // 64) * 2
    fields = [("gate_s", sb, 0.0), ("gate_b", sb, bg), ("up_s", sb, 0.0), ("up_b", sb, bu), ("down_s", sd, 0.0),
              ("down_b", sd, bd)]
    for _, n, v in fields:
        rec[off:off + n] = np.full(n // 2, bf16_bits(np.float32(v))[0], np.uint16).view(np.uint8)
        off += n
    return rec


def test_moe_closed_form():
    """moe (cpu.rs:504-541): router row e = alpha_e e_0 so logits are alpha_e
    x_0; the top-2 experts (15, 14) and the shared expert have constant
    gate/up/down weights, so each expert's output is the constant
    bd I silu(bg X) (bu X) for X = sum(x); the routed weights are the
    renormalised softmax probabilities and the shared term is scaled by
    sigmoid(gamma x_1).  bg != bu catches a swapped gate/up."""
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    H, E, I, k = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size, cfg.num_experts_per_tok
    layer = 0
    alpha = (np.arange(E) - 7) * 0.25
    router = np.zeros((E, H), np.float32)
    router[:, 0] = alpha
    m.set_bf16(layer, "moe.router", bf(router))
    gamma = -0.75
    sg = np.zeros(H, np.float32)
    sg[1] = gamma
    m.set_bf16(layer, "moe.shared_gate", bf(sg))
    params = {15: (0.5, -0.25, 0.125), 14: (-0.375, 0.75, 0.25)}
    n = len(m.expert_record(layer, 0))
    for e, (bg, bu, bd) in params.items():
        m.set_record(layer, e, expert_record(cfg, n, bg, bu, bd))
    sh = (0.25, 0.5, -0.0625)
    SI = cfg.shared_expert_intermediate_size
    m.set_q4(layer, "moe.sh_gate", *q4_bias(SI, H, sh[0]))
    m.set_q4(layer, "moe.sh_up", *q4_bias(SI, H, sh[1]))
    m.set_q4(layer, "moe.sh_down", *q4_bias(H, SI, sh[2]))
    rng = np.random.default_rng(32)
    x = (rng.normal(0, 0.05, H)).astype(np.float32)
    x[0], x[1] = 1.5, 0.5
    out, ids, wts, probs = m.moe(layer, x)
    logits = f(alpha) * 1.5
    p = np.exp(logits - logits.max())
    p /= p.sum()
    close(probs, p, "router softmax", rtol=1e-6)
    assert ids.tolist() == [15, 14]
    wt = p[[15, 14]] / p[[15, 14]].sum()
    close(wts, wt, "renormalised weights", rtol=1e-6)
    X = float(np.sum(x.astype(np.float64)))
    y = lambda bg, bu, bd, width: bd * width * silu(bg * X) * (bu * X)
    want = wt[0] * y(*params[15], I) + wt[1] * y(*params[14], I) + sig(gamma * 0.5) * y(*sh, SI)
    close(out, np.full(H, want), "moe out", rtol=1e-4)
    assert k == 2


# ----------------------------------------------------------------- deltanet

def test_deltanet_two_steps_closed_form():
    """deltanet (cpu.rs:722-826) over two tokens with projections chosen per
    channel (x = 1 on the first group, so each output is 64 x its row's
    group-0 bias) and conv weights [.., 0.5, 1]: step 1 sees silu(u), step 2
    silu(1.5 u).  q and k per key head are fixed directions, v per value
    head random; decay = exp(-exp(A_log) softplus(a + dt_bias)), beta =
    sigmoid(b).  The state after each step is S1 = beta k1 v1^T and
    S2 = decay S1 + k2 (beta (v2 - decay S1^T k2))^T ([k][v] per value
    head, value head h on key head h / (nv / nk)); the output is
    out_proj(rmsnorm(S^T q) w sigmoid(z)) with out_proj row r summing
    group r % G of y."""
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    st = m.new_state()
    H = cfg.hidden_size
    nk, nv, dk, dv = (cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                      cfg.linear_value_head_dim)
    ck = cfg.linear_conv_kernel_dim
    qk, vd = nk * dk, nv * dv
    conv_dim = 2 * qk + vd
    layer = 0
    rng = np.random.default_rng(33)

    def proj(name, rows, vals):
        b = np.zeros((rows, H // 64), np.float32)
        b[:, 0] = np.asarray(vals, np.float32) / 64.0
        m.set_q4(layer, name, *q4_bias(rows, H, b))
        return f(b[:, 0]) * 64.0

    pre = np.zeros(conv_dim, np.float32)
    for h in range(nk):
        pre[h * dk + h] = 1.0                   # q of key head h along dim h
        pre[qk + h * dk + h] = 0.5              # k of key head h: dims h and h + 7
        pre[qk + h * dk + h + 7] = -1.0
    pre[2 * qk:] = rng.normal(0, 1, vd)
    pre = proj("dn.qkv", conv_dim, pre)
    z = proj("dn.z", vd, rng.normal(0, 1, vd))
    a_in = proj("dn.a", nv, rng.normal(0, 1, nv))
    b_in = proj("dn.b", nv, rng.normal(0, 1, nv))
    conv = np.zeros((conv_dim, ck), np.float32)
    conv[:, ck - 1] = 1.0
    conv[:, ck - 2] = 0.5
    m.set_bf16(layer, "dn.conv", bf(conv))
    a_log = rng.normal(0, 0.5, nv)
    dt = rng.normal(0, 0.5, nv)
    m.set_bf16(layer, "dn.a_log", bf(a_log))
    m.set_bf16(layer, "dn.dt_bias", bf(dt))
    nw = rng.normal(1, 0.2, dv)
    m.set_bf16(layer, "dn.norm", bf(nw))
    G = vd // 64
    ob = np.zeros((H, G), np.float32)
    ob[np.arange(H), np.arange(H) % G] = 1.0
    m.set_q4(layer, "dn.out", *q4_bias(H, vd, ob))
    a_log, dt, nw = f(a_log), f(dt), f(nw)
    x = np.zeros(H, np.float32)
    x[:64] = 1.0
    S = np.zeros((nv, dk, dv))
    decay = np.exp(-np.exp(a_log) * np.array([softplus(a + d) for a, d in zip(a_in, dt)]))
    beta = sig(b_in)
    for step, gain in ((0, 1.0), (1, 1.5)):
        o = st.deltanet(layer, x)
        u = silu(gain * pre)
        q = u[:qk].reshape(nk, dk)
        kk = u[qk:2 * qk].reshape(nk, dk)
        v = u[2 * qk:].reshape(nv, dv)
        q = q / np.sqrt((q * q).sum(1, keepdims=True) + 1e-6) * dk ** -0.5
        kk = kk / np.sqrt((kk * kk).sum(1, keepdims=True) + 1e-6)
        y = np.zeros((nv, dv))
        for h in range(nv):
            hk = h // (nv // nk)
            S[h] *= decay[h]
            delta = beta[h] * (v[h] - S[h].T @ kk[hk])
            S[h] += np.outer(kk[hk], delta)
            yh = S[h].T @ q[hk]
            y[h] = yh / np.sqrt(np.mean(yh * yh) + 1e-6) * nw * sig(z[h * dv:(h + 1) * dv])
        s_got, c_got = st.delta_state(layer)
        close(s_got.reshape(nv, dk, dv), S, f"state after step {step + 1}", rtol=1e-5)
        hist = np.tile(pre[:, None], (1, ck - 1)) * np.array([[0.0] * (ck - 2) + [1.0]])
        if step:
            hist[:, ck - 3] = pre
        close(c_got.reshape(conv_dim, ck - 1), hist, f"conv history after step {step + 1}", rtol=0)
        gs = y.reshape(G, 64).sum(1)
        close(o, gs[np.arange(H) % G], f"output after step {step + 1}", rtol=1e-4)


# ---------------------------------------------------------------- attention

def attn_setup(cfg, m, layer, rng, tok_vals):
    """Projections that give token t (x = 1 on group t) the rows
    tok_vals[t] = (q, gate, k, v, idx) per head; norms 1."""
    H = cfg.hidden_size
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    ihd, inh = cfg.indexer_head_dim, cfg.indexer_n_heads
    G = H // 64
    qb = np.zeros((2 * nh * hd, G), np.float32)
    kb = np.zeros((nkv * hd, G), np.float32)
    vb = np.zeros((nkv * hd, G), np.float32)
    ib = np.zeros(((inh + 1) * ihd, G), np.float32)
    for t, (q, gate, k, v, idx) in enumerate(tok_vals):
        for h in range(nh):
            qb[h * 2 * hd:h * 2 * hd + hd, t] = q[h] / 64
            qb[h * 2 * hd + hd:(h + 1) * 2 * hd, t] = gate[h] / 64
        kb[:, t] = k.ravel() / 64
        vb[:, t] = v.ravel() / 64
        ib[:, t] = idx.ravel() / 64
    for name, rows, b in (("at.q", 2 * nh * hd, qb), ("at.k", nkv * hd, kb), ("at.v", nkv * hd, vb),
                          ("at.idx", (inh + 1) * ihd, ib)):
        m.set_q4(layer, name, *q4_bias(rows, H, b))
    for name, n in (("at.q_norm", hd), ("at.k_norm", hd), ("at.idx_q_norm", ihd), ("at.idx_k_norm", ihd)):
        m.set_bf16(layer, name, bf(np.ones(n)))
    ob = np.zeros((H, nh * hd // 64), np.float32)
    ob[np.arange(H), np.arange(H) % (nh * hd // 64)] = 1.0
    m.set_q4(layer, "at.o", *q4_bias(H, nh * hd, ob))
    def as64(a):  # the value a row carries: 64 x its bf16 bias
        return bf16_to_f32(bf16_bits(np.asarray(a, np.float32) / 64)).astype(np.float64) * 64

    return [tuple(as64(a) for a in tv) for tv in tok_vals]


def rms(x):
    return x / np.sqrt(np.mean(x * x) + EPS)


def attn_out(cfg, vals, t_q, visible):
    """Output of attention for query token t_q over visible tokens (f32 KV;
    q and k live outside the rotated dims, so RoPE leaves them)."""
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    grp = nh // nkv
    q, gate = vals[t_q][0], vals[t_q][1]
    out = np.zeros((nh, hd))
    for h in range(nh):
        hk = h // grp
        qh = rms(q[h])
        s = np.array([hd ** -0.5 * qh @ rms(vals[t][2][hk]) for t in visible])
        p = np.exp(s - s.max())
        p /= p.sum()
        o = sum(pi * vals[t][3][hk] for pi, t in zip(p, visible))
        out[h] = o * sig(gate[h])
    G = nh * hd // 64
    gs = out.ravel().reshape(G, 64).sum(1)
    return gs[np.arange(cfg.hidden_size) % G]


def test_attention_closed_form():
    """attention (cpu.rs:544-641) for two tokens: per head the rows are
    [q | gate] (cpu.rs:577-582), q and k are RMS-normed per head, scores
    scaled by hd^-0.5, softmax over the visible tokens, the output gated
    by sigmoid(gate), kv head h / (nh / nkv) serves query head h (distinct
    values per kv head catch a wrong mapping), o_proj row r sums group
    r % G.  q and k sit outside the rotated dims, so RoPE leaves them."""
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    st = m.new_state()
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    rot = int(hd * cfg.partial_rotary_factor)
    inh, ihd = cfg.indexer_n_heads, cfg.indexer_head_dim
    rng = np.random.default_rng(34)
    toks = []
    for t in range(2):
        q = np.zeros((nh, hd))
        q[:, rot:] = rng.normal(0, 1, (nh, hd - rot))
        k = np.zeros((nkv, hd))
        k[:, rot:] = rng.normal(0, 1, (nkv, hd - rot))
        toks.append((q, rng.normal(0, 1, (nh, hd)), k, rng.normal(0, 1, (nkv, hd)), rng.normal(0, 1, (inh + 1, ihd))))
    layer = 3
    vals = attn_setup(cfg, m, layer, rng, toks)
    for t in range(2):
        x = np.zeros(cfg.hidden_size, np.float32)
        x[t * 64:(t + 1) * 64] = 1.0
        o = st.attention(layer, x, t, kv_q8=False)  # the layer's own cache, f32 KV
        close(o, attn_out(cfg, vals, t, list(range(t + 1))), f"attention token {t}", rtol=1e-4)


@pytest.mark.parametrize("case", ["tie", "relu"])
def test_select_tokens_block_scores(case):
    """select_tokens (cpu.rs:643-719) past the budget (2 blocks of 4 kept):
    the tokens of block b carry one index key whose direction u_b (dims
    outside the rotated ones) is chosen per case; the pooled, RMS-normed
    key is then sqrt(ihd) u_b, and with index query heads along e_j and
    -e_j' a block scores relu(u_j) + relu(-u_j') (times 1, after the
    1/sqrt(ihd)).  "tie": scores 1, 1, 1.41, 0.71: block 2 and, of the tied
    0 and 1, the lower.  "relu": scores 1.41, 0.71 (0 without the relu),
    0.6: blocks 0 and 1.  Every query/key dot is 0, so the attention is
    uniform over the kept blocks and the query's own tail token, whose
    distinct values the output shows."""
    budget, ratio = 8, 4
    cfg = presets.tiny(mtp=0, indexer_budget=budget)
    assert cfg.indexer_compress_ratio == ratio
    m = OracleModel(cfg)
    st = m.new_state()
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    inh, ihd = cfg.indexer_n_heads, cfg.indexer_head_dim
    assert inh == 2
    rot = int(hd * cfg.partial_rotary_factor)
    j, j2, j3 = rot + 3, rot + 9, rot + 20
    r2 = 1 / np.sqrt(2)
    dirs = {"tie": [(1, 0, 0), (0, -1, 0), (r2, -r2, 0), (r2, r2, 0)],
            "relu": [(r2, -r2, 0), (r2, r2, 0), (0.6, 0, 0.8)]}[case]
    want_keep = {"tie": [0, 2], "relu": [0, 1]}[case]
    nb = len(dirs)
    n_tok = ratio * nb + 1
    rng = np.random.default_rng(35)
    groups = []
    for blk in range(nb + 1):  # one x group (projection column) per block, the last for the query
        q = np.zeros((nh, hd))
        q[:, hd - 1] = 1.0
        k = np.zeros((nkv, hd))
        k[:, hd - 2] = 1.0
        v = (blk + 1) * (1.0 + 0.01 * np.arange(hd))[None, :].repeat(nkv, 0)
        v[1] *= -0.5
        idx = np.zeros((inh + 1, ihd))
        idx[0, j] = 1.0
        idx[1, j2] = -1.0
        if blk < nb:
            idx[inh, [j, j2, j3]] = dirs[blk]
        groups.append((q, rng.normal(0, 1, (nh, hd)), k, v, idx))
    layer = 3
    vals_g = attn_setup(cfg, m, layer, rng, groups)
    vals = [vals_g[min(t // ratio, nb)] for t in range(n_tok)]
    out = None
    for t in range(n_tok):
        x = np.zeros(cfg.hidden_size, np.float32)
        g = min(t // ratio, nb)
        x[g * 64:(g + 1) * 64] = 1.0
        out = st.attention(layer, x, t, kv_q8=False)
    qn = [rms(vals[-1][4][h]) for h in range(inh)]
    scores = []
    for blk in range(nb):
        key = rms(vals[blk * ratio][4][inh])  # pooled mean of equal keys, normed
        scores.append(sum(max(0.0, qh @ key) for qh in qn) / np.sqrt(ihd))
    keep = sorted(sorted(range(nb), key=lambda b: (-scores[b], b))[:budget // ratio])
    assert keep == want_keep, (scores, keep)
    visible = [t for b in keep for t in range(b * ratio, (b + 1) * ratio)] + [n_tok - 1]
    close(out, attn_out(cfg, vals, n_tok - 1, visible), f"{case}: attention over the kept blocks", rtol=1e-4)


# ------------------------------------------- RoPE positions (relative angles)

def rel_dot(a, b, shift, rot, theta):
    """a . b after rotating a by position p_a and b by p_b under rotate-half
    RoPE on the first `rot` dims, p_a - p_b = shift: pair j = (j, j + rot/2)
    is a complex number turned by p * theta^(-2j/rot), so the pair's share of
    the dot is Re(a_j conj(b_j) e^{i shift w_j}) (the rotation group's
    relative-angle identity); dims past `rot` add their plain product."""
    half = rot // 2
    w = float(theta) ** (-2.0 * np.arange(half) / rot)
    ac = a[:half] + 1j * a[half:rot]
    bc = b[:half] + 1j * b[half:rot]
    return float(np.sum((ac * np.conj(bc) * np.exp(1j * shift * w)).real) + a[rot:] @ b[rot:])


def test_attention_rope_relative_positions():
    """attention (cpu.rs:544-641) with q and k inside the rotated dims
    (cpu.rs:575-587: q rotated at the query's position, k at its own, both
    after the per-head norm): the score of query token p against key token t
    is hd^-1/2 rel_dot(q^, k^, p - t), so the softmax weights depend on
    p - t through every pair's frequency.  Six tokens, each attended over
    its causal prefix; a rotation at the wrong position for q (p + 1, 0) or
    k (unrotated, the query's position) moves the weights by orders of
    magnitude more than the tolerance."""
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    st = m.new_state()
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    rot = int(hd * cfg.partial_rotary_factor)
    inh, ihd = cfg.indexer_n_heads, cfg.indexer_head_dim
    rng = np.random.default_rng(36)
    n_tok = 6
    toks = []
    for t in range(n_tok):
        q = rng.normal(0, 0.3, (nh, hd))
        q[:, :rot] = rng.normal(0, 2.0, (nh, rot))
        k = rng.normal(0, 0.3, (nkv, hd))
        k[:, :rot] = rng.normal(0, 2.0, (nkv, rot))
        toks.append((q, rng.normal(0, 1, (nh, hd)), k, rng.normal(0, 1, (nkv, hd)),
                     rng.normal(0, 1, (inh + 1, ihd))))
    layer = 3
    vals = attn_setup(cfg, m, layer, rng, toks)
    grp = nh // nkv
    G = nh * hd // 64

    def expect(p, q_shift=0, k_pos=None):
        out = np.zeros((nh, hd))
        for h in range(nh):
            hk = h // grp
            qh = rms(vals[p][0][h])
            s = np.array([hd ** -0.5 * rel_dot(qh, rms(vals[t][2][hk]),
                                               p + q_shift - (t if k_pos is None else k_pos(t, p)),
                                               rot, cfg.rope_theta) for t in range(p + 1)])
            pr = np.exp(s - s.max())
            pr /= pr.sum()
            out[h] = sum(pi * vals[t][3][hk] for pi, t in zip(pr, range(p + 1))) * sig(vals[p][1][h])
        gs = out.ravel().reshape(G, 64).sum(1)
        return gs[np.arange(cfg.hidden_size) % G]

    for p in range(n_tok):
        x = np.zeros(cfg.hidden_size, np.float32)
        x[p * 64:(p + 1) * 64] = 1.0
        o = st.attention(layer, x, p, kv_q8=False)
        want = expect(p)
        close(o, want, f"attention with rotated q/k, token {p}", rtol=1e-4)
        if p >= 2:  # the same closed form with a slipped position is far off
            scale = float(np.max(np.abs(want)))
            for label, wrong in (("q at p+1", expect(p, q_shift=1)), ("q at 0", expect(p, q_shift=-p)),
                                 ("k unrotated", expect(p, k_pos=lambda t, pp: 0)),
                                 ("k at the query's position", expect(p, k_pos=lambda t, pp: pp))):
                assert float(np.max(np.abs(wrong - want))) > 100 * 1e-4 * scale, label


def test_select_tokens_rope_positions():
    """select_tokens (cpu.rs:643-719) past the budget with the index query
    and the block keys inside the rotated dims (cpu.rs:676-690): the index
    query heads are rotated at the query's position p and block b's pooled,
    normed key at b * ratio, so head h scores relu(ihd cos(psi_h + p -
    phi_b - b ratio)) / sqrt(ihd) for a query of angle psi_h and a key of
    angle phi_b in the first rotated pair (frequency 1 rad per position).
    The angles are chosen so that the two kept blocks of four differ from
    the correct ones (the test checks this) if the query is rotated at 0,
    p - 1 or p + 1, or the keys at p, b, 0, (b + 1) ratio - 1 or
    (b + 1) ratio; the query/key dots of the attention proper are 0, so the
    output shows which blocks are kept."""
    budget, ratio = 8, 4
    cfg = presets.tiny(mtp=0, indexer_budget=budget)
    assert cfg.indexer_compress_ratio == ratio
    m = OracleModel(cfg)
    st = m.new_state()
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    inh, ihd = cfg.indexer_n_heads, cfg.indexer_head_dim
    assert inh == 2
    rot = int(hd * cfg.partial_rotary_factor)
    half = rot // 2
    psi = [1.11, -0.61]
    phi = [2.11, 0.45, -2.7, -2.69]
    nb = len(phi)
    n_tok = ratio * nb + 1
    p = n_tok - 1
    rng = np.random.default_rng(37)
    groups = []
    for blk in range(nb + 1):
        q = np.zeros((nh, hd))
        q[:, hd - 1] = 1.0
        k = np.zeros((nkv, hd))
        k[:, hd - 2] = 1.0
        v = (blk + 1) * (1.0 + 0.01 * np.arange(hd))[None, :].repeat(nkv, 0)
        v[1] *= -0.5
        idx = np.zeros((inh + 1, ihd))
        for h in range(inh):
            idx[h, 0], idx[h, half] = np.cos(psi[h]), np.sin(psi[h])
        if blk < nb:
            idx[inh, 0], idx[inh, half] = np.cos(phi[blk]), np.sin(phi[blk])
        groups.append((q, rng.normal(0, 1, (nh, hd)), k, v, idx))
    layer = 3
    vals_g = attn_setup(cfg, m, layer, rng, groups)
    vals = [vals_g[min(t // ratio, nb)] for t in range(n_tok)]
    qn = [rms(vals[-1][4][h]) for h in range(inh)]

    def kept(q_pos, k_pos):
        scores = []
        for blk in range(nb):
            key = rms(vals[blk * ratio][4][inh])
            scores.append(sum(max(0.0, rel_dot(qh, key, q_pos - k_pos(blk), rot, cfg.rope_theta)) for qh in qn)
                          / np.sqrt(ihd))
        order = sorted(range(nb), key=lambda b: (-scores[b], b))
        s = sorted(scores, reverse=True)
        assert s[budget // ratio - 1] - s[budget // ratio] > 1.0, scores  # no near-tie at the cut
        return sorted(order[:budget // ratio])

    keep = kept(p, lambda b: b * ratio)
    for label, q_pos, k_pos in (("q at 0", 0, lambda b: b * ratio), ("q at p-1", p - 1, lambda b: b * ratio),
                                ("q at p+1", p + 1, lambda b: b * ratio), ("keys at p", p, lambda b: p),
                                ("keys at b", p, lambda b: b), ("keys at 0", p, lambda b: 0),
                                ("keys at the block end", p, lambda b: (b + 1) * ratio - 1),
                                ("keys at the next block", p, lambda b: (b + 1) * ratio)):
        assert kept(q_pos, k_pos) != keep, label
    out = None
    for t in range(n_tok):
        x = np.zeros(cfg.hidden_size, np.float32)
        g = min(t // ratio, nb)
        x[g * 64:(g + 1) * 64] = 1.0
        out = st.attention(layer, x, t, kv_q8=False)
    visible = [t for b in keep for t in range(b * ratio, (b + 1) * ratio)] + [n_tok - 1]
    close(out, attn_out(cfg, vals, n_tok - 1, visible), "attention over the blocks kept by rotated scores",
          rtol=1e-4)


# ---------------------------------------------------------------- MTP head

def zero_layer_outputs(cfg, m, layer):
    """Mixer and MoE outputs of `layer` become 0 (o/out projections, shared
    and routed down weights zero), so its injections add nothing."""
    H = cfg.hidden_size
    linear = layer < cfg.num_hidden_layers and (layer + 1) % cfg.full_attention_interval != 0
    if linear:
        m.set_q4(layer, "dn.out", *q4_bias(H, cfg.linear_num_value_heads * cfg.linear_value_head_dim, 0.0))
    else:
        m.set_q4(layer, "at.o", *q4_bias(H, cfg.num_attention_heads * cfg.head_dim, 0.0))
    m.set_q4(layer, "moe.sh_down", *q4_bias(H, cfg.shared_expert_intermediate_size, 0.0))
    n = len(m.expert_record(0, 0))
    rec = expert_record(cfg, n, 0.0, 0.0, 0.0)
    for e in range(cfg.num_experts):
        m.set_record(layer, e, rec)


def test_mtp_forward_closed_form():
    """mtp_forward (cpu.rs:328-389): e = embed(token) and each trunk stream
    h_g pass the (1 + w) RMSNorm (rms_norm_shift, cpu.rs:999-1008: w = 0
    is the plain norm, w = -1 zeroes); fc_e = c_e, fc_h = c_h make
    hyper_g = c_e sum(rms(e)) + c_h sum(rms(h_g)), a constant per stream;
    the MTP layer's outputs are zeroed, the MTP mixer's up is zero
    (sigmoid 1/2) and lm_head row r is beta_r, so logits_r = beta_r *
    sum(1/2 mean_g sign(hyper_g) w_g)."""
    cfg = presets.tiny(mtp=1)
    m = OracleModel(cfg)
    st = m.new_state()
    H, hc, L = cfg.hidden_size, cfg.hc_count, cfg.num_hidden_layers
    hh = H * hc
    rng = np.random.default_rng(36)
    ce, ch = 0.5, -0.25
    m.set_bf16(L, "mtp.enorm", bf(np.zeros(H)))
    hn = np.zeros(hh)
    hn[H:2 * H] = -1.0  # stream 1 is zeroed by the (1 + w) convention
    m.set_bf16(L, "mtp.hnorm", bf(hn))
    m.set_q4(L, "mtp.fc_e", *q4_bias(H, H, ce))
    m.set_q4(L, "mtp.fc_h", *q4_bias(H, H, ch))
    zero_layer_outputs(cfg, m, L)
    m.set_q4(L, "mtp_mixer.up", *q4_bias(hh, cfg.hc_lowrank, 0.0))
    mw = rng.normal(1, 0.3, hh)
    m.set_bf16(L, "mtp_mixer.norm", bf(mw))
    beta = rng.normal(0, 1, cfg.vocab_size)
    m.set_q4(L, "lm_head", *q4_bias(cfg.vocab_size, H, beta[:, None]))
    eb = rng.normal(0, 1, (cfg.vocab_size, H // 64))
    m.set_q4(L, "embed", *q4_bias(cfg.vocab_size, H, eb))
    st.forward_token(7)
    h_in = rng.normal(0, 1, hh).astype(np.float32) * np.repeat([1.0, 5.0, 0.2, 2.0], H).astype(np.float32)
    token = 11
    logits, hyper = st.mtp_forward(token, h_in, 0)
    e = np.repeat(f(eb[token]), 64)  # the embedding row: its group biases
    se = np.sum(rms(e))
    want_h = np.empty(hh)
    for g in range(hc):
        hg = h_in[g * H:(g + 1) * H].astype(np.float64)
        sh = 0.0 if g == 1 else np.sum(rms(hg))
        want_h[g * H:(g + 1) * H] = ce * se + ch * sh
    close(hyper, want_h, "MTP hyper", rtol=1e-4)
    normed = grouped_norm(want_h, f(mw), H)
    mixed = 0.5 * normed.reshape(hc, H).mean(0)
    close(logits, f(beta) * mixed.sum(), "MTP logits", rtol=1e-4)


# ------------------------------------------------------------ forward_token

def test_forward_token_closed_form():
    """forward_token (cpu.rs:392-456): the embedding row replicated into
    every stream; every mixer and MoE output zeroed except layer 0's MoE,
    whose only non-zero part is the shared expert (constant weights, gate
    vector 0: sigmoid 1/2) behind an mlp_hc read with zero up (mixed = 1/2
    mean of normed streams) and inject biases gamma_g: after layer 0,
    hyper_g = e + 1/2 y inj_g with inj_g = 2 sigmoid(gamma_g N / hc); the
    attn_hc inject (different biases) must not apply.  The final mixer
    (zero up, no inject) and lm_head rows beta_r give logits_r = beta_r
    sum(mixed)."""
    cfg = presets.tiny(mtp=0)
    m = OracleModel(cfg)
    st = m.new_state()
    H, hc, V = cfg.hidden_size, cfg.hc_count, cfg.vocab_size
    hh = H * hc
    SI = cfg.shared_expert_intermediate_size
    rng = np.random.default_rng(37)
    eb = rng.normal(0, 1, (V, H // 64))
    m.set_q4(0, "embed", *q4_bias(V, H, eb))
    for layer in range(cfg.num_hidden_layers):
        zero_layer_outputs(cfg, m, layer)
    bg, bu, bd = 0.25, -0.5, 0.125
    m.set_q4(0, "moe.sh_gate", *q4_bias(SI, H, bg))
    m.set_q4(0, "moe.sh_up", *q4_bias(SI, H, bu))
    m.set_q4(0, "moe.sh_down", *q4_bias(H, SI, bd))
    m.set_bf16(0, "moe.shared_gate", bf(np.zeros(H)))
    m.set_q4(0, "mlp_hc.up", *q4_bias(hh, cfg.hc_lowrank, 0.0))
    gamma = np.array([0.5, -1.0, 0.25, 2.0])
    m.set_q4(0, "mlp_hc.inject", *q4_bias(hc, hh, gamma[:, None]))
    m.set_q4(0, "attn_hc.inject", *q4_bias(hc, hh, -gamma[:, None]))
    wm = rng.normal(1, 0.3, hh)
    m.set_bf16(0, "mlp_hc.norm", bf(wm))
    m.set_q4(0, "final.up", *q4_bias(hh, cfg.hc_lowrank, 0.0))
    wf = rng.normal(1, 0.3, hh)
    m.set_bf16(0, "final.norm", bf(wf))
    beta = rng.normal(0, 1, V)
    m.set_q4(0, "lm_head", *q4_bias(V, H, beta[:, None]))
    token = 123
    logits = st.forward_token(token)
    e = np.repeat(f(eb[token]), 64)
    hyper = np.tile(e, hc)
    normed = grouped_norm(hyper, f(wm), H)
    mixed = 0.5 * normed.reshape(hc, H).mean(0)
    X = mixed.sum()
    y = bd * SI * silu(bg * X) * (bu * X)
    inj = 2 * sig(gamma * normed.sum() / hc)
    hyper = hyper + np.repeat(0.5 * y * inj, H)
    close(st.last_hyper(), hyper, "hyper after the stack", rtol=1e-5)
    nf = grouped_norm(hyper, f(wf), H)
    close(logits, f(beta) * (0.5 * nf.reshape(hc, H).mean(0)).sum(), "logits", rtol=1e-4)
