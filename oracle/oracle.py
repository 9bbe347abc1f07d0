"""ctypes bindings of liboracle.so, the C++ restatement of the reference's
CPU path (oracle.cpp).  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product path."""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

from cherenkov_amd.abi import ChkConfig

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

u32, u64, f32, i32, P = C.c_uint32, C.c_uint64, C.c_float, C.c_int, C.c_void_p

_SIGS = [
    ("orc_last_error", C.c_char_p, []),
    ("orc_model_new", P, [C.POINTER(ChkConfig), u32]),
    ("orc_model_free", None, [P]),
    ("orc_state_new", P, [P]),
    ("orc_state_free", None, [P]),
    ("orc_state_pos", u32, [P]),
    ("orc_forward_token", i32, [P, P, u32, i32, P]),
    ("orc_state_last_hyper", i32, [P, P, C.c_size_t]),
    ("orc_mtp_forward", i32, [P, P, u32, P, u32, i32, P, P]),
    ("orc_moe", i32, [P, u32, P, P, P, P, P]),
    ("orc_set_record_bits", i32, [P, u32, u32, u32]),
    ("orc_state_last_selection", i32, [P, P, u32, P, u32, P]),
    ("orc_gated_residual", i32, [P, u32, u32, P, P, P]),
    ("orc_deltanet", i32, [P, P, u32, P, P]),
    ("orc_delta_state", i32, [P, P, u32, P, P]),
    ("orc_attention", i32, [P, P, u32, P, u32, i32, P]),
    ("orc_attention_kv", i32, [P, u32, P, u32, P, P, u32, i32, P]),
    ("orc_q4_matvec", None, [P, P, P, u32, u32, P, P]),
    ("orc_q4_dequant_row", None, [P, P, P, u32, u32, u32, P]),
    ("orc_lowbit_matvec", None, [P, P, P, u32, u32, u32, P, P]),
    ("orc_pack_matrix", None, [P, u64, u32, P]),
    ("orc_q2_slots", None, [P, P]),
    ("orc_q3_slots", None, [P, P, P]),
    ("orc_softmax", None, [P, u32]),
    ("orc_rms_norm", None, [P, P, u32, f32]),
    ("orc_l2_norm", None, [P, u32, f32]),
    ("orc_rope_partial", None, [P, u32, u32, f32]),
    ("orc_softplus", f32, [f32]),
    ("orc_route_topk", None, [P, u32, u32, i32, P, P]),
    ("orc_attend", None, [P, P, P, u32, u32, u32, u32, P]),
    ("orc_delta_head_step", None, [P, P, P, P, f32, f32, u32, u32, P]),
    ("orc_q8_roundtrip", None, [P, u32]),
    ("orc_f32_to_f16", C.c_uint16, [f32]),
    ("orc_causal_conv", None, [P, u32, P, P, u32]),
    ("orc_expert_record", i32, [P, u32, u32, P, u64]),
    ("orc_record_stride", u64, [P]),
    ("orc_qsa_pick", None, [P, u32, u32, u32, P, P]),
    ("orc_state_fill_prefix", i32, [P, P, u32, u64]),
    ("orc_state_route_hints", i32, [P, P, P, u32, f32]),
    ("orc_state_route_swaps", u64, [P]),
    ("orc_state_last_routes", i32, [P, P, u32, P, P]),
    ("orc_set_q4", i32, [P, u32, C.c_char_p, P, P, P, u64]),
    ("orc_set_bf16", i32, [P, u32, C.c_char_p, P, u64]),
    ("orc_set_record", i32, [P, u32, u32, P, u64]),
    ("orc_get_q4", i32, [P, u32, C.c_char_p, P, P, P, u64]),
    ("orc_get_bf16", i32, [P, u32, C.c_char_p, P, u64]),
    ("orc_ngram_ids", i32, [P, P, u32, P, u32, P]),
    ("orc_ple", i32, [P, P, u32, P, P, P]),
    ("orc_ngram_meta", i32, [P, P, P, P, i32]),
    ("orc_ngram_table_bytes", u64, [P]),
    ("orc_ngram_row", i32, [P, u64, P]),
    ("orc_ngram_table", i32, [P, P, u64, i32]),
]

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        L = C.CDLL(str(LIB))
        for n, r, a in _SIGS:
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().orc_last_error().decode())


class OracleModel:
    """CpuModel over the synthetic weights of `cfg` (expert_bits selects the
    low-bit expert reconstruction for Q3/Q2 stores)."""

    def __init__(self, cfg: ChkConfig, expert_bits: int = 4):
        self.cfg = cfg
        self.L = lib()
        self.h = self.L.orc_model_new(C.byref(cfg), expert_bits)
        if not self.h:
            raise RuntimeError(self.L.orc_last_error().decode())

    def __del__(self):
        try:
            if self.h:
                self.L.orc_model_free(self.h)
        except Exception:
            pass

    def new_state(self) -> "OracleState":
        return OracleState(self)

    def set_record_bits(self, record_layer: int, expert: int, bits: int) -> None:
        """One routed-expert record's precision (4, 3 or 2; 0: the model's)."""
        _check(self.L.orc_set_record_bits(self.h, record_layer, expert, bits))

    def moe(self, layer: int, x: np.ndarray):
        c = self.cfg
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(c.hidden_size, np.float32)
        ids = np.empty(c.num_experts_per_tok, np.uint32)
        w = np.empty(c.num_experts_per_tok, np.float32)
        probs = np.empty(c.num_experts, np.float32)
        _check(self.L.orc_moe(self.h, layer, _p(x), _p(out), _p(ids), _p(w), _p(probs)))
        return out, ids, w, probs

    def gated_residual(self, layer: int, which: int, hyper: np.ndarray):
        c = self.cfg
        hyper = np.ascontiguousarray(hyper, dtype=np.float32)
        mixed = np.empty(c.hidden_size, np.float32)
        inj = np.empty(c.hc_count, np.float32)
        _check(self.L.orc_gated_residual(self.h, layer, which, _p(hyper), _p(mixed), _p(inj)))
        return mixed, inj

    def attention_kv(self, layer: int, x: np.ndarray, k: np.ndarray, v: np.ndarray, kv_q8: bool = True):
        """Attention of x rows [rows][H] at positions T.. over a cache of T
        explicit K/V rows; later rows also see earlier rows' K/V."""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        out = np.empty((x.shape[0], self.cfg.hidden_size), np.float32)
        _check(self.L.orc_attention_kv(self.h, layer, _p(x), x.shape[0], _p(k), _p(v), k.shape[0], int(kv_q8), _p(out)))
        return out if x.shape[0] > 1 else out[0]

    def expert_record(self, layer: int, e: int) -> np.ndarray:
        n = self.L.orc_record_stride(self.h)
        out = np.empty(n, np.uint8)
        _check(self.L.orc_expert_record(self.h, layer, e, _p(out), n))
        return out

    # ---- weight overrides: special weights for closed-form checks ----
    def set_q4(self, layer: int, name: str, w: np.ndarray, s: np.ndarray, b: np.ndarray) -> None:
        w = np.ascontiguousarray(w, dtype=np.uint32)
        s = np.ascontiguousarray(s, dtype=np.uint16)
        b = np.ascontiguousarray(b, dtype=np.uint16)
        assert s.size == b.size == w.size // 8
        _check(self.L.orc_set_q4(self.h, layer, name.encode(), _p(w), _p(s), _p(b), w.size))

    def set_bf16(self, layer: int, name: str, v: np.ndarray) -> None:
        v = np.ascontiguousarray(v, dtype=np.uint16)
        _check(self.L.orc_set_bf16(self.h, layer, name.encode(), _p(v), v.size))

    def get_q4(self, layer: int, name: str, out_dim: int, in_dim: int):
        w = np.empty((out_dim, in_dim // 8), np.uint32)
        s = np.empty((out_dim, in_dim // 64), np.uint16)
        b = np.empty((out_dim, in_dim // 64), np.uint16)
        _check(self.L.orc_get_q4(self.h, layer, name.encode(), _p(w), _p(s), _p(b), w.size))
        return w, s, b

    def get_bf16(self, layer: int, name: str, n: int) -> np.ndarray:
        v = np.empty(n, np.uint16)
        _check(self.L.orc_get_bf16(self.h, layer, name.encode(), _p(v), n))
        return v

    def set_record(self, record_layer: int, e: int, rec: np.ndarray) -> None:
        rec = np.ascontiguousarray(rec, dtype=np.uint8)
        _check(self.L.orc_set_record(self.h, record_layer, e, _p(rec), rec.size))

    # ---- PLE ----
    def ngram_heads(self) -> int:
        c = self.cfg
        return (c.ngram_size - 1) * c.heads_per_ngram

    def ngram_ids(self, tokens) -> np.ndarray:
        """ngram_ids_from: the row ids of the last of `tokens`."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(64, np.uint64)
        n = C.c_uint32()
        _check(self.L.orc_ngram_ids(self.h, _p(t), t.size, _p(out), out.size, C.byref(n)))
        return out[: n.value].copy()

    def ngram_meta(self):
        """(multipliers int64 [ngram_size], head offsets, head sizes uint64 [heads])."""
        mult = np.empty(self.cfg.ngram_size, np.int64)
        offs = np.empty(self.ngram_heads(), np.uint64)
        sizes = np.empty(self.ngram_heads(), np.uint64)
        _check(self.L.orc_ngram_meta(self.h, _p(mult), _p(offs), _p(sizes), 0))
        return mult, offs, sizes

    def set_ngram_meta(self, mult, offs, sizes) -> None:
        mult = np.ascontiguousarray(mult, dtype=np.int64)
        offs = np.ascontiguousarray(offs, dtype=np.uint64)
        sizes = np.ascontiguousarray(sizes, dtype=np.uint64)
        assert mult.size == self.cfg.ngram_size and offs.size == sizes.size == self.ngram_heads()
        _check(self.L.orc_ngram_meta(self.h, _p(mult), _p(offs), _p(sizes), 1))

    def ngram_table(self) -> np.ndarray:
        n = self.L.orc_ngram_table_bytes(self.h)
        out = np.empty(n, np.uint8)
        _check(self.L.orc_ngram_table(self.h, _p(out), n, 0))
        return out

    def ngram_row(self, row: int) -> np.ndarray:
        c = self.cfg
        out = np.empty(c.ple_embed_dim // self.ngram_heads(), np.float32)
        _check(self.L.orc_ngram_row(self.h, row, _p(out)))
        return out

    def set_ngram_table(self, t: np.ndarray) -> None:
        t = np.ascontiguousarray(t, dtype=np.uint8)
        _check(self.L.orc_ngram_table(self.h, _p(t), t.size, 1))


class OracleState:
    def __init__(self, m: OracleModel):
        self.m = m
        self.h = m.L.orc_state_new(m.h)

    def __del__(self):
        try:
            self.m.L.orc_state_free(self.h)
        except Exception:
            pass

    @property
    def pos(self) -> int:
        return self.m.L.orc_state_pos(self.h)

    def route_hints(self, ids, tol: float) -> None:
        """Near-tie route hints for the next forward_token / mtp_forward:
        ids[layers][k] (row num_hidden_layers is the MTP layer), taken per
        layer only where they differ from the oracle's own top-k by experts
        within `tol` (relative) of its k-th probability; used once."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        assert ids.ndim == 2 and ids.shape[1] == self.m.cfg.num_experts_per_tok
        _check(self.m.L.orc_state_route_hints(self.m.h, self.h, _p(ids), ids.shape[0], tol))

    def last_routes(self, layer: int):
        """(ids in rank order, softmax) of `layer` in the latest pass."""
        c = self.m.cfg
        ids = np.empty(c.num_experts_per_tok, np.uint32)
        probs = np.empty(c.num_experts, np.float32)
        _check(self.m.L.orc_state_last_routes(self.m.h, self.h, layer, _p(ids), _p(probs)))
        return ids, probs

    @property
    def route_swaps(self) -> int:
        """Layers (cumulative) whose routing followed a hint."""
        return self.m.L.orc_state_route_swaps(self.h)

    def forward_token(self, token: int, kv_q8: bool = True) -> np.ndarray:
        out = np.empty(self.m.cfg.vocab_size, np.float32)
        _check(self.m.L.orc_forward_token(self.m.h, self.h, token, int(kv_q8), _p(out)))
        return out

    def last_selection(self, layer: int) -> list[int]:
        """The tokens the latest query of attention layer `layer` attended
        to (select_tokens, cpu.rs:643-719), ascending."""
        n = C.c_uint32()
        _check(self.m.L.orc_state_last_selection(self.m.h, self.h, layer, None, 0, C.byref(n)))
        out = np.empty(max(1, n.value), np.uint32)
        _check(self.m.L.orc_state_last_selection(self.m.h, self.h, layer, _p(out), n.value, C.byref(n)))
        return out[: n.value].tolist()

    def fill_prefix(self, n: int, seed: int = 1) -> None:
        """Jump to position n with seeded synthetic caches (timing only)."""
        _check(self.m.L.orc_state_fill_prefix(self.m.h, self.h, n, seed))

    def last_hyper(self) -> np.ndarray:
        c = self.m.cfg
        out = np.empty(c.hidden_size * c.hc_count, np.float32)
        _check(self.m.L.orc_state_last_hyper(self.h, _p(out), out.size))
        return out

    def mtp_forward(self, token: int, hyper_in: np.ndarray, pos: int, kv_q8: bool = True):
        c = self.m.cfg
        hyper_in = np.ascontiguousarray(hyper_in, dtype=np.float32)
        logits = np.empty(c.vocab_size, np.float32)
        hy = np.empty(c.hidden_size * c.hc_count, np.float32)
        _check(self.m.L.orc_mtp_forward(self.m.h, self.h, token, _p(hyper_in), pos, int(kv_q8), _p(logits), _p(hy)))
        return logits, hy

    def deltanet(self, layer: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(self.m.cfg.hidden_size, np.float32)
        _check(self.m.L.orc_deltanet(self.m.h, self.h, layer, _p(x), _p(out)))
        return out

    def delta_state(self, layer: int):
        c = self.m.cfg
        s = np.empty(c.linear_num_value_heads * c.linear_key_head_dim * c.linear_value_head_dim, np.float32)
        conv_dim = 2 * c.linear_num_key_heads * c.linear_key_head_dim + c.linear_num_value_heads * c.linear_value_head_dim
        conv = np.empty(conv_dim * (c.linear_conv_kernel_dim - 1), np.float32)
        _check(self.m.L.orc_delta_state(self.m.h, self.h, layer, _p(s), _p(conv)))
        return s, conv

    def attention(self, layer: int, x: np.ndarray, pos: int, kv_q8: bool = True) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(self.m.cfg.hidden_size, np.float32)
        _check(self.m.L.orc_attention(self.m.h, self.h, layer, _p(x), pos, int(kv_q8), _p(out)))
        return out

    def ple(self, token: int, hyper: np.ndarray):
        """The PLE block for the next token (appended to the history) on
        `hyper`: (addend, gvn), each hc * hidden."""
        c = self.m.cfg
        hyper = np.ascontiguousarray(hyper, dtype=np.float32)
        add = np.empty(c.hidden_size * c.hc_count, np.float32)
        gvn = np.empty_like(add)
        _check(self.m.L.orc_ple(self.m.h, self.h, token, _p(hyper), _p(add), _p(gvn)))
        return add, gvn


# ---- primitives ----

def qsa_pick(scores, t_len: int, topk: int, ratio: int) -> np.ndarray:
    """Visible tokens of select_tokens' sparse branch for given block
    scores (cpu.rs:701-716)."""
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    vis = np.empty(topk * ratio + ratio, np.uint32)
    n = C.c_uint32(0)
    lib().orc_qsa_pick(_p(scores), t_len, topk, ratio, _p(vis), C.byref(n))
    return vis[: n.value].copy()


def q4_matvec(w, s, b, out_dim, in_dim, x) -> np.ndarray:
    y = np.empty(out_dim, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().orc_q4_matvec(_p(w), _p(s), _p(b), out_dim, in_dim, _p(x), _p(y))
    return y


def q4_dequant_row(w, s, b, out_dim, in_dim, row) -> np.ndarray:
    y = np.empty(in_dim, np.float32)
    lib().orc_q4_dequant_row(_p(w), _p(s), _p(b), out_dim, in_dim, row, _p(y))
    return y


def lowbit_matvec(w, s, b, out_dim, in_dim, bits, x) -> np.ndarray:
    y = np.empty(out_dim, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().orc_lowbit_matvec(_p(w), _p(s), _p(b), out_dim, in_dim, bits, _p(x), _p(y))
    return y


def pack_matrix(src: np.ndarray, codes: int, bits: int) -> np.ndarray:
    dst = np.zeros(codes * bits // 8, np.uint8)
    src = np.ascontiguousarray(src, dtype=np.uint8)
    lib().orc_pack_matrix(_p(src), codes, bits, _p(dst))
    return dst


def q2_slots():
    t = np.empty(32, np.int32)
    off = np.empty(32, np.uint32)
    lib().orc_q2_slots(_p(t), _p(off))
    return list(zip(t.tolist(), off.tolist()))


def q3_slots():
    t = np.empty(32, np.int32)
    up = np.empty(32, np.uint32)
    lo = np.empty(32, np.uint32)
    lib().orc_q3_slots(_p(t), _p(up), _p(lo))
    return list(zip(t.tolist(), up.tolist(), lo.tolist()))


def softmax(x) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().orc_softmax(_p(x), x.size)
    return x


def rms_norm(x, w_bf16, eps) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    lib().orc_rms_norm(_p(x), _p(w), x.size, eps)
    return x


def l2_norm(x, eps) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().orc_l2_norm(_p(x), x.size, eps)
    return x


def rope_partial(x, pos, rot, theta) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().orc_rope_partial(_p(x), pos, rot, theta)
    return x


def softplus(v: float) -> float:
    return lib().orc_softplus(v)


def attend(qg, k, v, nh: int, nkv: int, hd: int) -> np.ndarray:
    """Attention core over all T cached tokens: qg [nh][2 hd] ([q | gate]
    per head), k, v [T][nkv hd] -> out [nh][hd]."""
    qg = np.ascontiguousarray(qg, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    T = k.size // (nkv * hd)
    out = np.empty(nh * hd, np.float32)
    lib().orc_attend(_p(qg), _p(k), _p(v), T, nh, nkv, hd, _p(out))
    return out.reshape(nh, hd)


def route_topk(probs, k: int, norm: bool):
    """Expert ids in rank order and their (renormalised) weights."""
    p = np.ascontiguousarray(probs, dtype=np.float32)
    ids = np.empty(k, np.uint32)
    w = np.empty(k, np.float32)
    lib().orc_route_topk(_p(p), p.size, k, int(norm), _p(ids), _p(w))
    return ids, w


def delta_head_step(state, q, k, v, decay: float, beta: float):
    """One gated delta-rule step of one value head: returns (new state
    [dk][dv], y [dv]); the input state is not modified."""
    s = np.array(state, dtype=np.float32)
    dk, dv = s.shape
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    y = np.zeros(dv, np.float32)
    lib().orc_delta_head_step(_p(s), _p(q), _p(k), _p(v), decay, beta, dk, dv, _p(y))
    return s, y


def q8_roundtrip(x) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().orc_q8_roundtrip(_p(x), x.size)
    return x


def f32_to_f16_bits(v: float) -> int:
    return lib().orc_f32_to_f16(v)


def causal_conv(qkv, w_bf16, hist, ck):
    qkv = np.array(qkv, dtype=np.float32)
    hist = np.array(hist, dtype=np.float32)
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    lib().orc_causal_conv(_p(qkv), qkv.size, _p(w), _p(hist), ck)
    return qkv, hist
