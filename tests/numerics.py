"""Independent numpy helpers of the CPU and GPU parity tests: bf16/f16
conversions, the reference tests' LCG, and the Q2/Q3 chunk unpackers
written from the slot tables' definition (not from the oracle's code)."""

from __future__ import annotations

import numpy as np

MASK64 = (1 << 64) - 1


def bf16_bits(x) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_round(x) -> np.ndarray:
    """IEEE binary16 round-to-nearest-even and back (numpy's cast)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


class Lcg:
    """The reference GPU tests' generator (tests/unit/qwen4_exp/gpu/mod.rs:12-23):
    a 64-bit LCG whose top 24 bits of state map to [-1, 1).  `fill` draws
    n values at once with a jump-ahead table (state_{i} = A_i s + C_i mod
    2^64), the same sequence as n calls of `f`."""

    A = 6364136223846793005
    C = 1442695040888963407
    _BLOCK = 4096
    _tab = None

    def __init__(self, seed: int):
        self.state = seed & MASK64

    @staticmethod
    def _value(s):
        return (np.asarray(s >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0)

    def f(self) -> float:
        self.state = (self.state * self.A + self.C) & MASK64
        return float(self._value(np.uint64(self.state)))

    @classmethod
    def _table(cls):
        if cls._tab is None:
            a = np.empty(cls._BLOCK, np.uint64)
            c = np.empty(cls._BLOCK, np.uint64)
            ai, ci = 1, 0
            for i in range(cls._BLOCK):
                ai = (ai * cls.A) & MASK64
                ci = (ci * cls.A + cls.C) & MASK64
                a[i], c[i] = ai, ci
            cls._tab = (a, c)
        return cls._tab

    def fill(self, n: int) -> np.ndarray:
        a, c = self._table()
        out = np.empty(n, np.float32)
        done = 0
        with np.errstate(over="ignore"):
            while done < n:
                m = min(self._BLOCK, n - done)
                st = a[:m] * np.uint64(self.state) + c[:m]
                out[done:done + m] = self._value(st)
                self.state = int(st[-1])
                done += m
        return out


def rust_round(x: np.ndarray) -> np.ndarray:
    """f32::round: half away from zero."""
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def mlx_quantize(rows: np.ndarray):
    """The affine Q4 g64 quantizer of the reference's matvec test
    (tests/unit/quant.rs:5-40): per 64-group scale = max((max-min)/15, 1e-8),
    bias = min, both stored bf16; q = round((v - b) / s) clamped to 0..15,
    8 nibbles per u32 LSB-first."""
    rows = np.asarray(rows, dtype=np.float32)
    out_dim, in_dim = rows.shape
    g = rows.reshape(out_dim, in_dim // 64, 64)
    mx, mn = g.max(axis=2), g.min(axis=2)
    scale = np.maximum((mx - mn) / np.float32(15.0), np.float32(1e-8)).astype(np.float32)
    sb, bb = bf16_bits(scale), bf16_bits(mn)
    s, b = bf16_to_f32(sb), bf16_to_f32(bb)
    q = np.clip(rust_round((g - b[:, :, None]) / s[:, :, None]), 0, 15).astype(np.uint32)
    q = q.reshape(out_dim, in_dim // 8, 8)
    words = np.zeros((out_dim, in_dim // 8), np.uint32)
    for j in range(8):
        words |= q[:, :, j] << np.uint32(4 * j)
    return words, sb.reshape(out_dim, -1), bb.reshape(out_dim, -1)


def q4_codes(words: np.ndarray) -> np.ndarray:
    """u32 words -> nibble codes, LSB-first (shape [..., 8 * words])."""
    w = np.asarray(words, dtype=np.uint32)
    c = np.stack([(w >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], axis=-1)
    return c.reshape(*w.shape[:-1], w.shape[-1] * 8)


def _slot_position(part: int, byte: int) -> int:
    # the position r (0..15) within a 16-code half-chunk that slot (part,
    # byte) holds, per the kernels' unpacking (lowbit.rs:12-19)
    return {0: 2 * byte, 1: 2 * byte + 8, 2: 2 * byte + 1, 3: 2 * byte + 9}[part]


def unpack_q2(dst: np.ndarray, chunks: int) -> np.ndarray:
    """Codes [chunks][32] as a 2-bit kernel lane reads them: two u32 per
    chunk; word t holds half-chunk t, part p at bits 2p of each byte."""
    w = np.frombuffer(np.ascontiguousarray(dst).tobytes(), dtype="<u4")[: 2 * chunks].reshape(chunks, 2)
    out = np.zeros((chunks, 32), np.uint8)
    for t in range(2):
        for p in range(4):
            cast = (w[:, t] >> np.uint32(2 * p)) & np.uint32(0x03030303)
            for b in range(4):
                out[:, 16 * t + _slot_position(p, b)] = (cast >> np.uint32(8 * b)) & np.uint32(3)
    return out


def unpack_q3(dst: np.ndarray, chunks: int) -> np.ndarray:
    """Codes [chunks][32] as a 3-bit kernel lane reads them: two u32 of
    upper 2 bits (as Q2) plus a third u32 of low bits, bit 4t + j of each
    byte."""
    w = np.frombuffer(np.ascontiguousarray(dst).tobytes(), dtype="<u4")[: 3 * chunks].reshape(chunks, 3)
    out = np.zeros((chunks, 32), np.uint8)
    for t in range(2):
        for j in range(4):
            lo = (w[:, t] >> np.uint32(2 * j)) & np.uint32(0x03030303)
            hi = (w[:, 2] >> np.uint32(4 * t + j)) & np.uint32(0x01010101)
            for b in range(4):
                q = 2 * ((lo >> np.uint32(8 * b)) & np.uint32(3)) + ((hi >> np.uint32(8 * b)) & np.uint32(1))
                out[:, 16 * t + _slot_position(j, b)] = q
    return out
