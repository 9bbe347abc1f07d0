"""Request sampling options and the host sampler (reference:
src/sampling.rs:8-226).

`Sampling` holds a request's options with the reference's defaults,
validation and JSON-request merge; `Sampler` drives the native sampler
(sampler.cpp) that a non-greedy decode draws its tokens from.  The random
stream is rand 0.9's StdRng (ChaCha12, seeded by seed_from_u64), so a
seeded request draws the same stream as the reference's.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import asdict, dataclass
from typing import Any, Optional, Sequence

import numpy as np

from .abi import ChkSampling, EngineError, check, lib

_FLOAT_FIELDS = ("temperature", "top_p", "presence_penalty", "frequency_penalty")
_KEYS = ("temperature", "top_p", "top_k", "seed", "presence_penalty", "frequency_penalty")


@dataclass(frozen=True)
class Sampling:
    """Sampling (sampling.rs:8-42): temperature 0 keeps greedy decoding."""

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    seed: Optional[int] = None
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    def native(self) -> ChkSampling:
        s = ChkSampling()
        s.temperature = self.temperature
        s.top_p = self.top_p
        if not 0 <= self.top_k < 1 << 32:
            raise EngineError("top_k must be 0..1000000")
        s.top_k = self.top_k
        s.has_seed = int(self.seed is not None)
        s.seed = 0 if self.seed is None else self.seed
        s.presence_penalty = self.presence_penalty
        s.frequency_penalty = self.frequency_penalty
        return s

    def validate(self) -> None:
        """Sampling::validate (sampling.rs:46-68)."""
        check(lib().chk_sampling_validate(C.byref(self.native())))

    def greedy(self) -> bool:
        """Sampling::greedy (sampling.rs:71-73)."""
        return bool(lib().chk_sampling_greedy(C.byref(self.native())))

    @classmethod
    def from_request(cls, value: dict, defaults: "Sampling" = None) -> "Sampling":
        """Sampling::from_request (sampling.rs:75-96): the request's non-null
        fields over `defaults`, typed as serde reads them (floats accept JSON
        integers; top_k and seed are unsigned integers), then validated."""
        fields: dict[str, Any] = asdict(defaults or cls())
        for key in _KEYS:
            v = value.get(key)
            if v is None:
                continue
            if isinstance(v, bool):
                raise EngineError(f"invalid type: boolean for {key}")
            if key in _FLOAT_FIELDS:
                if not isinstance(v, (int, float)):
                    raise EngineError(f"invalid type for {key}, expected f64")
                fields[key] = float(v)
            else:
                if not isinstance(v, int) or not 0 <= v < 1 << 64:
                    raise EngineError(f"invalid value for {key}, expected an unsigned integer")
                fields[key] = v
        out = cls(**fields)
        out.validate()
        return out


class Sampler:
    """Sampler (sampling.rs:98-209): counts of the prompt and emitted
    tokens, penalties, temperature, top-k, nucleus and the seeded draw."""

    def __init__(self, options: Sampling, prompt: Sequence[int], vocab: int):
        self._keep = options.native()
        p = (C.c_uint32 * max(len(prompt), 1))(*prompt)
        self._h = C.c_void_p()
        check(lib().chk_sampler_new(C.byref(self._keep), p, len(prompt), vocab, C.byref(self._h)))

    def accept(self, token: int) -> None:
        check(lib().chk_sampler_accept(self._h, token))

    def sample(self, logits) -> int:
        a = np.ascontiguousarray(logits, dtype=np.float32)
        out = C.c_uint32()
        check(lib().chk_sampler_sample(self._h, a.ctypes.data_as(C.POINTER(C.c_float)), a.size, C.byref(out)))
        return out.value

    def __del__(self):
        try:
            if self._h:
                lib().chk_sampler_free(self._h)
        except Exception:
            pass


def rng_u64(n: int, seed: Optional[int] = None, seed32: Optional[bytes] = None) -> list[int]:
    """n next_u64 draws of StdRng::seed_from_u64(seed), or of
    StdRng::from_seed(seed32) (the sampler's stream alone)."""
    if seed32 is not None and len(seed32) != 32:
        raise ValueError("seed32 must be 32 bytes")
    out = (C.c_uint64 * n)()
    lib().chk_rng_u64(seed32, 0 if seed is None else seed, out, n)
    return list(out)
