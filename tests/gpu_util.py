"""Shared helpers of the GPU parity tests (device buffers via torch, the
parity tolerances of the north star)."""

from __future__ import annotations

import collections

import numpy as np


def torch_dev():
    import torch

    return torch


# Device tensors handed to the engine as raw pointers must outlive the
# call: `to_dev(x).data_ptr()` would otherwise drop the tensor before the
# call and let torch's caching allocator hand its block to the next tensor.
_KEEP: collections.deque = collections.deque(maxlen=64)


def to_dev(a: np.ndarray):
    torch = torch_dev()
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    torch.cuda.synchronize()
    _KEEP.append(t)
    return t


def empty_dev(shape, dtype=np.float32):
    torch = torch_dev()
    tdt = {np.float32: torch.float32, np.uint32: torch.int32, np.int32: torch.int32}[dtype]
    t = torch.empty(shape, dtype=tdt, device="cuda")
    torch.cuda.synchronize()
    _KEEP.append(t)
    return t


def to_host(t, dtype=None) -> np.ndarray:
    torch = torch_dev()
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


# Relative band around a layer's k-th router probability inside which the
# engine and the oracle may pick different experts from f32 rounding alone
# (the oracle then follows the engine's pick: OracleState.route_hints).
ROUTE_TIE_TOL = 2e-3


def engine_routes(eng, layers: int, row: int = 0) -> np.ndarray:
    """The engine's expert ids of layers 0..layers-1 in its latest step."""
    return np.array([eng.last_routes(layer, row)[0] for layer in range(layers)], np.uint32)


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 or nb == 0:
        return 1.0 if na == nb else 0.0
    return float(a @ b / (na * nb))


def assert_close(got: np.ndarray, ref: np.ndarray, label: str, abs_frac: float = 2e-2, min_cos: float = 0.999):
    """North-star float bar: cosine >= 0.999 and max-abs within
    2e-2 * max(1, max|ref|) (the reference's logits convention,
    tests/import.rs:20-39), with fp32 accumulation."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, (label, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{label}: non-finite output"
    err = float(np.max(np.abs(got - ref))) if got.size else 0.0
    scale = max(1.0, float(np.max(np.abs(ref)))) if ref.size else 1.0
    cos = cosine(got, ref)
    assert err <= abs_frac * scale and cos >= min_cos, f"{label}: max-abs {err:.3e} (scale {scale:.3f}), cos {cos:.6f}"
    return err, cos


def topk_margin(probs: np.ndarray, k: int) -> float:
    """Logit gap between the k-th and (k+1)-th expert (softmax keeps logit
    differences: l_i - l_j = ln p_i - ln p_j)."""
    p = np.sort(probs.astype(np.float64))[::-1]
    if k >= p.size:
        return np.inf
    return float(np.log(max(p[k - 1], 1e-300)) - np.log(max(p[k], 1e-300)))


def argmax_margin(logits: np.ndarray) -> float:
    s = np.sort(logits.astype(np.float64))[::-1]
    return float(s[0] - s[1])


def lowest_argmax(x: np.ndarray) -> int:
    """Greedy rule of the engine: the lowest index wins exact ties."""
    return int(np.argmax(x))
