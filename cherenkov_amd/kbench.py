"""Kernel-level timing drivers for the profiles (run under rocprofv3).

    python3 -m cherenkov_amd.kbench dn_scan --rows 4096
    python3 -m cherenkov_amd.kbench attn --ctx 1024 8192 32768

dn_scan: the prefill's gated delta rule alone through the kernel test
entry chk_dn_scan at the 80B shape (16 key / 32 value heads of 128) on
synthetic inputs (conv rows ~ N(0, 0.05^2), decays U(0.3, 1), betas
U(0, 1), zero state): the chunked form `--reps` times, then the sequential
kernel twice.  Prints one line per pass with its wall time.

attn: the q8 flash-decode core (chk_attn_decode_q8: partials + combine, no
projections) at the 80B shape (16 query / 2 kv heads of 256) over a cache
of each given length: int8 K/V uniform in [-127, 127], fp16 scales
0.01 +- 0.005, q ~ N(0, 1), `--reps` calls per length.
"""

from __future__ import annotations

import argparse
import time

import numpy as np


def dn_scan(rows: int, reps: int) -> None:
    import torch

    from .abi import check, lib

    nk, nv, dk, dv = 16, 32, 128, 128
    rng = np.random.default_rng(0)
    dev = "cuda"
    conv = torch.from_numpy((0.05 * rng.standard_normal((rows, 2 * nk * dk + nv * dv))).astype(np.float32)).to(dev)
    decay = torch.from_numpy(rng.uniform(0.3, 1.0, (rows, nv)).astype(np.float32)).to(dev)
    beta = torch.from_numpy(rng.uniform(0.0, 1.0, (rows, nv)).astype(np.float32)).to(dev)
    state = torch.zeros((nv, dv, dk), device=dev)
    y = torch.empty((rows, nv * dv), device=dev)
    torch.cuda.synchronize()
    for chunked in [1] * reps + [0, 0]:
        t0 = time.perf_counter()
        check(lib().chk_dn_scan(conv.data_ptr(), decay.data_ptr(), beta.data_ptr(), state.data_ptr(), y.data_ptr(),
                                rows, nk, nv, dk, dv, chunked, None))
        print(f"dn_scan rows={rows} chunked={chunked} wall_ms={1e3 * (time.perf_counter() - t0):.3f}", flush=True)


def attn(ctxs, reps: int) -> None:
    import torch

    from .abi import check, lib

    nh, nkv, hd = 16, 2, 256
    rng = np.random.default_rng(1)
    for T in ctxs:
        q = torch.from_numpy(rng.standard_normal((nh, 2 * hd)).astype(np.float32)).cuda()
        k = torch.from_numpy(rng.integers(-127, 128, (T, nkv * hd), dtype=np.int8)).cuda()
        v = torch.from_numpy(rng.integers(-127, 128, (T, nkv * hd), dtype=np.int8)).cuda()
        ks = torch.from_numpy(rng.uniform(0.005, 0.015, (T, nkv * hd // 32)).astype(np.float16)).cuda()
        vs = torch.from_numpy(rng.uniform(0.005, 0.015, (T, nkv * hd // 32)).astype(np.float16)).cuda()
        out = torch.empty((nh, hd), device="cuda")
        torch.cuda.synchronize()
        for _ in range(reps):
            t0 = time.perf_counter()
            check(lib().chk_attn_decode_q8(q.data_ptr(), k.data_ptr(), v.data_ptr(), ks.data_ptr(), vs.data_ptr(), T, nh,
                                           nkv, hd, out.data_ptr(), None))
            print(f"attn ctx={T} wall_ms={1e3 * (time.perf_counter() - t0):.3f}", flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("case", choices=["dn_scan", "attn"])
    ap.add_argument("--rows", type=int, default=4096)
    ap.add_argument("--ctx", type=int, nargs="+", default=[1024, 8192, 32768])
    ap.add_argument("--reps", type=int, default=4)
    args = ap.parse_args()
    if args.case == "dn_scan":
        dn_scan(args.rows, args.reps)
    else:
        attn(args.ctx, args.reps)


if __name__ == "__main__":
    main()
