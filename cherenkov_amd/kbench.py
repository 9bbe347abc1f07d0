"""Kernel-level timing drivers for the profiles (run under rocprofv3).

    python3 -m cherenkov_amd.kbench dn_scan --rows 4096
    python3 -m cherenkov_amd.kbench attn --ctx 1024 8192 32768

dn_scan: the prefill's gated delta rule alone through the kernel test
entry chk_dn_scan at the 80B shape (16 key / 32 value heads of 128) on
synthetic inputs (conv rows ~ N(0, 0.05^2), decays U(0.3, 1), betas
U(0, 1), zero state): the chunked form `--reps` times, then the sequential
kernel twice.  Prints one line per pass with its wall time.

phases: the cost of one dependent phase (chk_phase_bench): graph launch
cadence, streaming launches, a persistent kernel's grid barrier with its
weights streamed after or issued before it, and float-atomic throughput.

    python3 -m cherenkov_amd.kbench phases --wgs 128 256 512 --mbytes 1.5 14

attn: the q8 flash-decode core (chk_attn_decode_q8: partials + combine, no
projections) at the 80B shape (16 query / 2 kv heads of 256) over a cache
of each given length: int8 K/V uniform in [-127, 127], fp16 scales
0.01 +- 0.005, q ~ N(0, 1), `--reps` calls per length.

blocks: configs 2-4 as the decode step runs them (chk_time_blocks: one
captured graph of blocks over a rotation of layers, each with its own
weights, replayed between HIP events), on working sets past the 256 MB
last-level cache:

    python3 -m cherenkov_amd.kbench blocks --config 2 --bits 4 3 2
    python3 -m cherenkov_amd.kbench blocks --config 3
    python3 -m cherenkov_amd.kbench blocks --config 4 --ctx 1024 8192 32768

config 2: the MoE block (router, routed top-10 + shared expert, combine)
of all 48 layers of the 80B shape, 16 inputs rms_norm(N(0, 1)) in
rotation, >= 1000 blocks; config 3: the DeltaNet layer of all 36 DeltaNet
layers, the decode step (1 row) and the 3-row verify (snapshots); config
4: the attention layer (projections, q8 cache, combine, o-projection) of
the 16 attention layers of a 64-layer model of the same shape, at batch 1
and 2 (two sequence slots), K/V ~ N(0, 1) through the q8 rule.  Prints a
JSON line per case with the algorithmic bytes per block (the blueprint's
per-config accounting) and the achieved rate.
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


def _time_blocks(eng, kind, nb, layers, x, nx, pos, reps):
    import ctypes as C

    from .abi import check

    us = C.c_float()
    la = (C.c_uint32 * len(layers))(*layers)
    pa = (C.c_uint32 * max(1, len(pos)))(*(pos or [0]))
    check(eng.L.chk_time_blocks(eng.handle, kind, nb, la, len(layers), x.data_ptr(), nx, pa, reps, C.byref(us)))
    return us.value


def _report(case: dict, us: float, nbytes: int, working_set: int) -> None:
    import json

    gbs = nbytes / (us * 1e-6) / 1e9
    case.update(us_per_block=round(us, 3), bytes_per_block=nbytes, gb_s=round(gbs, 1),
                frac_of_8tbs=round(gbs / 8000, 4), rotated_working_set_mb=round(working_set / 1e6, 1))
    print(json.dumps(case), flush=True)


def blocks(config: int, bits_list, ctxs, min_blocks: int) -> None:
    import torch

    from . import presets
    from .abi import check
    from .engine import Engine

    H = 2048
    g = torch.Generator(device="cuda").manual_seed(7)

    def inputs(nx, nb):
        x = torch.randn((nx, nb, H), generator=g, device="cuda")
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    if config == 2:
        # router 2,097,152 + 10 records + shared expert 1,769,472 + gate
        # vector + x / out (the shared expert stays Q4)
        per = {4: 21565440, 3: 17633280, 2: 13701120}
        for bits in bits_list:
            eng = Engine(presets.qwen3next_80b_shape(mtp=0), experts=bits, drafts=0, max_t=64)
            try:
                layers = list(range(48))
                x = inputs(16, 1)
                reps = -(-min_blocks // len(layers))
                us = _time_blocks(eng, 2, 1, layers, x, 16, [], reps)
                _report({"config": 2, "block": "moe", "experts_bits": bits, "rows": 1, "blocks_timed": reps * 48}, us,
                        per[bits], 48 * per[bits])
            finally:
                eng.close()
    elif config == 3:
        # Q4 projections 18,948,096 + state read + write 4,194,304 + conv
        # history read + write 196,608 + conv weights 65,536; the 3-row
        # verify adds two snapshot planes of state and history
        step = 18948096 + 4194304 + 196608 + 65536
        eng = Engine(presets.qwen3next_80b_shape(mtp=1), experts=4, drafts=2, max_t=64)
        try:
            layers = [l for l in range(48) if (l + 1) % 4]
            for nb in (1, 3):
                x = inputs(16, nb)
                reps = -(-min_blocks // len(layers))
                us = _time_blocks(eng, 3, nb, layers, x, 16, [], reps)
                nbytes = step + (nb - 1) * (4194304 // 2 + 196608 // 2)
                _report({"config": 3, "block": "deltanet", "rows": nb, "form": "decode" if nb == 1 else "verify",
                         "blocks_timed": reps * len(layers)}, us, nbytes, len(layers) * nbytes)
        finally:
            eng.close()
    else:
        # q, k, v, o projections 15,335,424 + index projection 737,280 +
        # (T + 1) x 1,088 q8 K/V bytes per request (the new row appended)
        cfg = presets.qwen3next_80b_shape(layers=64, mtp=1)
        eng = Engine(cfg, experts=4, drafts=1, max_t=max(ctxs) + 8)
        try:
            layers = [l for l in range(64) if (l + 1) % 4 == 0]
            kv_row = cfg.num_key_value_heads * cfg.head_dim
            for T in ctxs:
                for seq in (0, 1):
                    for l in layers:
                        k = torch.randn((T, kv_row), generator=g, device="cuda")
                        v = torch.randn((T, kv_row), generator=g, device="cuda")
                        torch.cuda.synchronize()
                        check(eng.L.chk_kv_fill(eng.handle, l, seq, k.data_ptr(), v.data_ptr(), T))
                for nb in (1, 2):
                    x = inputs(16, nb)
                    reps = -(-min_blocks // len(layers))
                    us = _time_blocks(eng, 4, nb, layers, x, 16, [T] * nb, reps)
                    nbytes = 15335424 + 737280 + nb * (T + 1) * 1088
                    _report({"config": 4, "block": "attention", "ctx": T, "batch": nb,
                             "blocks_timed": reps * len(layers)}, us, nbytes, len(layers) * nbytes)
        finally:
            eng.close()


PHASE_MODES = {
    0: "graph of empty dependent launches",
    1: "graph of dependent launches streaming weights",
    2: "persistent kernel, grid barrier only",
    3: "persistent kernel, barrier then weights",
    4: "persistent kernel, next weights issued before the barrier",
    6: "persistent kernel, XCD-local barrier in L2",
}


def phases(wgs_list, mbytes_list, n: int) -> None:
    """What one dependent phase costs (chk_phase_bench): launch cadence in a
    graph, streaming launches, and a persistent kernel's grid barrier with
    its weights streamed after it or issued before it; then float-atomic
    throughput with and without contention."""
    import ctypes as C

    from .abi import check, lib

    us, err = C.c_double(), C.c_uint32()

    def bench(mode, wgs, n_ph, nbytes):
        check(lib().chk_phase_bench(mode, wgs, n_ph, nbytes, C.byref(us), C.byref(err)))
        if err.value:  # a barrier that saw wrong data or hit its spin limit measures nothing
            raise RuntimeError(f"phase mode={mode} wgs={wgs} bytes={nbytes}: {err.value} errors, not reported")

    for wgs in wgs_list:
        for mode in (0, 2, 6):
            if mode == 6 and wgs % 8:
                continue
            bench(mode, wgs, n, 0)
            print(f"phase mode={mode} wgs={wgs} mbytes=0 us_per_phase={us.value:.3f} errors={err.value}  # {PHASE_MODES[mode]}",
                  flush=True)
        for mb in mbytes_list:
            for mode in (1, 3, 4):
                bench(mode, wgs, min(n, 400), int(mb * 1e6))
                print(f"phase mode={mode} wgs={wgs} mbytes={mb} us_per_phase={us.value:.3f} errors={err.value}  "
                      f"# {PHASE_MODES[mode]}", flush=True)
    for wgs, window, per_wg in ((256, 1 << 22, 1300), (256, 1300, 1300), (64, 1300, 1300), (256, 2048, 2048)):
        check(lib().chk_phase_bench(5, wgs, window, per_wg * 4, C.byref(us), C.byref(err)))
        n_at = wgs * per_wg
        print(f"atomics wgs={wgs} adds_per_wg={per_wg} window={window} us={us.value:.3f} "
              f"adds_per_us={n_at / us.value:.0f}", flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("case", choices=["dn_scan", "attn", "phases", "blocks"])
    ap.add_argument("--config", type=int, choices=[2, 3, 4], default=2)
    ap.add_argument("--bits", type=int, nargs="+", default=[4, 3, 2])
    ap.add_argument("--min-blocks", type=int, default=1000)
    ap.add_argument("--wgs", type=int, nargs="+", default=[256])
    ap.add_argument("--mbytes", type=float, nargs="+", default=[1.5, 14.0])
    ap.add_argument("--phases", type=int, default=2000)
    ap.add_argument("--rows", type=int, default=4096)
    ap.add_argument("--ctx", type=int, nargs="+", default=[1024, 8192, 32768])
    ap.add_argument("--reps", type=int, default=4)
    args = ap.parse_args()
    if args.case == "dn_scan":
        dn_scan(args.rows, args.reps)
    elif args.case == "attn":
        attn(args.ctx, args.reps)
    elif args.case == "blocks":
        blocks(args.config, args.bits, args.ctx, args.min_blocks)
    else:
        phases(args.wgs, args.mbytes, args.phases)


if __name__ == "__main__":
    main()
