"""Builds the in-tree gfx950 engine library and the CPU oracle.

`python -m cherenkov_amd.build` (or __graft_entry__.build()) compiles every
HIP translation unit under cherenkov_amd/csrc with hipcc for gfx950 and
links cherenkov_amd/libcherenkov.so; it also builds oracle/liboracle.so
(test infrastructure) with g++.  Objects go to cherenkov_amd/_build/.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "cherenkov_amd"
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcherenkov.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
SOURCES = ["gen.hip", "decode.hip", "attn.hip", "misc.hip", "prefill.hip", "dnscan.hip", "engine.cpp", "runner.cpp", "sampler.cpp", "prefix_cache.cpp", "store.cpp",
           "noalloc.hip", "phasebench.hip", "ple.hip"]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-8000:]}")
    return obj


def build_engine(jobs: int = 5) -> Path:
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, [CSRC / s for s in SOURCES]))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-8000:]}")
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr[-8000:]}")
    return ROOT / "oracle" / "liboracle.so"


def main() -> None:
    print(build_engine(), flush=True)
    print(build_oracle(), flush=True)


if __name__ == "__main__":
    sys.exit(main())
