"""Builds the in-tree gfx950 engine library and the CPU oracle.

`python -m cherenkov_amd.build` (or __graft_entry__.build()) compiles every
HIP translation unit under cherenkov_amd/csrc with hipcc for gfx950 and
links cherenkov_amd/libcherenkov.so; it also builds oracle/liboracle.so
(test infrastructure) with g++.  Objects go to cherenkov_amd/_build/.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import re
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


# Kernels allowed to use scratch memory: the generic-width conv fallback
# (taps indexed at run time; conv widths other than 4 only).
SCRATCH_OK = ("_ZN3chk12k_pf_dn_convILi0EEEvNS_8PfDnArgsE",)


def _resources(stderr: str) -> dict[str, dict[str, int]]:
    """Per-kernel resource usage from the compiler's kernel-resource-usage
    remarks (VGPRs, scratch bytes per lane, VGPR spills, occupancy)."""
    res: dict[str, dict[str, int]] = {}
    name = None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            res[name] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs|ScratchSize \[bytes/lane\]|VGPRs Spill|Occupancy \[waves/SIMD\]): (\d+)", line)
        if m and name:
            res[name][m.group(1).split()[0] + (" spill" if "Spill" in m.group(1) else "")] = int(m.group(2))
    return res


def _compile(src: Path) -> tuple[Path, dict[str, dict[str, int]]]:
    obj = BUILD / (src.stem + ".o")
    remarks = ["-Rpass-analysis=kernel-resource-usage"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *FLAGS, *remarks, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-8000:]}")
    return obj, _resources(r.stderr)


def build_engine(jobs: int = 5) -> Path:
    """Compiles and links the library; fails if any kernel spills registers
    or uses scratch memory (a silent slowdown no parity test sees), and
    writes every kernel's resource usage to _build/kernel_resources.txt."""
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        done = list(ex.map(_compile, [CSRC / s for s in SOURCES]))
    objs = [o for o, _ in done]
    res = {k: v for _, r in done for k, v in r.items()}
    with open(BUILD / "kernel_resources.txt", "w") as f:
        for k in sorted(res):
            f.write(f"{k} {res[k]}\n")
    bad = [k for k, v in res.items()
           if (v.get("ScratchSize", 0) or v.get("VGPRs spill", 0)) and k not in SCRATCH_OK]
    if bad:
        raise RuntimeError("kernels using scratch memory or spilling registers:\n" +
                           "\n".join(f"{k} {res[k]}" for k in sorted(bad)))
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
