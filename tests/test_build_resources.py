"""The build's register-budget guard (cherenkov_amd/build.py): the compiler's
kernel-resource-usage remarks are parsed per kernel, and a kernel that
spills or uses scratch memory fails the build.  CPU only."""

from __future__ import annotations

import ast

from cherenkov_amd import build

SAMPLE = """\
x.hip:15:1: remark: Function Name: _ZN3chk4k_okEv [-Rpass-analysis=kernel-resource-usage]
x.hip:15:1: remark:     TotalSGPRs: 32 [-Rpass-analysis=kernel-resource-usage]
x.hip:15:1: remark:     VGPRs: 13 [-Rpass-analysis=kernel-resource-usage]
x.hip:15:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:15:1: remark:     Occupancy [waves/SIMD]: 8 [-Rpass-analysis=kernel-resource-usage]
x.hip:15:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:44:1: remark: Function Name: _ZN3chk5k_badEv [-Rpass-analysis=kernel-resource-usage]
x.hip:44:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:44:1: remark:     ScratchSize [bytes/lane]: 1544 [-Rpass-analysis=kernel-resource-usage]
x.hip:44:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
x.hip:44:1: remark:     VGPRs Spill: 501 [-Rpass-analysis=kernel-resource-usage]
"""


def test_remarks_parse_per_kernel():
    res = build._resources(SAMPLE)
    assert res["_ZN3chk4k_okEv"] == {"VGPRs": 13, "ScratchSize": 0, "Occupancy": 8, "VGPRs spill": 0}
    assert res["_ZN3chk5k_badEv"] == {"VGPRs": 256, "ScratchSize": 1544, "Occupancy": 2, "VGPRs spill": 501}


def test_built_library_has_no_spilling_kernel():
    """If the library was built here, its report lists no spilling kernel
    beyond the allowed one (the build itself refuses otherwise)."""
    path = build.BUILD / "kernel_resources.txt"
    if not path.exists():
        return
    bad = []
    for line in path.read_text().splitlines():
        name, _, rest = line.partition(" ")
        r = ast.literal_eval(rest)
        if (r.get("ScratchSize", 0) or r.get("VGPRs spill", 0)) and name not in build.SCRATCH_OK:
            bad.append(line)
    assert not bad, bad
