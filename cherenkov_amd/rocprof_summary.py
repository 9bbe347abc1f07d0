"""Summaries of rocprofv3 traces of bench.py (the tables under profiles/).

    python3 -m cherenkov_amd.rocprof_summary steps <kernel_trace.csv> [first last]
    python3 -m cherenkov_amd.rocprof_summary pmc <counter_collection.csv> <kernel-name-prefix>
    python3 -m cherenkov_amd.rocprof_summary mfma <counter_collection.csv> [rows] [name-prefixes]
    python3 -m cherenkov_amd.rocprof_summary traffic <fetch.csv> <write.csv> <fetch-scale> <write-scale> <name-prefixes>

steps: splits the trace into decode steps (each from a `k_embed` to the
following `k_argmax_final`) and prints kernels per step, kernel busy time
per step and a per-kernel table (launches per step, average / minimum
duration, time per step, share); `first last` restricts it to decode steps
first..last (1-based, inclusive; negative counts from the end).

pmc: the average of each counter over the dispatches of one kernel (e.g.
FETCH_SIZE and WRITE_SIZE in KiB per dispatch).

traffic: from a FETCH_SIZE pass and a WRITE_SIZE pass (KiB per dispatch)
and the copy-calibration factors that turn each into bytes, per kernel
and launch grid (kernels whose names start with one of the comma-separated
prefixes): launches, average KiB of each counter, HBM bytes per launch.

mfma: from a pass of SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE,
SQ_INSTS_VALU_MFMA_MOPS_F16 and SQ_INSTS_VALU_MFMA_MOPS_BF16, per kernel
and launch grid (the `rows` largest by total time, default 12, of the
kernels whose names start with one of the comma-separated prefixes, if
given): launches,
average dispatch duration, MFMA busy = busy cycles / (GRBM_GUI_ACTIVE / 8
XCDs x 1024 SIMDs) and MFMA TFLOP/s = (MOPS_F16 + MOPS_BF16) x 512 /
duration.
"""

from __future__ import annotations

import collections
import csv
import statistics
import sys


def _name(r: dict) -> str:
    return r["Kernel_Name"].split("(")[0].replace("void ", "").replace("chk::", "")


def steps(path: str, first: int | None = None, last: int | None = None) -> None:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    found, cur = [], None
    for r in rows:
        n = _name(r)
        if n == "k_embed":
            cur = [r]
        elif cur is not None:
            cur.append(r)
            if n == "k_argmax_final":
                found.append(cur)
                cur = None
    if not found:
        print("no decode steps in the trace")
        return
    total = len(found)
    if first is not None:
        if first == 0 or last == 0:
            raise SystemExit("steps are numbered from 1 (negative: from the end)")
        lo = first - 1 if first > 0 else total + first
        hi = last if last > 0 else total + last + 1
        found = found[lo:hi]
        print(f"decode steps {lo + 1}..{lo + len(found)} of {total}")
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    per = collections.defaultdict(list)
    busy, wall = [], []
    for s in found:
        b = 0.0
        for r in s:
            per[_name(r)].append(dur(r))
            b += dur(r)
        busy.append(b)
        wall.append((int(s[-1]["End_Timestamp"]) - int(s[0]["Start_Timestamp"])) / 1e3)
    ns = len(found)
    tot = statistics.mean(busy)
    print(f"decode steps: {ns}; kernels per step: {statistics.median(len(s) for s in found):.0f}; "
          f"kernel busy per step {tot:.1f} us; median step wall {statistics.median(wall):.1f} us")
    print()
    print("| kernel | launches/step | avg us | min us | us/step | share |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{k}` | {len(v) / ns:.0f} | {statistics.mean(v):.2f} | {min(v):.2f} | {sum(v) / ns:.1f} | "
              f"{100 * sum(v) / ns / tot:.1f}% |")


def pmc(path: str, prefix: str) -> None:
    vals = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if _name(r).startswith(prefix):
            vals[r["Counter_Name"]].append(float(r["Counter_Value"]))
    for k, v in sorted(vals.items()):
        print(f"{prefix} {k}: dispatches {len(v)}, mean {statistics.mean(v):.1f}")


def traffic(fetch: str, write: str, fscale: float, wscale: float, prefixes: str) -> None:
    keep = tuple(x for x in prefixes.split(",") if x)
    per: dict[tuple, dict[str, list]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for path, counter in ((fetch, "FETCH_SIZE"), (write, "WRITE_SIZE")):
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter and _name(r).startswith(keep):
                per[(_name(r), r["Grid_Size"])][counter].append(float(r["Counter_Value"]))
    print("| kernel | grid (threads) | launches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes per launch |")
    print("|---|---:|---:|---:|---:|---:|")
    for (name, grid), c in sorted(per.items()):
        f = statistics.mean(c["FETCH_SIZE"]) if c["FETCH_SIZE"] else 0.0
        w = statistics.mean(c["WRITE_SIZE"]) if c["WRITE_SIZE"] else 0.0
        n = max(len(c["FETCH_SIZE"]), len(c["WRITE_SIZE"]))
        print(f"| `{name}` | {grid} | {n} | {f:,.1f} | {w:,.1f} | {1024 * (f * fscale + w * wscale):,.0f} |")


def mfma(path: str, rows: int = 12, prefixes: str = "") -> None:
    keep = tuple(x for x in prefixes.split(",") if x)
    disp: dict[str, dict] = {}
    for r in csv.DictReader(open(path)):
        if keep and not _name(r).startswith(keep):
            continue
        d = disp.setdefault(r["Dispatch_Id"], {"name": _name(r), "grid": r["Grid_Size"], "c": {},
                                               "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
        d["c"][r["Counter_Name"]] = float(r["Counter_Value"])
    agg = collections.defaultdict(list)
    for d in disp.values():
        agg[(d["name"], d["grid"])].append(d)
    print("| kernel | grid (threads) | launches | avg us | MFMA busy | MFMA TFLOP/s |")
    print("|---|---:|---:|---:|---:|---:|")
    for (name, grid), ds in sorted(agg.items(), key=lambda kv: -sum(d["us"] for d in kv[1]))[:rows]:
        us = statistics.mean(d["us"] for d in ds)
        busy = statistics.mean(d["c"].get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) /
                               max(d["c"].get("GRBM_GUI_ACTIVE", 0.0) / 8 * 1024, 1.0) for d in ds)
        ops = statistics.mean(d["c"].get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) +
                              d["c"].get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) for d in ds)
        tf = ops * 512 / (us * 1e-6) / 1e12 if us > 0 else 0.0
        print(f"| `{name}` | {grid} | {len(ds)} | {us:.1f} | {100 * busy:.0f}% | {tf:.0f} |")


def main() -> None:
    if len(sys.argv) >= 5 and sys.argv[1] == "steps":
        steps(sys.argv[2], int(sys.argv[3]), int(sys.argv[4]))
    elif len(sys.argv) >= 3 and sys.argv[1] == "steps":
        steps(sys.argv[2])
    elif len(sys.argv) >= 4 and sys.argv[1] == "pmc":
        pmc(sys.argv[2], sys.argv[3])
    elif len(sys.argv) >= 7 and sys.argv[1] == "traffic":
        traffic(sys.argv[2], sys.argv[3], float(sys.argv[4]), float(sys.argv[5]), sys.argv[6])
    elif len(sys.argv) >= 3 and sys.argv[1] == "mfma":
        mfma(sys.argv[2], int(sys.argv[3]) if len(sys.argv) >= 4 else 12, sys.argv[4] if len(sys.argv) >= 5 else "")
    else:
        print(__doc__)
        sys.exit(2)


if __name__ == "__main__":
    main()
