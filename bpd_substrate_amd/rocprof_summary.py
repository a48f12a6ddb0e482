"""Reduce rocprofv3 CSV output to per-kernel figures.

    python3 -m bpd_substrate_amd.rocprof_summary --trace T_kernel_trace.csv \
        [--fetch F_counter_collection.csv] [--write W_counter_collection.csv] \
        [--counters Q_counter_collection.csv] -o summary.json

Kernels are keyed by (name, grid threads, workgroup threads), so two launch shapes
of one kernel stay apart.  Per key: dispatch count and duration statistics (us) from the
kernel trace, and for every counter in the PMC files the per-dispatch mean and
median.  FETCH_SIZE and WRITE_SIZE are the counters' own figures (KiB per
dispatch); the factor that turns them into bytes is measured separately, on a
streaming kernel of known size, and applied by whoever reads the summary.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import statistics
from typing import Dict, Iterator, List, Optional


def _rows(path: str) -> Iterator[dict]:
    with open(path, newline="") as f:
        yield from csv.DictReader(f)


def _col(r: dict, *names: str) -> Optional[str]:
    for n in names:
        if n in r:
            return r[n]
    return None


def _total(r: dict, stem: str) -> str:
    """Total threads of the grid (or workgroup): the kernel trace gives X, Y, Z,
    the counter collection the product."""
    if _col(r, stem) is not None:
        return _col(r, stem)
    dims = [_col(r, f"{stem}_{a}") for a in "XYZ"]
    if any(v is None for v in dims):
        return "?"
    n = 1
    for v in dims:
        n *= int(v)
    return str(n)


def _key(r: dict) -> str:
    return "|".join((_col(r, "Kernel_Name") or "?", _total(r, "Grid_Size"), _total(r, "Workgroup_Size")))


_META = ("VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "LDS_Block_Size", "Scratch_Size")


def trace_summary(path: str) -> Dict[str, dict]:
    durs: Dict[str, List[float]] = collections.defaultdict(list)
    meta: Dict[str, dict] = {}
    for r in _rows(path):
        k = _key(r)
        durs[k].append((int(_col(r, "End_Timestamp")) - int(_col(r, "Start_Timestamp"))) / 1000.0)
        meta[k] = {m: _col(r, m) for m in _META if _col(r, m) is not None}
    return {k: {"n": len(v), "avg_us": round(statistics.mean(v), 3), "median_us": round(statistics.median(v), 3),
                "min_us": round(min(v), 3), "max_us": round(max(v), 3), **meta[k]} for k, v in durs.items()}


def counter_summary(path: str) -> Dict[str, dict]:
    acc: Dict[str, Dict[str, List[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in _rows(path):
        acc[_key(r)][_col(r, "Counter_Name")].append(float(_col(r, "Counter_Value")))
    return {k: {c: {"n": len(v), "mean": statistics.mean(v), "median": statistics.median(v)} for c, v in cs.items()}
            for k, cs in acc.items()}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--counters", action="append", default=[])
    ap.add_argument("-o", "--out", required=True)
    a = ap.parse_args(argv)
    out: Dict[str, dict] = {}
    if a.trace:
        out["trace"] = trace_summary(a.trace)
    if a.fetch:
        out["fetch"] = counter_summary(a.fetch)
    if a.write:
        out["write"] = counter_summary(a.write)
    for i, p in enumerate(a.counters):
        out["sq" if i == 0 else f"counters{i}"] = counter_summary(p)
    with open(a.out, "w") as f:
        json.dump(out, f, indent=0)
    print("rocprof_summary:", {k: len(v) for k, v in out.items()})
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
