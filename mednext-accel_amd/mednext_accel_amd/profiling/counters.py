"""Attribute rocprofv3 ``--pmc`` passes over ``bench.py --sweep`` to the sweep's
kernel phases and print one markdown table.

``bench.py --sweep`` issues two GPU spin kernels at start-up and then, per
phase, a spin before the warm-up launches and a spin before the timed
launches. Split at the spin kernels, the dispatch stream's segment 4 + 2i is
therefore phase i's timed launches. Per phase and counter: the median over
those dispatches of each kernel of this package (plus the calibration copy),
summed over the kernels one launch runs.

HBM traffic: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what
they read for the sweep's first phase, a ``torch.neg`` copy that moves a known
number of bytes (half of them read, half written). MFMA FLOPs are
512 x SQ_INSTS_VALU_MFMA_MOPS_BF16. MfmaUtil and MeanOccupancyPerActiveCU are
reported for the phase's main kernel (the one with the most wave cycles, or
MFMA operations where it has any).

    python -m mednext_accel_amd.profiling.counters --sweep sweep.jsonl \\
        --pass p1/run_counter_collection.csv --pass p2/... > counters.md
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
import sys
from collections import defaultdict
from collections.abc import Sequence

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
FLOPS_PER_MOP = 512
_OURS = ("dw_", "pw_", "gn_", "s2_", "up_", "grn_", "neg_kernel")


def kernel_name(raw: str) -> str:
    if "neg_kernel_cuda" in raw:
        return "neg_kernel"
    name = raw.replace("(anonymous namespace)::", "").replace("void ", "").replace("mednext::", "")
    return re.sub(r"\(.*", "", name)


def _segments(path: str):
    names: dict[int, str] = {}
    values: dict[int, dict[str, float]] = defaultdict(dict)
    with open(path, newline="") as fh:
        for row in csv.DictReader(fh):
            dispatch = int(row["Dispatch_Id"])
            names[dispatch] = kernel_name(row["Kernel_Name"])
            values[dispatch][row["Counter_Name"]] = float(row["Counter_Value"])
    segments, current = [], []
    for dispatch in sorted(names):
        if "spin_kernel" in names[dispatch]:
            segments.append(current)
            current = []
        else:
            current.append(dispatch)
    segments.append(current)
    return names, values, segments


def attribute(path: str, n_phases: int) -> list[dict[str, dict[str, float]]]:
    """Per phase: {kernel: {counter: median per dispatch}}."""
    names, values, segments = _segments(path)
    spins = len(segments) - 1
    if spins != 2 + 2 * n_phases:
        raise ValueError(f"{path}: {spins} spin kernels, expected {2 + 2 * n_phases} for {n_phases} phases")
    out = []
    for i in range(n_phases):
        samples: dict[str, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
        for dispatch in segments[4 + 2 * i]:
            if names[dispatch].startswith(_OURS):
                for counter, value in values[dispatch].items():
                    samples[names[dispatch]][counter].append(value)
        out.append({k: {c: statistics.median(v) for c, v in cs.items()} for k, cs in samples.items()})
    return out


def merge(passes: Sequence[list[dict[str, dict[str, float]]]]) -> list[dict[str, dict[str, float]]]:
    merged = [defaultdict(dict) for _ in passes[0]]
    for phases in passes:
        for i, kernels in enumerate(phases):
            for kernel, counters in kernels.items():
                merged[i][kernel].update(counters)
    return [dict(m) for m in merged]


def _total(kernels: dict[str, dict[str, float]], counter: str) -> float | None:
    vals = [c[counter] for c in kernels.values() if counter in c]
    return sum(vals) if vals else None


def _main_kernel(kernels: dict[str, dict[str, float]]) -> str | None:
    if not kernels:
        return None
    mfma = {k: c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) for k, c in kernels.items()}
    if any(v > 0 for v in mfma.values()):
        return max(mfma, key=mfma.get)
    return max(kernels, key=lambda k: kernels[k].get("SQ_WAVE_CYCLES", 0.0))


def table(sweep: list[dict], phases: list[dict[str, dict[str, float]]]) -> str:
    calib = phases[0] if sweep[0]["op"] == "copy_calibration" else None
    fetch_scale = write_scale = None
    if calib:
        moved = sweep[0]["bytes"] / 2 / 1024  # KiB read (= KiB written)
        fetch, write = _total(calib, "FETCH_SIZE"), _total(calib, "WRITE_SIZE")
        fetch_scale = moved / fetch if fetch else None
        write_scale = moved / write if write else None
    lines = [
        f"FETCH_SIZE scale {fetch_scale:.3f}, WRITE_SIZE scale {write_scale:.3f} (from the calibration copy)."
        if fetch_scale and write_scale else "No calibration phase: traffic columns unscaled.",
        "",
        "| op | shape | us | alg. GB/s | % of 8 TB/s | HBM traffic MiB | traffic / alg. | HBM GB/s (counted) "
        "| MFMA TFLOP/s (counted) | % of 2.5 PF | MfmaUtil % | wait % | LDS conflict % | occupancy (waves/CU) "
        "| main kernel |",
        "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|",
    ]

    def fmt(v, spec):
        return "-" if v is None else format(v, spec)

    for rec, kernels in zip(sweep, phases):
        us = rec["us"]
        fetch, write = _total(kernels, "FETCH_SIZE"), _total(kernels, "WRITE_SIZE")
        traffic = None
        if fetch is not None and write is not None:
            traffic = (fetch * (fetch_scale or 1.0) + write * (write_scale or 1.0)) * 1024
        mops = _total(kernels, "SQ_INSTS_VALU_MFMA_MOPS_BF16")
        tflops = mops * FLOPS_PER_MOP / (us * 1e-6) / 1e12 if mops else None
        wait, cycles = _total(kernels, "SQ_WAIT_INST_ANY"), _total(kernels, "SQ_WAVE_CYCLES")
        conflict, lds = _total(kernels, "SQ_LDS_BANK_CONFLICT"), _total(kernels, "SQ_LDS_IDX_ACTIVE")
        main = _main_kernel(kernels)
        mc = kernels.get(main, {}) if main else {}
        lines.append(
            "| {op} | {shape} | {us:.2f} | {gbs:.0f} | {frac:.1f} | {traffic} | {ratio} | {hbm} | {tf} | {tff} | {mu} "
            "| {wait} | {conf} | {occ} | `{main}` |".format(
                op=rec["op"], shape=rec["shape"], us=us, gbs=rec["gbs"], frac=100 * rec["hbm_frac"],
                traffic=fmt(traffic / 2**20 if traffic else None, ".1f"),
                ratio=fmt(traffic / rec["bytes"] if traffic else None, ".2f"),
                hbm=fmt(traffic / (us * 1e-6) / 1e9 if traffic else None, ".0f"),
                tf=fmt(tflops, ".1f"), tff=fmt(100 * tflops / MFMA_BF16_PEAK_TFLOPS if tflops else None, ".2f"),
                mu=fmt(mc.get("MfmaUtil"), ".1f"),
                wait=fmt(100 * wait / cycles if wait is not None and cycles else None, ".0f"),
                conf=fmt(100 * conflict / lds if conflict is not None and lds else None, ".1f"),
                occ=fmt(mc.get("MeanOccupancyPerActiveCU"), ".1f"), main=main or "-"))
    return "\n".join(lines)


def main(argv: Sequence[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m mednext_accel_amd.profiling.counters", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--sweep", required=True, help="bench.py --sweep output (one JSON line per phase)")
    ap.add_argument("--pass", dest="passes", action="append", required=True,
                    help="run_counter_collection.csv of one rocprofv3 --pmc pass (repeatable)")
    args = ap.parse_args(argv)
    with open(args.sweep) as fh:
        sweep = [json.loads(line) for line in fh if line.startswith("{")]
    phases = merge([attribute(p, len(sweep)) for p in args.passes])
    print(table(sweep, phases))
    return 0


if __name__ == "__main__":
    sys.exit(main())
