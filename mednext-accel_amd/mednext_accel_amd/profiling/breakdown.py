"""Per-step kernel time of a training step from a ``rocprofv3 --kernel-trace``
CSV: kernel time by category and the top kernels, as one markdown report.

Steps are delimited by the optimizer: every run of AdamW multi-tensor kernels
(launches no more than ``gap`` dispatches apart) closes one step. The report
covers the last ``steps`` complete steps (those after the first delimiter, so
the first partial step is never counted) and divides each kernel's summed
duration by the step count.

    rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o run -- \\
        python3 bench.py --train-only --train-variants base --train-steps 10 --train-warmup 3
    python -m mednext_accel_amd.profiling.breakdown OUT/run_kernel_trace.csv \\
        --title "..." --command "..." > report.md
"""

from __future__ import annotations

import argparse
import csv
import re
import sys
from collections import defaultdict
from collections.abc import Sequence

_OPTIMIZER = re.compile(r"multi_tensor|[Aa]dam|_foreach")

# (category, predicate on the short kernel name), first match wins.
CATEGORIES: tuple[tuple[str, object], ...] = (
    ("depthwise (HIP)", lambda n: n.startswith(("dw_", "s2_"))),
    ("GroupNorm (HIP)", lambda n: n.startswith("gn_")),
    ("GRN (HIP)", lambda n: n.startswith("grn_")),
    ("pointwise GEMMs (HIP)", lambda n: n.startswith("pw_")),
    ("upsample / join (HIP)", lambda n: n.startswith("up_")),
    ("native conv / GEMM", lambda n: n.startswith(("Cijk", "ck::", "Im3d2Col", "Col2Im", "batched_transpose",
                                                   "naive_conv"))),
    ("AdamW (native)", lambda n: "multi_tensor" in n),
    ("loss (native)", lambda n: "nll_loss" in n or "SoftMax" in n),
    ("autocast casts (native)", lambda n: "copy" in n),
    ("GELU (native)", lambda n: "gelu" in n.lower()),
)


def short_name(raw: str) -> str:
    name = raw
    for noise in ("(anonymous namespace)::", "void ", "mednext::", "at::native::"):
        name = name.replace(noise, "")
    return re.sub(r"\(.*", "", name)


def category(name: str) -> str:
    for label, pred in CATEGORIES:
        if pred(name):
            return label
    return "other native elementwise / reductions"


def step_bounds(names: Sequence[str], gap: int = 60) -> list[int]:
    """Index of the last optimizer kernel of each step, in dispatch order."""
    ends: list[int] = []
    for i, name in enumerate(names):
        if _OPTIMIZER.search(name):
            if ends and i - ends[-1] <= gap:
                ends[-1] = i
            else:
                ends.append(i)
    return ends


def per_step(rows: Sequence[dict], steps: int = 5, gap: int = 60) -> tuple[dict[str, list[float]], int]:
    """{kernel: [ms per step, launches per step]} over the last ``steps``
    complete steps, and the number of steps used."""
    rows = sorted(rows, key=lambda r: int(r["Start_Timestamp"]))
    ends = step_bounds([r["Kernel_Name"] for r in rows], gap)
    used = min(steps, len(ends) - 1)
    if used < 1:
        raise ValueError("the trace holds fewer than two optimizer steps")
    agg: dict[str, list[float]] = defaultdict(lambda: [0.0, 0.0])
    for r in rows[ends[-used - 1] + 1: ends[-1] + 1]:
        name = short_name(r["Kernel_Name"])
        agg[name][0] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6
        agg[name][1] += 1
    return {k: [ms / used, n / used] for k, (ms, n) in agg.items()}, used


def report(rows: Sequence[dict], title: str, command: str, steps: int = 5, top: int = 30, gap: int = 60) -> str:
    kernels, used = per_step(rows, steps, gap)
    busy = sum(ms for ms, _ in kernels.values())
    cats: dict[str, float] = defaultdict(float)
    for name, (ms, _) in kernels.items():
        cats[category(name)] += ms
    out = [f"# {title}", "", "Command (from the repository root, on one MI355X):", "", f"    {command}", "",
           f"Source: `run_kernel_trace.csv`, the last {used} steps (delimited by the AdamW multi-tensor kernels), "
           f"summed per kernel and divided by {used}. GPU busy time {busy:.2f} ms per step.", "",
           "| category | ms per step | share |", "|---|---|---|"]
    for label, ms in sorted(cats.items(), key=lambda kv: -kv[1]):
        out.append(f"| {label} | {ms:.3f} | {100 * ms / busy:.1f}% |")
    out += ["", "Top kernels:", "", "| kernel | ms per step | launches per step | avg us |", "|---|---|---|---|"]
    for name, (ms, n) in sorted(kernels.items(), key=lambda kv: -kv[1][0])[:top]:
        out.append(f"| `{name[:80]}` | {ms:.3f} | {n:.0f} | {1000 * ms / n:.1f} |")
    return "\n".join(out) + "\n"


def main(argv: Sequence[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m mednext_accel_amd.profiling.breakdown", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("trace", help="run_kernel_trace.csv of rocprofv3 --kernel-trace --output-format csv")
    ap.add_argument("--title", default="Training step: per-step kernel time by category (MI355X)")
    ap.add_argument("--command", default="(not given)", help="the rocprofv3 command that wrote the trace")
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--top", type=int, default=30)
    args = ap.parse_args(argv)
    with open(args.trace, newline="") as fh:
        rows = list(csv.DictReader(fh))
    sys.stdout.write(report(rows, args.title, args.command, args.steps, args.top))
    return 0


if __name__ == "__main__":
    sys.exit(main())
