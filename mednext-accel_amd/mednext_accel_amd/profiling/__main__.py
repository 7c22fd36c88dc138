"""``python -m mednext_accel_amd.profiling``: regenerate a device policy."""

from __future__ import annotations

import argparse
import sys


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m mednext_accel_amd.profiling", description=__doc__)
    ap.add_argument("--variant", default="base", choices=("small", "base", "medium", "large", "v2-base", "v2-wide"))
    ap.add_argument("--size", type=int, default=128, help="cubic input size the stage shapes derive from")
    ap.add_argument("--kernel-size", type=int, action="append", dest="kernel_sizes",
                    help="depthwise kernel size (repeatable; default 3)")
    ap.add_argument("--family", action="append", dest="families",
                    choices=("depthwise_conv3d", "group_norm3d", "pointwise_conv3d"))
    ap.add_argument("--repetitions", type=int, default=10)
    ap.add_argument("--policy", required=True, help="output policy YAML path")
    ap.add_argument("--evidence", help="output evidence JSON path")
    args = ap.parse_args(argv)
    import torch

    if not torch.cuda.is_available():
        print("profiling needs a GPU", file=sys.stderr)
        return 1
    from .api import profile

    profile(args.variant, size=args.size, kernel_sizes=tuple(args.kernel_sizes or (3,)),
            families=tuple(args.families or ("depthwise_conv3d", "group_norm3d", "pointwise_conv3d")),
            repetitions=args.repetitions, policy_path=args.policy, evidence_path=args.evidence,
            progress=lambda line: print(line, flush=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())
