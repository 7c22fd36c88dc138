#!/usr/bin/env python
"""Benchmark of the MedNeXt operator path on one MI355X.

Headline (BASELINE.json metric "depthwise Conv3d fwd+bwd GB/s (% of HBM
peak)"): one step = depthwise Conv3d forward + input-grad + weight-grad (with
the fused bias grad) at the configs[1] headline shape, N=1 C=32 D=H=W=128, k=3,
bf16 in / fp32 accumulate. ``value`` = algorithmic bytes of the three phases
(12 * E bytes: two bf16 streams per phase) / the sum of their per-launch
times. Each phase is timed on its own (as configs[1] asks) over K back-to-back
launches between two HIP events, inputs resident in HBM and rotated over three
input sets (>256 MiB Infinity Cache) so repeated timing cannot hit in MALL.

Also reported: per-phase microseconds, the roofline of the dominant kernel
(with HBM traffic from the committed rocprofv3 --pmc summary when present),
the reference's CPU path timed on this host (``cpu_baseline``) and, when the
model path is available, the MedNeXt-Base 128^3 training-step time.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _path in (ROOT / "mednext-accel_amd", ROOT):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))
# A HIP selection must never run PyTorch's operators in its place here.
os.environ.setdefault("MEDNEXT_ACCEL_AMD_REQUIRE_HIP", "1")

METRIC = "depthwise Conv3d fwd+bwd GB/s (% of HBM peak); MedNeXt-B 128³ train step ms"
HBM_PEAK_GBS = 8000.0
TRAFFIC_SUMMARY = ROOT / "profiles" / "depthwise_k3_c32_128_bf16_traffic.json"


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--channels", type=int, default=32)
    ap.add_argument("--size", type=int, default=128)
    ap.add_argument("--kernel-size", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-block", action="store_true", help="skip the configs[2] block timing")
    ap.add_argument("--no-train-step", action="store_true", help="skip the MedNeXt-Base training-step timing")
    ap.add_argument("--train-steps", type=int, default=50)
    ap.add_argument("--train-warmup", type=int, default=20)
    ap.add_argument("--train-size", type=int, default=128)
    ap.add_argument("--no-eager-step", action="store_true", help="time only the HIP-backed training step")
    ap.add_argument("--no-large-step", action="store_true",
                    help="skip the MedNeXt-Large k5 checkpointed training step (configs[4])")
    ap.add_argument("--large-steps", type=int, default=10)
    ap.add_argument("--large-warmup", type=int, default=5)
    ap.add_argument("--no-v2-step", action="store_true", help="skip the MedNeXt v2 Base training step")
    ap.add_argument("--v2-steps", type=int, default=10)
    ap.add_argument("--v2-warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time budget")
    ap.add_argument("--no-graph-step", action="store_true",
                    help="skip the HIP-graph-captured variants of the training steps")
    ap.add_argument("--train-only", action="store_true", help="time only the training step(s) of --train-variants")
    ap.add_argument("--train-variants", default="base,large,v2",
                    help="comma list of base / large / v2 (eager) and base-graph / large-graph / v2-graph (captured) for "
                         "--train-only (--no-large-step / --no-v2-step drop the eager large / v2)")
    ap.add_argument(
        "--sweep",
        action="store_true",
        help="instead of the headline line, print one JSON line per kernel phase of the configs[1] stage sweep "
        "(depthwise k3/k5 fwd, dX, dW; stride-2 maps; GroupNorm; pointwise GEMMs) and exit",
    )
    ap.add_argument("--sweep-reps", type=int, default=40, help="timed launches per op in --sweep")
    ap.add_argument(
        "--copy-calibration",
        action="store_true",
        help="before timing, run 3 untimed torch.neg launches over 2^27 bf16 elements (256 MiB read, "
        "256 MiB written): the known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE",
    )
    return ap.parse_args()


class GpuLead:
    """Keeps the GPU busy while the host enqueues a timed region, so that HIP
    event intervals measure kernel time rather than Python launch overhead.
    torch.cuda._sleep spins for a number of GPU clock cycles; the rate is
    calibrated once with events."""

    def __init__(self, torch):
        self.torch = torch
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 16)
        torch.cuda.synchronize()
        cycles = 1 << 22
        start.record()
        torch.cuda._sleep(cycles)
        end.record()
        torch.cuda.synchronize()
        self.cycles_per_ms = cycles / max(1e-3, start.elapsed_time(end))

    def __call__(self, ms: float) -> None:
        self.torch.cuda._sleep(int(ms * self.cycles_per_ms))


def time_depthwise(args, torch, hip_ops, lead: GpuLead):
    dev = torch.device("cuda:0")
    c, s, k = args.channels, args.size, args.kernel_size
    shape = (1, c, s, s, s)
    elements = c * s**3
    gen = torch.Generator(device=dev).manual_seed(1234)
    bound = 1.0 / (k**3) ** 0.5
    w = ((torch.rand(c, 1, k, k, k, generator=gen, device=dev) * 2 - 1) * bound).bfloat16()
    b = ((torch.rand(c, generator=gen, device=dev) * 2 - 1) * bound).bfloat16()
    # Three resident input sets (x, dy): 3 * 2 * 134 MB > 256 MB Infinity Cache.
    sets = [
        (
            torch.randn(shape, generator=gen, device=dev).bfloat16(),
            torch.randn(shape, generator=gen, device=dev).bfloat16(),
        )
        for _ in range(3)
    ]
    if args.copy_calibration:
        src = torch.randn(2**27, generator=gen, device=dev).bfloat16()
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        del src, dst
    torch.cuda.synchronize()

    phases = {
        "forward": lambda i: hip_ops.depthwise_forward(sets[i % 3][0], w, b),
        "input_grad": lambda i: hip_ops.depthwise_input_grad(sets[i % 3][1], w),
        "weight_grad": lambda i: hip_ops.depthwise_weight_grad(sets[i % 3][0], sets[i % 3][1], k),
    }
    for i in range(args.warmup):
        for fn in phases.values():
            fn(i)
    torch.cuda.synchronize()
    # Each phase: `steps` back-to-back launches (inputs rotated over the three
    # sets) between two events, after a ~20 ms GPU spin so the host has
    # enqueued them all before the first starts: the mean per launch is the
    # kernels' own time (plus the inter-launch gap).
    mean_ms = {}
    enqueue = 0.0
    for name, fn in phases.items():
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        lead(20.0)
        t0 = time.perf_counter()
        start.record()
        for i in range(args.steps):
            fn(i)
        end.record()
        enqueue += time.perf_counter() - t0
        torch.cuda.synchronize()
        mean_ms[name] = start.elapsed_time(end) / args.steps
    step_ms = sum(mean_ms.values())
    bytes_per_phase = 2 * elements * 2  # two bf16 streams of E elements
    return {
        "elements": elements,
        "bytes_per_phase": bytes_per_phase,
        "mean_ms": mean_ms,
        "step_ms": step_ms,
        "host_enqueue_ms_per_step": 1000.0 * enqueue / max(1, args.steps),
        "gbs": 3 * bytes_per_phase / (step_ms * 1e-3) / 1e9,
    }


def time_cfg0_gpu(args, torch, hip_ops, lead: GpuLead) -> dict:
    """configs[0] on the GPU: fp32 1x32x64^3 k3 forward + input grad + weight
    grad (+ bias grad) through the HIP kernels, the like-for-like counterpart of
    ``cpu_baseline`` (same shape, dtype and 24*E byte count). Inputs rotate over
    six resident sets (402 MB > 256 MB Infinity Cache)."""
    dev = torch.device("cuda:0")
    c, s, k = 32, 64, 3
    gen = torch.Generator(device=dev).manual_seed(1)
    w = (torch.rand(c, 1, k, k, k, generator=gen, device=dev) * 2 - 1) / (k**3) ** 0.5
    b = torch.zeros(c, device=dev)
    sets = [(torch.randn(1, c, s, s, s, generator=gen, device=dev), torch.randn(1, c, s, s, s, generator=gen, device=dev))
            for _ in range(6)]
    phases = {
        "forward": lambda i: hip_ops.depthwise_forward(sets[i % 6][0], w, b),
        "input_grad": lambda i: hip_ops.depthwise_input_grad(sets[i % 6][1], w),
        "weight_grad": lambda i: hip_ops.depthwise_weight_grad(sets[i % 6][0], sets[i % 6][1], k),
    }
    us = {name: _timed_launches(torch, lead, fn, 6, max(10, args.steps)) for name, fn in phases.items()}
    elements = c * s**3
    total_us = sum(us.values())
    return {
        "value": round(3 * 2 * elements * 4 / (total_us * 1e-6) / 1e9, 1),
        "unit": "GB/s",
        "phase_us": {k_: round(v, 2) for k_, v in us.items()},
        "sample": f"HIP kernels (VALU engine, fp32) on cfg0 fp32 1x{c}x{s}^3 k{k}, fwd + dX + dW(+dB), "
                  "mean per launch over back-to-back launches; 24*E algorithmic bytes as cpu_baseline",
    }


def block_reference_op_bytes(channels: int, size: int, ratio: int) -> int:
    """Algorithmic HBM bytes of one MedNeXt block's forward as the reference
    runs it, one operator at a time under bf16 autocast (E = C * S^3 elements,
    hidden R*E): depthwise 4E (bf16 read + write), GroupNorm 6E (bf16 read,
    fp32 write), expand 2E + 2RE, GELU 4RE, project 2RE + 2E, residual add
    6E. Forward + backward counts the forward three times (backward ~ 2x)."""
    e = channels * size**3
    forward = 4 * e + 6 * e + (2 * e + 2 * ratio * e) + 4 * ratio * e + (2 * ratio * e + 2 * e) + 6 * e
    return 3 * forward


def time_block(args, torch, channels: int, size: int, ratio: int, reps: int = 20) -> dict:
    """one MedNeXt block (dw k3 -> GroupNorm -> expand -> GELU ->
    project -> + residual), bf16 autocast, forward + backward, this package's
    block vs the same block as plain PyTorch modules, on the same GPU."""
    import copy

    from mednext_accel_amd import MedNeXtBlock
    from mednext_accel_amd.adaptive import ModelOptimizationContext, install_adaptive_operators
    from mednext_accel_amd.optimization import PolicyRegistry

    torch.manual_seed(11)
    ref = MedNeXtBlock(spatial_dims=3, in_channels=channels, out_channels=channels, expansion_ratio=ratio,
                       kernel_size=3).cuda().train()
    hip = copy.deepcopy(ref)
    install_adaptive_operators(hip, resolver=PolicyRegistry().resolver(),
                               model_context=ModelOptimizationContext("mednext_v1", "base", "none"))
    xs = [torch.randn(1, channels, size, size, size, device="cuda", requires_grad=True) for _ in range(3)]
    g = torch.randn(1, channels, size, size, size, device="cuda").bfloat16()
    out = {}
    for name, block in (("hip", hip), ("reference_eager", ref)):
        def step(i, block=block):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = block(xs[i % 3])
            y.backward(g)

        for i in range(3):
            step(i)
        torch.cuda.synchronize()
        times = []
        for i in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            step(i)
            end.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end))
        out[name] = round(1000.0 * statistics.median(times), 1)
    nbytes = block_reference_op_bytes(channels, size, ratio)
    return {
        "block": f"C={channels} {size}^3 R={ratio} k3",
        "hip_us": out["hip"],
        "reference_eager_us": out["reference_eager"],
        "speedup": round(out["reference_eager"] / out["hip"], 2),
        "reference_op_bytes": nbytes,
        "hip_gbs_at_reference_op_bytes": round(nbytes / (out["hip"] * 1e-6) / 1e9, 1),
        "note": "fwd + bwd, event median of single synchronised steps (host launch time included); "
                "reference_op_bytes = the reference's per-operator HBM traffic (forward x3)",
    }


# Kernel-name prefixes (rocprofv3 short names) launched by each phase at k=3 bf16.
PHASE_KERNELS = {
    "forward": ("dw_mfma_stencil_kernel<3, false",),
    "input_grad": ("dw_mfma_stencil_kernel<3, true",),
    "weight_grad": ("dw_mfma_wgrad_kernel<3,", "dw_wgrad_finish_kernel<"),
}


def time_copy_ceiling(torch) -> dict:
    """Attainable streaming rate on this GPU: torch.neg over 2^27 bf16 elements
    (256 MiB read + 256 MiB written), median of 20 event-timed launches over
    two rotating buffer pairs (1 GiB in total, above the 256 MiB Infinity Cache)."""
    n = 2**27
    pairs = [(torch.randn(n, device="cuda").bfloat16(), torch.empty(n, device="cuda", dtype=torch.bfloat16)) for _ in range(2)]
    for i in range(4):
        torch.neg(pairs[i % 2][0], out=pairs[i % 2][1])
    torch.cuda.synchronize()
    events = []
    for i in range(20):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        torch.neg(pairs[i % 2][0], out=pairs[i % 2][1])
        b.record()
        events.append((a, b))
    torch.cuda.synchronize()
    ms = statistics.median(a.elapsed_time(b) for a, b in events)
    del pairs
    torch.cuda.empty_cache()
    return {"kernel": "torch.neg, 2^27 bf16 (512 MiB moved)", "us": round(ms * 1000, 2),
            "gbs": round(2 * n * 2 / (ms * 1e-3) / 1e9, 1)}


def time_train_step(args, torch, optimization: str, variant: str = "base", steps: int | None = None,
                    warmup: int | None = None, graph: bool = False) -> dict:
    """MedNeXt training step at 1x1xS^3 in bf16 autocast with AdamW, the
    reference's step protocol (benchmarks/implementations.py:133-190): event
    median over the timed steps. ``base``: MedNeXt-Base k3, no checkpointing
    (configs[3]); ``large``: MedNeXt-Large k5 with expansion-branch
    checkpointing on all stages; ``v2``: MedNeXt v2 Base (GRN in
    every expansion), no checkpointing. ``graph``: the whole step (forward,
    loss, backward, AdamW with device-side step counters) captured once as a
    HIP graph after the warm-up steps and replayed; every replay does the
    full step's work."""
    from mednext_accel_amd import CheckpointConfig, mednext_base, mednext_large, mednext_v2_base
    from mednext_accel_amd.step import GraphedTrainingStep, make_training_step

    steps = args.train_steps if steps is None else steps
    warmup = args.train_warmup if warmup is None else warmup
    torch.manual_seed(1234)
    if variant == "v2":
        model = mednext_v2_base(in_channels=1, out_channels=3, deep_supervision=True, optimization=optimization)
    elif variant == "large":
        model = mednext_large(in_channels=1, out_channels=3, kernel_size=5, deep_supervision=True,
                              checkpointing=CheckpointConfig(style="expansion", stages=None), optimization=optimization)
    else:
        model = mednext_base(in_channels=1, out_channels=3, kernel_size=3, deep_supervision=True,
                             optimization=optimization)
    model = model.cuda().train()
    step = make_training_step(model, size=args.train_size, device="cuda", capturable=graph)
    if graph:
        step = GraphedTrainingStep(step, warmup=max(1, warmup))
    else:
        for _ in range(warmup):
            step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    events = []
    wall0 = time.perf_counter()
    for _ in range(steps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        step()
        end.record()
        events.append((start, end))
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    times = [a.elapsed_time(b) for a, b in events]
    result = {
        "median_step_ms": round(statistics.median(times), 3),
        "mean_wall_step_ms": round(1000.0 * wall / max(1, steps), 3),
        "peak_allocated_mib": round(torch.cuda.max_memory_allocated() / 2**20, 1),
        "final_loss": round(float(step.last_loss.detach()), 5),
        "steps_run": warmup + steps,
    }
    if graph:
        result["captured"] = "hip_graph"
    del step, model
    torch.cuda.empty_cache()
    return result


def load_traffic(phase: str, kernel_size: int):
    """HBM bytes per launch of ``phase`` from the committed, calibrated
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (k=3 headline workload only)."""
    if kernel_size != 3 or not TRAFFIC_SUMMARY.exists():
        return None
    try:
        kernels = json.loads(TRAFFIC_SUMMARY.read_text())["kernels"]
    except (OSError, ValueError, KeyError):
        return None
    total, found = 0, set()
    for name, entry in kernels.items():
        for prefix in PHASE_KERNELS[phase]:
            if name.startswith(prefix):
                total += entry["hbm_bytes_per_launch"]
                found.add(prefix)
    return total if len(found) == len(PHASE_KERNELS[phase]) else None


def cpu_baseline(args, torch):
    """The reference's CPU path (F.conv3d + aten.convolution_backward) on a
    bounded sample: cfg0's fp32 1x32x64^3 (fp32: bf16 CPU depthwise-3D is not a
    reliable baseline), repeated until ~cpu_seconds are spent."""
    from oracle.reference_cpu import depthwise_phases

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(1)
    c, s, k = 32, 64, 3
    x = torch.randn(1, c, s, s, s, generator=gen)
    w = (torch.rand(c, 1, k, k, k, generator=gen) * 2 - 1) / (k**3) ** 0.5
    b = torch.zeros(c)
    dy = torch.randn(1, c, s, s, s, generator=torch.Generator().manual_seed(2))
    depthwise_phases(x, w, b, dy)  # warmup
    times = []
    budget_end = time.perf_counter() + args.cpu_seconds
    while len(times) < 3 or (time.perf_counter() < budget_end and len(times) < 50):
        t0 = time.perf_counter()
        depthwise_phases(x, w, b, dy)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    elements = c * s**3
    bytes_fwd_bwd = 3 * 2 * elements * 4  # three phases, two fp32 streams each
    return {
        "value": round(bytes_fwd_bwd / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": (
            f"reference CPU path (F.conv3d fwd + aten.convolution_backward dX, dW+dB) on cfg0 "
            f"fp32 1x{c}x{s}^3 k{k}, {len(times)} reps, median {med * 1000:.1f} ms per fwd+bwd; "
            f"same 24*E algorithmic-byte count as the GPU metric's fp32 form; os.cpu_count()={threads}"
        ),
    }

STAGE_SHAPES = ((32, 128), (64, 64), (128, 32), (256, 16), (512, 8))
# MedNeXt-Base expansion ratios of the encoder stages 0-4 (stage 4 = bottleneck).
BASE_RATIOS = (2, 3, 4, 4, 4)
V2_RATIOS = (3, 4, 8, 8, 8)  # MedNeXt v2 encoder expansion ratios
MFMA_BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 768 << 20  # rotate inputs over > 3x the 256 MiB Infinity Cache


def _timed_launches(torch, lead: GpuLead, launch, sets: int, reps: int) -> float:
    """Mean microseconds per launch of ``launch(i)`` over ``reps`` launches
    bracketed by two events, inputs rotated over ``sets`` resident copies.
    The warm-up launches and the timed launches each follow a GPU spin
    kernel, so a kernel trace splits into (warm-up, timed) segments per op in
    sweep order (what the rocprofv3 counter summaries attribute by)."""
    lead(0.01)
    for i in range(min(reps, 3)):
        launch(i % sets)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    lead(20.0)
    start.record()
    for i in range(reps):
        launch(i % sets)
    end.record()
    torch.cuda.synchronize()
    return 1000.0 * start.elapsed_time(end) / reps


def _emit(record: dict) -> None:
    print(json.dumps(record), flush=True)


def sweep(args, torch, hip_ops, lead: GpuLead) -> None:
    """configs[1] stage sweep (depthwise k3/k5 fwd, dX, dW at every MedNeXt
    stage shape, N=1, bf16) plus the other kernels of the training step at the
    same shapes: stride-2 gather / scatter / reduce (k3 and k5), GroupNorm
    forward and backward, and the six pointwise GEMMs of a fused MedNeXt-Base
    block expansion in the form the training step runs at that width. One JSON line per kernel phase: mean microseconds per launch
    (events around ``reps`` back-to-back launches, the GPU kept ahead of the
    host), algorithmic bytes, GB/s and, for the GEMMs, TFLOP/s."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1234)
    reps = args.sweep_reps

    def randn(*shape):
        return torch.randn(shape, generator=gen, device=dev).bfloat16()

    def record(op, shape, us, nbytes, flops=None, **extra):
        rec = {"op": op, "shape": shape, "us": round(us, 2), "bytes": nbytes,
               "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if flops is not None:
            tf = flops / (us * 1e-6) / 1e12
            rec.update(tflops=round(tf, 2), mfma_frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4))
        rec.update(extra)
        _emit(rec)

    # A plain copy of known size first: the counter summaries scale rocprofv3's
    # FETCH_SIZE / WRITE_SIZE by what they read for it.
    src = randn(2**27)
    dsts = [torch.empty_like(src) for _ in range(2)]
    us = _timed_launches(torch, lead, lambda i: torch.neg(src, out=dsts[i]), 2, reps)
    record("copy_calibration", "2^27 bf16 (torch.neg)", us, 2 * src.numel() * 2)
    del src, dsts
    torch.cuda.empty_cache()

    for (c, s), ratio in zip(STAGE_SHAPES, V2_RATIOS):
        # GRN of a MedNeXt v2 expansion (C * ratio channels) at this stage, bf16
        # in / out, float32 affine, autocast form (bf16 upstream gradient).
        # Algorithmic bytes: forward reads x, writes y; backward reads dy and x,
        # writes dx (the kernels read x a second time to apply the norms).
        m = c * ratio
        e = m * s**3
        nsets = max(1, min(12, -(-ROTATE_BYTES // (4 * e))))
        gx = [randn(1, m, s, s, s) for _ in range(nsets)]
        gdy = [randn(1, m, s, s, s) for _ in range(nsets)]
        gam = torch.randn(1, m, 1, 1, 1, generator=gen, device=dev)
        bet = torch.randn(1, m, 1, 1, 1, generator=gen, device=dev)
        us = _timed_launches(torch, lead, lambda i: hip_ops.grn_forward(gx[i], gam, bet), nsets, reps)
        record("grn_forward", f"1x{m}x{s}^3", us, 4 * e)
        coefs = [hip_ops.grn_forward(gx[i], gam, bet)[1] for i in range(nsets)]
        us = _timed_launches(
            torch, lead, lambda i: hip_ops.grn_backward(gdy[i], gx[i], coefs[i], gam, param_shape=(1, m, 1, 1, 1)),
            nsets, reps)
        record("grn_backward", f"1x{m}x{s}^3", us, 6 * e)
        del gx, gdy, coefs
        torch.cuda.empty_cache()

    for (c, s), ratio in zip(STAGE_SHAPES, BASE_RATIOS):
        e = c * s**3
        nsets = max(1, min(24, -(-ROTATE_BYTES // (4 * e))))
        xs = [randn(1, c, s, s, s) for _ in range(nsets)]
        dys = [randn(1, c, s, s, s) for _ in range(nsets)]
        shape = f"1x{c}x{s}^3"
        for k in (3, 5):
            bound = 1.0 / (k**3) ** 0.5
            w = ((torch.rand(c, 1, k, k, k, generator=gen, device=dev) * 2 - 1) * bound).bfloat16()
            b = ((torch.rand(c, generator=gen, device=dev) * 2 - 1) * bound).bfloat16()
            us = _timed_launches(torch, lead, lambda i: hip_ops.depthwise_forward(xs[i], w, b), nsets, reps)
            record(f"depthwise_k{k}_forward", shape, us, 4 * e)
            us = _timed_launches(torch, lead, lambda i: hip_ops.depthwise_input_grad(dys[i], w), nsets, reps)
            record(f"depthwise_k{k}_input_grad", shape, us, 4 * e)
            us = _timed_launches(torch, lead, lambda i: hip_ops.depthwise_weight_grad(xs[i], dys[i], k), nsets, reps)
            record(f"depthwise_k{k}_weight_grad", shape, us, 4 * e)
        if s >= 16:
            # Stride-2 maps of the down block entering the next stage (C -> C at S -> S/2), k3 and k5.
            small = hip_ops.strided_spatial((s, s, s))
            es = c * small[0] * small[1] * small[2]
            smalls = [randn(1, c, *small) for _ in range(nsets)]
            for k2 in (3, 5):
                wk = randn(c, 1, k2, k2, k2) * (0.6 / k2**1.5)
                us = _timed_launches(torch, lead, lambda i: hip_ops.depthwise_s2_gather(xs[i], wk, None, small), nsets,
                                     reps)
                record(f"depthwise_s2_k{k2}_gather", shape, us, 2 * (e + es))
                us = _timed_launches(torch, lead, lambda i: hip_ops.depthwise_s2_scatter(smalls[i], wk, None, (s, s, s)),
                                     nsets, reps)
                record(f"depthwise_s2_k{k2}_scatter", shape, us, 2 * (e + es))
                us = _timed_launches(torch, lead, lambda i: hip_ops.depthwise_s2_wgrad(xs[i], smalls[i], k2), nsets, reps)
                record(f"depthwise_s2_k{k2}_wgrad", shape, us, 2 * (e + es))
            del smalls
        gamma = torch.ones(c, device=dev)
        beta = torch.zeros(c, device=dev)
        # Autocast form: bf16 in, fp32 out (forward); fp32 dy, bf16 x, bf16 dx (backward).
        us = _timed_launches(torch, lead, lambda i: hip_ops.group_norm_forward(xs[i], gamma, beta, out_dtype=torch.float32), nsets, reps)
        record("group_norm_forward_bf16_to_fp32", shape, us, 2 * e + 2 * e + 4 * e)
        us = _timed_launches(torch, lead, lambda i: hip_ops.group_norm_forward(xs[i], gamma, beta, out_dtype=torch.bfloat16), nsets, reps)
        record("group_norm_forward_bf16", shape, us, 2 * e + 2 * e + 2 * e)
        _, mean, rstd = hip_ops.group_norm_forward(xs[0], gamma, beta)
        dys32 = [t.float() for t in dys[: max(1, nsets // 2)]]
        us = _timed_launches(
            torch, lead, lambda i: hip_ops.group_norm_backward(dys32[i], xs[i], mean, rstd, gamma), len(dys32), reps
        )
        record("group_norm_backward_fp32dy", shape, us, 2 * (4 * e + 2 * e) + 2 * e)
        del dys32
        # Pointwise GEMMs of a fused block expansion C -> R*C -> C at this stage
        # (stages whose hidden width exceeds the matrix-core kernel's K limit run
        # PyTorch's GEMMs in the model and are not swept).
        m = ratio * c
        from mednext_accel_amd.tiles import pointwise_supported

        if not pointwise_supported(c, m, s**3):
            del xs, dys
            torch.cuda.empty_cache()
            continue
        hs = [randn(1, m, s, s, s) for _ in range(max(1, nsets // ratio))]
        nh = len(hs)
        w1 = randn(m, c, 1, 1, 1) * 0.1
        b1 = randn(m) * 0.1
        w2 = randn(c, m, 1, 1, 1) * 0.1
        b2 = randn(c) * 0.1
        v = s**3
        fl = 2 * m * c * v
        P = hip_ops
        from mednext_accel_amd.adaptive import AdaptiveExpansion

        if m >= AdaptiveExpansion.stored_gelu_from:
            # The fused expansion's stored-GELU form (what the training step
            # runs at this width): expand writes GELU and GELU', project reads
            # GELU as is, its input gradient scales by the stored GELU'.
            gs = [randn(1, m, s, s, s) for _ in range(nh)]
            us = _timed_launches(
                torch, lead, lambda i: P.pointwise_conv(xs[i % nh], w1, b1, epilogue=P.PW_EPILOGUE_BIAS_GELU_PAIR),
                nh, reps)
            record("pointwise_expand_fwd_gelu_pair", f"{shape} {c}->{m}", us, 2 * v * (c + 2 * m), fl)
            us = _timed_launches(
                torch, lead, lambda i: P.pointwise_conv(hs[i], w2, b2, aux=xs[i], epilogue=P.PW_EPILOGUE_BIAS_RESIDUAL),
                nh, reps)
            record("pointwise_project_fwd_residual", f"{shape} {m}->{c}", us, 2 * v * (m + 2 * c), fl)
            us = _timed_launches(
                torch, lead,
                lambda i: P.pointwise_conv(dys[i], w2, aux=gs[i], epilogue=P.PW_EPILOGUE_AUX_SCALE, transpose=True),
                nh, reps)
            record("pointwise_project_dgrad_aux_scale", f"{shape} {c}->{m}", us, 2 * v * (c + 2 * m), fl)
            us = _timed_launches(torch, lead, lambda i: P.pointwise_weight_grad(dys[i], hs[i]), nh, reps)
            record("pointwise_project_wgrad", f"{shape} {m}x{c}", us, 2 * v * (m + c), fl)
            del gs
        else:
            us = _timed_launches(torch, lead, lambda i: P.pointwise_conv(xs[i % nh], w1, b1), nh, reps)
            record("pointwise_expand_fwd", f"{shape} {c}->{m}", us, 2 * v * (c + m), fl)
            us = _timed_launches(
                torch, lead,
                lambda i: P.pointwise_conv(hs[i], w2, b2, aux=xs[i], prologue=P.PW_PROLOGUE_GELU,
                                           epilogue=P.PW_EPILOGUE_BIAS_RESIDUAL),
                nh, reps)
            record("pointwise_project_fwd_gelu_residual", f"{shape} {m}->{c}", us, 2 * v * (m + 2 * c), fl)
            us = _timed_launches(
                torch, lead,
                lambda i: P.pointwise_conv(dys[i], w2, aux=hs[i], epilogue=P.PW_EPILOGUE_GELU_GRAD, transpose=True),
                nh, reps)
            record("pointwise_project_dgrad_gelu_grad", f"{shape} {c}->{m}", us, 2 * v * (c + 2 * m), fl)
            us = _timed_launches(
                torch, lead, lambda i: P.pointwise_weight_grad(dys[i], hs[i], prologue=P.PW_PROLOGUE_GELU), nh, reps)
            record("pointwise_project_wgrad_gelu", f"{shape} {m}x{c}", us, 2 * v * (m + c), fl)
        us = _timed_launches(torch, lead, lambda i: P.pointwise_weight_grad(hs[i], xs[i]), nh, reps)
        record("pointwise_expand_wgrad", f"{shape} {m}x{c}", us, 2 * v * (m + c), fl)
        us = _timed_launches(torch, lead, lambda i: P.pointwise_conv(hs[i], w1, transpose=True), nh, reps)
        record("pointwise_expand_dgrad", f"{shape} {m}->{c}", us, 2 * v * (m + c), fl)
        del xs, dys, hs
        torch.cuda.empty_cache()


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only (got --gpus {args.gpus}): this operator path has no "
            "multi-GPU mode (it would shard by data parallelism: one process per GPU, each running "
            "these kernels on its own batch share, gradients all-reduced in buckets over RCCL).",
            file=sys.stderr,
        )
        return 2
    import torch

    from mednext_accel_amd import hip_ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    lead = GpuLead(torch)
    if args.sweep:
        sweep(args, torch, hip_ops, lead)
        return 0
    if args.train_only:
        variants = {v.strip() for v in args.train_variants.split(",") if v.strip()}
        out = {}
        if "base" in variants:
            out["train_step_hip"] = time_train_step(args, torch, "auto")
        if "large" in variants and not args.no_large_step:
            out["train_step_large_hip"] = time_train_step(args, torch, "auto", "large", args.large_steps,
                                                          args.large_warmup)
        if "v2" in variants and not args.no_v2_step:
            out["train_step_v2_hip"] = time_train_step(args, torch, "auto", "v2", args.v2_steps, args.v2_warmup)
        if "base-graph" in variants:
            out["train_step_hip_graph"] = time_train_step(args, torch, "auto", graph=True)
        if "large-graph" in variants:
            out["train_step_large_hip_graph"] = time_train_step(args, torch, "auto", "large", args.large_steps,
                                                                args.large_warmup, graph=True)
        if "v2-graph" in variants:
            out["train_step_v2_hip_graph"] = time_train_step(args, torch, "auto", "v2", args.v2_steps,
                                                             args.v2_warmup, graph=True)
        print(json.dumps(out))
        return 0
    dw = time_depthwise(args, torch, hip_ops, lead)
    ceiling = time_copy_ceiling(torch)
    phase_us = {name: round(1000.0 * ms, 2) for name, ms in dw["mean_ms"].items()}
    dominant = max(dw["mean_ms"], key=dw["mean_ms"].get)
    achieved = dw["bytes_per_phase"] / (dw["mean_ms"][dominant] * 1e-3) / 1e9
    roofline = {
        "bound": "hbm",
        "kernel": {
            "forward": "dw_mfma_stencil_kernel<K,FLIP=false>",
            "input_grad": "dw_mfma_stencil_kernel<K,FLIP=true>",
            "weight_grad": "dw_mfma_wgrad_kernel + dw_wgrad_finish_kernel",
        }[dominant],
        "phase": dominant,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": load_traffic(dominant, args.kernel_size) if (args.channels, args.size) == (32, 128) else None,
        "copy_ceiling_gbs": ceiling["gbs"],
        "frac_of_copy_ceiling": round(achieved / ceiling["gbs"], 4),
        "algorithmic_bytes_per_launch": dw["bytes_per_phase"],
    }
    result = {
        "metric": METRIC,
        "value": round(dw["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dw["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (
                f"depthwise_conv3d k{args.kernel_size} forward + input_grad + weight_grad(+fused bias_grad), "
                f"N=1 C={args.channels} D=H=W={args.size}, bf16 in / fp32 accumulate, inputs ~N(0,1) "
                "rotated over 3 resident sets (BASELINE configs[1] headline shape)"
            ),
            "hbm_frac_of_peak": round(dw["gbs"] / HBM_PEAK_GBS, 4),
            "phase_us": phase_us,
            "host_enqueue_ms_per_step": round(dw["host_enqueue_ms_per_step"], 4),
            "copy_ceiling": ceiling,
        },
        "roofline": roofline,
    }
    if not args.no_train_step:
        ours = time_train_step(args, torch, "auto")
        ours_graph = None if args.no_graph_step else time_train_step(args, torch, "auto", graph=True)
        eager = None if args.no_eager_step else time_train_step(args, torch, "reference")
        result["train_step"] = {
            "model": (
                f"MedNeXt-Base k3, 1x1x{args.train_size}^3, 5-head deep supervision, bf16 autocast, AdamW lr 1e-3, "
                "random init, synthetic N(0,1) input and uniform labels (BASELINE configs[3])"
            ),
            "steps": args.train_steps,
            "warmup": args.train_warmup,
            "hip": ours,
            "hip_graph": ours_graph,
            "reference_eager": eager,
            "speedup_vs_reference_eager": round(eager["median_step_ms"] / ours["median_step_ms"], 3) if eager else None,
            "graph_speedup_vs_reference_eager": round(eager["median_step_ms"] / ours_graph["median_step_ms"], 3)
            if eager and ours_graph else None,
        }
        if not args.no_large_step:
            big = time_train_step(args, torch, "auto", "large", args.large_steps, args.large_warmup)
            big_graph = None if args.no_graph_step else time_train_step(
                args, torch, "auto", "large", args.large_steps, args.large_warmup, graph=True)
            # Same warm-up and timed step counts as the HIP legs, so the final
            # losses are taken after the same number of AdamW steps.
            big_eager = None if args.no_eager_step else time_train_step(
                args, torch, "reference", "large", args.large_steps, args.large_warmup)
            result["train_step_large"] = {
                "model": (
                    f"MedNeXt-Large k5, 1x1x{args.train_size}^3, 5-head deep supervision, expansion-branch "
                    "checkpointing on all stages, bf16 autocast, AdamW lr 1e-3 (BASELINE configs[4])"
                ),
                "hip": big,
                "hip_graph": big_graph,
                "reference_eager": big_eager,
                "speedup_vs_reference_eager": round(big_eager["median_step_ms"] / big["median_step_ms"], 3)
                if big_eager else None,
                "graph_speedup_vs_reference_eager": round(big_eager["median_step_ms"] / big_graph["median_step_ms"], 3)
                if big_eager and big_graph else None,
            }
    if not args.no_train_step and not args.no_v2_step:
        v2 = time_train_step(args, torch, "auto", "v2", args.v2_steps, args.v2_warmup)
        v2_graph = None if args.no_graph_step else time_train_step(
            args, torch, "auto", "v2", args.v2_steps, args.v2_warmup, graph=True)
        v2_eager = None if args.no_eager_step else time_train_step(
            args, torch, "reference", "v2", args.v2_steps, args.v2_warmup)
        result["train_step_v2"] = {
            "model": (
                f"MedNeXt v2 Base (GRN), 1x1x{args.train_size}^3, 5-head deep supervision, no checkpointing, "
                "bf16 autocast, AdamW lr 1e-3, random init, synthetic N(0,1) input and uniform labels"
            ),
            "hip": v2,
            "hip_graph": v2_graph,
            "reference_eager": v2_eager,
            "speedup_vs_reference_eager": round(v2_eager["median_step_ms"] / v2["median_step_ms"], 3)
            if v2_eager else None,
            "graph_speedup_vs_reference_eager": round(v2_eager["median_step_ms"] / v2_graph["median_step_ms"], 3)
            if v2_eager and v2_graph else None,
        }
    if not args.no_block:
        result["block_cfg2"] = [time_block(args, torch, 32, 128, 2), time_block(args, torch, 128, 32, 4)]
    result["cfg0_gpu_fp32"] = time_cfg0_gpu(args, torch, hip_ops, lead)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, torch)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
