"""Integrated per-phase operator measurement on the GPU (reference
profiling/operator_benchmark.py:39-252, ``benchmark_operator``).

The native PyTorch module and the adaptive wrapper around a copy of it run
on the same seeded inputs. The wrapper's resolver holds a single-rule policy
that selects the candidate (implementation, launch recipe) for the measured
phase only, so every other phase stays native in both modules and the
difference is this case's dispatch decision. Each component the phase
produces is validated (``validation.validate_components``) before timing.

Only the measured phase's gradients require grad (input for dX, weight and
bias for dW and dB), so no backward op also computes another phase.

Timing: ``repetitions`` launches of the phase, each between two HIP events,
queued behind a GPU spin so the host has enqueued them all before the first
starts; the median per launch is reported. Backward phases build their
forward graphs before the timed region and time only the gradient call.
"""

from __future__ import annotations

import copy
import statistics

import torch
from torch import nn

from ..adaptive import (
    AdaptiveDepthwise3d,
    AdaptiveGroupNorm3d,
    AdaptivePointwise3d,
    ModelOptimizationContext,
    device_facts,
)
from ..optimization.policy import parse_policy
from ..optimization.policy_resolver import PolicyResolver
from .matrix import KernelCase
from .validation import validate_components


def _native_module(case: KernelCase) -> nn.Module:
    if case.family == "depthwise_conv3d":
        c, k = case.in_channels, case.kernel_size
        return nn.Conv3d(c, c, k, padding=k // 2, groups=c)
    if case.family == "group_norm3d":
        norm = nn.GroupNorm(case.in_channels, case.in_channels)
        with torch.no_grad():  # non-trivial affine parameters exercise every gradient term
            norm.weight.uniform_(0.5, 1.5)
            norm.bias.uniform_(-0.5, 0.5)
        return norm
    if case.family == "pointwise_conv3d":
        return nn.Conv3d(case.in_channels, case.out_channels, 1)
    raise ValueError(f"no integrated benchmark for family {case.family!r}")


def candidate_policy(case: KernelCase, arch: str | None) -> dict[str, object]:
    """Single-rule policy selecting the case's candidate for its phase."""
    use: dict[str, object] = {"implementation": case.implementation}
    if case.parameters:
        use["parameters"] = dict(case.parameters)
    target: dict[str, object] = {"vendor": "amd"}
    if arch:
        target["arch"] = arch
    return {
        "version": 2,
        "kind": "mednext-accel-policy",
        "name": "integrated-candidate",
        "target": target,
        "rules": [{"id": "candidate", "when": {"family": case.family}, "use": {case.phase: use},
                   "confidence": "measured-exact-context"}],
    }


class _Spin:
    def __init__(self) -> None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 14)
        a.record()
        torch.cuda._sleep(1 << 21)
        b.record()
        torch.cuda.synchronize()
        self.cycles_per_ms = (1 << 21) / max(1e-3, a.elapsed_time(b))

    def __call__(self, ms: float) -> None:
        torch.cuda._sleep(int(ms * self.cycles_per_ms))


def _median_ms(spin: _Spin, calls, lead_ms: float) -> float:
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in calls]
    spin(lead_ms)
    for (a, b), call in zip(events, calls):
        a.record()
        call()
        b.record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in events)


def benchmark_operator(case: KernelCase, *, seed: int = 0, repetitions: int = 10, warmup: int = 2,
                       reference_ms: float | None = None) -> dict[str, object]:
    """Validate and time one candidate; returns scalar evidence only.

    ``reference_ms`` skips re-timing the native module when the caller has
    already measured it for this context and phase."""
    if not torch.cuda.is_available():
        raise RuntimeError("benchmark_operator needs a GPU")
    if case.dtype != "bfloat16":
        raise ValueError("integrated operator benchmarks run under bf16 autocast")
    torch.manual_seed(seed)
    dev = torch.device("cuda")
    native = _native_module(case).to(dev).train()
    _, _, arch = device_facts(torch.cuda.current_device())
    resolver = PolicyResolver(external=parse_policy(candidate_policy(case, arch)))
    context = ModelOptimizationContext("mednext_v1", "base", "none")
    wrapper = {"depthwise_conv3d": AdaptiveDepthwise3d, "group_norm3d": AdaptiveGroupNorm3d,
               "pointwise_conv3d": AdaptivePointwise3d}[case.family]
    candidate = wrapper(copy.deepcopy(native), resolver, context)
    # Gradient mask (as the reference's): only the measured phase's gradients
    # are requested, so a backward op never also computes another phase.
    need_x = case.phase in ("forward", "backward_input", "training")
    need_params = case.phase in ("forward", "backward_weight", "training")
    for module in (native, candidate):
        module.weight.requires_grad_(need_params)
        module.bias.requires_grad_(need_params)
    x = torch.randn(case.batch, case.in_channels, *case.spatial_shape, device=dev, dtype=torch.bfloat16,
                    requires_grad=need_x)
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    out_shape = (case.batch, case.out_channels, *case.spatial_shape)
    grad = torch.randn(out_shape, device=dev, generator=gen).bfloat16()

    def forward(module):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return module(x)

    def targets(module):
        if case.phase == "backward_input":
            return (x,)
        if case.phase == "backward_weight":
            return (module.weight, module.bias)
        if case.phase == "training":
            return (x, module.weight, module.bias)
        return ()

    names = {"forward": ("output",), "backward_input": ("dX",), "backward_weight": ("dW", "dB"),
             "training": ("output", "dX", "dW", "dB")}[case.phase]

    def components(module) -> dict[str, torch.Tensor]:
        out = forward(module)
        got = {"output": out.detach().float()} if "output" in names else {}
        tg = targets(module)
        if tg:
            grads = torch.autograd.grad(out, tg, grad.to(out.dtype))
            got.update({n: g.detach().float() for n, g in zip(names[-len(tg):], grads)})
        return got

    verdict = validate_components(components(candidate), components(native))
    result: dict[str, object] = {"case": case, **verdict, "status": "ok"}
    if not verdict["valid"]:
        return result
    spin = _Spin()

    def phase_ms(module) -> float:
        for _ in range(warmup):
            components(module)
        torch.cuda.synchronize()
        if case.phase == "forward":
            calls = [lambda: forward(module)] * repetitions
        elif case.phase == "training":
            def step():
                out = forward(module)
                torch.autograd.grad(out, targets(module), grad.to(out.dtype))
            calls = [step] * repetitions
        else:
            outs = [forward(module) for _ in range(repetitions)]
            calls = [lambda o=o: torch.autograd.grad(o, targets(module), grad.to(o.dtype)) for o in outs]
        return _median_ms(spin, calls, lead_ms=2.0 * repetitions)

    cand = phase_ms(candidate)
    ref = reference_ms if reference_ms is not None else phase_ms(native)
    result.update(candidate_ms=cand, reference_ms=ref, speedup=ref / cand if cand > 0 else None)
    return result
