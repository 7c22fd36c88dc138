"""The rocprofv3 report tools (CPU, synthetic traces): the training-step
breakdown's step delimiting and per-step sums, and the counter attribution's
phase segmentation and traffic calibration."""

from __future__ import annotations

import csv
import json

import pytest

from mednext_accel_amd.profiling import breakdown, counters


def _trace(kernels):
    """rocprofv3 kernel-trace rows for (name, duration ns) in dispatch order."""
    rows, t = [], 1000
    for name, dur in kernels:
        rows.append({"Kernel_Name": name, "Start_Timestamp": str(t), "End_Timestamp": str(t + dur)})
        t += dur + 10
    return rows


def _step(scale=1):
    return [("void mednext::(anonymous namespace)::dw_band_stencil_kernel<bf16_t>(float*)", 3000 * scale),
            ("void mednext::pw_fwd_kernel<2, 2, 0, 6>(bf16_t const*)", 5000),
            ("void mednext::pw_fwd_kernel<2, 2, 0, 6>(bf16_t const*)", 7000),
            ("void at::native::vectorized_elementwise_kernel<4, bfloat16_copy_kernel_cuda>()", 1000),
            ("void multi_tensor_apply_kernel<FusedAdamMathFunc>()", 2000),
            ("void multi_tensor_apply_kernel<FusedAdamMathFunc>()", 2000)]


def test_breakdown_counts_only_whole_steps():
    # A partial first step (no optimizer before it) and three whole steps; the
    # first step's depthwise kernel is 100x slower and must not be counted.
    rows = _trace(_step(100) + _step() + _step() + _step())
    kernels, used = breakdown.per_step(rows, steps=5, gap=2)
    assert used == 3  # four optimizer runs close four steps; the first is partial
    assert kernels["dw_band_stencil_kernel<bf16_t>"] == [pytest.approx(0.003), 1.0]
    assert kernels["pw_fwd_kernel<2, 2, 0, 6>"] == [pytest.approx(0.012), 2.0]
    assert kernels["multi_tensor_apply_kernel<FusedAdamMathFunc>"][1] == 2.0
    text = breakdown.report(rows, "t", "cmd", steps=2, gap=2)
    assert "the last 2 steps" in text and "GPU busy time 0.02 ms per step" in text
    assert "| pointwise GEMMs (HIP) | 0.012 | 60.0% |" in text


def test_breakdown_categories_and_short_names():
    assert breakdown.short_name("void mednext::(anonymous namespace)::gn_apply_kernel<bf16_t, bf16_t>(x)") == \
        "gn_apply_kernel<bf16_t, bf16_t>"
    assert breakdown.category("s2_wgrad_kernel<bf16_t, float, 5>") == "depthwise (HIP)"
    assert breakdown.category("Cijk_Ailk_Bljk") == "native conv / GEMM"
    assert breakdown.category("reduce_kernel<512>") == "other native elementwise / reductions"
    with pytest.raises(ValueError):
        breakdown.per_step(_trace(_step()), steps=5, gap=2)
    # with the default gap, optimizer launches this close merge into one run
    assert breakdown.step_bounds([n for n, _ in _step() * 3]) == [17]


def _pmc_csv(path, dispatches):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, values) in enumerate(dispatches):
            for c, v in values.items():
                w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": c, "Counter_Value": v})


def test_counters_attribute_timed_segments_and_scale_traffic(tmp_path):
    spin = ("spin_kernel(int)", {"FETCH_SIZE": 0, "WRITE_SIZE": 0})
    neg = ("void at::native::neg_kernel_cuda(x)", {"FETCH_SIZE": 2048, "WRITE_SIZE": 1024})
    dw = ("void mednext::dw_band_stencil_kernel<bf16_t>(x)", {"FETCH_SIZE": 4096, "WRITE_SIZE": 512})
    # start-up spins, then per phase: spin, warm-up launches, spin, timed launches
    seq = [spin, spin, spin, neg, spin, neg, neg, spin, dw, spin, dw, dw]
    _pmc_csv(tmp_path / "p.csv", seq)
    phases = counters.attribute(str(tmp_path / "p.csv"), 2)
    assert phases[0]["neg_kernel"]["FETCH_SIZE"] == 2048
    assert phases[1]["dw_band_stencil_kernel<bf16_t>"]["WRITE_SIZE"] == 512
    with pytest.raises(ValueError):
        counters.attribute(str(tmp_path / "p.csv"), 3)
    sweep = [{"op": "copy_calibration", "shape": "-", "us": 10.0, "bytes": 2 * 4096 * 1024, "gbs": 1, "hbm_frac": 0},
             {"op": "dw", "shape": "s", "us": 10.0, "bytes": 8 * 2**20, "gbs": 1, "hbm_frac": 0}]
    text = counters.table(sweep, phases)
    # calibration: 4096 KiB moved each way; fetch counted 2048 -> x2, write 1024 -> x4
    assert text.startswith("FETCH_SIZE scale 2.000, WRITE_SIZE scale 4.000")
    row = text.splitlines()[-1]
    assert "| 10.0 |" in row  # (4096 * 2 + 512 * 4) KiB = 10 MiB of traffic
    (tmp_path / "s.jsonl").write_text("\n".join(json.dumps(r) for r in sweep) + "\n")
    assert counters.main(["--sweep", str(tmp_path / "s.jsonl"), "--pass", str(tmp_path / "p.csv")]) == 0
