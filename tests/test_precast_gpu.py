"""The per-forward parameter pre-cast on the GPU: one MedNeXt v1 and one v2
training step with and without it, from the same weights on the same data.
The pre-cast copies and the per-operator casts round the same fp32 values,
and the gradients come back through the same bf16 -> fp32 widening, so loss
and every gradient agree to fp32 summation-order noise (1e-6); the number of
dtype-conversion ops per step drops from one or two per parameter to a
handful."""

from __future__ import annotations

import copy

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

from helpers import rel_l2
from mednext_accel_amd import mednext_base, mednext_v2_base
from mednext_accel_amd.step import make_training_step

pytestmark = pytest.mark.gpu
DEV = "cuda"


class CountCasts(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.casts = 0

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        if func._schema.name == "aten::_to_copy":
            self.casts += 1
        return func(*args, **(kwargs or {}))


@pytest.mark.parametrize("family", ["v1", "v2"])
def test_precast_step_matches_per_operator_casts(family):
    print(f"[precast] {family}", flush=True)
    torch.manual_seed(5)
    build = mednext_base if family == "v1" else mednext_v2_base
    model = build(in_channels=1, out_channels=3, deep_supervision=True).to(DEV).train()
    plain = copy.deepcopy(model)
    n_params = len(model.__dict__["_mednext_precast_params"])
    assert n_params > 100
    plain.__dict__["_mednext_precast_params"] = []
    losses, casts = [], []
    for m in (model, plain):
        step = make_training_step(m, size=64, device=DEV)
        step.optimizer.zero_grad(set_to_none=True)
        with CountCasts() as counter:
            with torch.autocast(DEV, dtype=torch.bfloat16):
                loss = step.loss(m(step.sample))
            loss.backward()
        losses.append(float(loss.detach()))
        casts.append(counter.casts)
    print(f"  loss {losses[0]:.7f} / {losses[1]:.7f}, casts {casts[0]} / {casts[1]}", flush=True)
    assert abs(losses[0] - losses[1]) <= 1e-6 * abs(losses[1])
    assert casts[1] - casts[0] >= n_params
    for (name, p), q in zip(model.named_parameters(), plain.parameters(), strict=True):
        assert (p.grad is None) == (q.grad is None), name
        if p.grad is not None:
            assert rel_l2(p.grad.float(), q.grad.float()) <= 1e-6, name
    torch.cuda.empty_cache()
