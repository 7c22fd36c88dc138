"""The per-forward parameter pre-cast (precast.py) on the CPU: the batched cast
is the per-tensor casts (values, gradients, unused outputs), and a model with
the pre-cast installed trains exactly like one without."""

from __future__ import annotations

import copy
from dataclasses import replace

import torch
from torch import nn
from torch.utils.checkpoint import checkpoint

from mednext_accel_amd import MedNeXtV1
from mednext_accel_amd.config import get_mednext_v1_config
from mednext_accel_amd.mednext_v1 import configure_optimization
from mednext_accel_amd.precast import _CastMany, cast_param, precast_parameters


def test_cast_many_is_the_per_tensor_casts():
    gen = torch.Generator().manual_seed(3)
    params = [torch.randn(shape, generator=gen, requires_grad=True) for shape in ((3, 4), (5,), (2, 1, 3, 3, 3))]
    outs = _CastMany.apply(torch.bfloat16, object(), *params)
    for o, p in zip(outs, params, strict=True):
        assert o.dtype == torch.bfloat16 and o.shape == p.shape
        assert torch.equal(o, p.detach().to(torch.bfloat16))
    grads = [torch.randn(o.shape, generator=gen).bfloat16() for o in outs]
    torch.autograd.backward([outs[0], outs[2]], [grads[0], grads[2]])  # the second copy is unused
    assert torch.equal(params[0].grad, grads[0].float())
    assert params[1].grad is None
    assert torch.equal(params[2].grad, grads[2].float())


def test_cast_param_outside_a_forward_is_a_plain_cast():
    p = torch.randn(4, 3)
    assert torch.equal(cast_param(p, torch.bfloat16), p.to(torch.bfloat16))
    assert cast_param(p, torch.float32) is p


def test_model_with_precast_trains_like_one_without():
    cfg = replace(get_mednext_v1_config("base", in_channels=1, out_channels=2, kernel_size=3, deep_supervision=False),
                  base_channels=4, block_counts=(1,) * 9)
    torch.manual_seed(0)
    model = configure_optimization(MedNeXtV1(cfg), "auto").train()
    assert len(precast_parameters(model)) == len(model.__dict__["_mednext_precast_params"]) > 0
    plain = copy.deepcopy(model)
    plain.__dict__["_mednext_precast_params"] = []  # hooks stay, but cast nothing
    x = torch.randn(1, 1, 32, 32, 32)
    for m in (model, plain):
        with torch.autocast("cpu", dtype=torch.bfloat16):
            m(x).float().square().mean().backward()
    for (name, p), q in zip(model.named_parameters(), plain.parameters(), strict=True):
        assert (p.grad is None) == (q.grad is None), name
        if p.grad is not None:
            assert torch.equal(p.grad, q.grad), name


def test_copies_start_on_16_byte_boundaries():
    params = [torch.randn(n, requires_grad=True) for n in (3, 8, 13, 1, 27)]
    outs = _CastMany.apply(torch.bfloat16, object(), *params)
    base = outs[0].data_ptr()
    for o, p in zip(outs, params, strict=True):
        assert (o.data_ptr() - base) % 16 == 0
        assert torch.equal(o, p.detach().bfloat16())
    sum(o.float().sum() for o in outs).backward()
    for p in params:
        assert torch.equal(p.grad, torch.ones_like(p))


def test_failed_forward_leaves_no_stale_copies():
    """A forward that raises (e.g. a caught out-of-memory error) must not leave
    its bf16 copies active: the next forward (here an evaluation pass without
    autocast) reads the fp32 parameters."""
    from mednext_accel_amd import precast

    cfg = replace(get_mednext_v1_config("base", in_channels=1, out_channels=2, kernel_size=3, deep_supervision=False),
                  base_channels=4, block_counts=(1,) * 9)
    torch.manual_seed(0)
    model = configure_optimization(MedNeXtV1(cfg), "auto").train()
    reference = copy.deepcopy(model)
    boom = model.stem.register_forward_hook(lambda *a: (_ for _ in ()).throw(RuntimeError("boom")))
    with torch.autocast("cpu", dtype=torch.bfloat16):
        try:
            model(torch.randn(1, 1, 32, 32, 32))
        except RuntimeError as error:
            assert "boom" in str(error)
    boom.remove()
    assert precast._ACTIVE is None
    model.eval()
    reference.eval()
    x = torch.randn(1, 1, 32, 32, 32)
    with torch.no_grad():
        assert torch.equal(model(x), reference(x))


class _Checkpointed(nn.Module):
    """A checkpointed branch that fetches its weight through cast_param, as the
    fused expansions do."""

    def __init__(self) -> None:
        super().__init__()
        self.w = nn.Parameter(torch.randn(16, 16))

    def forward(self, x):
        return checkpoint(lambda t: torch.tanh(t @ cast_param(self.w, torch.bfloat16)), x, use_reentrant=False)


def test_copies_serve_the_backward_recompute_then_drop():
    """The pre-cast copies outlive the forward so that a checkpointed branch
    recomputed in the backward reuses them (no second cast of its weights);
    the backward through the copies drops them before any optimizer step, and
    a copy whose parameter changed in place is never served. Gradients match a
    plain per-use cast."""
    from mednext_accel_amd import precast

    torch.manual_seed(1)
    model, plain = _Checkpointed(), _Checkpointed()
    plain.load_state_dict(model.state_dict())
    model.__dict__["_mednext_precast_params"] = [model.w]
    model.__dict__["_mednext_precast_dtype"] = torch.bfloat16
    model.register_forward_pre_hook(precast._precast_before)
    model.register_forward_hook(precast._precast_after, always_call=True)
    x = torch.randn(4, 16)
    served = []
    real = precast._copy_of

    def spy(p, dtype):
        t = real(p, dtype)
        served.append(t is not None)
        return t

    precast._copy_of = spy
    try:
        with torch.autocast("cpu", dtype=torch.bfloat16):
            out = model(x)
        assert precast._ACTIVE is not None  # kept for the backward
        out.float().sum().backward()
    finally:
        precast._copy_of = real
    assert served == [True, True]  # the forward and the recompute both got the copy
    assert precast._ACTIVE is None  # dropped by the backward through the copies
    with torch.autocast("cpu", dtype=torch.bfloat16):
        plain(x).float().sum().backward()
    assert torch.equal(model.w.grad, plain.w.grad)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        model(x)
    copy_now = cast_param(model.w, torch.bfloat16)
    assert copy_now is precast._ACTIVE[id(model.w)][0]
    with torch.no_grad():
        model.w.add_(1.0)
    fresh = cast_param(model.w, torch.bfloat16)
    assert fresh is not copy_now and torch.equal(fresh, model.w.detach().bfloat16())
    precast._drop()
