"""MedNeXt v2 on the CPU: configuration schema, published parameter counts,
topology, shapes, deep supervision, checkpointing equivalence, adaptive
installation and the optimization report (mirrors the reference's
tests/models/test_config_v2.py, test_blocks_v2.py and test_mednext_v2.py)."""

from __future__ import annotations

import copy
from dataclasses import replace
from types import SimpleNamespace

import pytest
import torch
from torch.nn import functional as F

import mednext_accel_amd as m
from mednext_accel_amd import (
    AdaptiveDepthwise3d,
    AdaptiveGlobalResponseNorm3d,
    AdaptivePointwise3d,
    CheckpointConfig,
    EvalModeGELU,
    GlobalResponseNorm3d,
    MedNeXtV2,
    MedNeXtV2Block,
    MedNeXtV2Config,
    MedNeXtV2DownBlock,
    MedNeXtV2UpBlock,
    get_mednext_v2_config,
)
from mednext_accel_amd import mednext_v2 as v2


@pytest.fixture(scope="module", autouse=True)
def one_thread():
    previous = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(previous)


def small_config(*, deep_supervision=False):
    return replace(
        get_mednext_v2_config("base", in_channels=1, out_channels=3),
        base_channels=2,
        block_counts=(1,) * 9,
        expansion_ratios=(2,) * 9,
        downsample_expansion_ratios=(2,) * 4,
        upsample_expansion_ratios=(2,) * 4,
        deep_supervision=deep_supervision,
    )


VALID = dict(
    variant="base", in_channels=1, out_channels=3, base_channels=32, kernel_size=3,
    block_counts=(3,) * 9, expansion_ratios=(3,) * 9,
    downsample_expansion_ratios=(4,) * 4, upsample_expansion_ratios=(4,) * 4,
)


# --------------------------------------------------------------------- config


@pytest.mark.parametrize("variant,width", [("base", 32), ("wide", 64), ("WIDE", 64)])
def test_published_configuration(variant, width):
    cfg = get_mednext_v2_config(variant, in_channels=1, out_channels=3)
    assert cfg.base_channels == width and cfg.kernel_size == 3
    assert cfg.block_counts == (3, 4, 8, 8, 8, 8, 8, 4, 3)
    assert cfg.expansion_ratios == (3, 4, 8, 8, 8, 8, 8, 4, 3)
    assert cfg.downsample_expansion_ratios == (4, 8, 8, 8)
    assert cfg.upsample_expansion_ratios == (8, 8, 4, 3)


def test_yaml_lists_become_tuples():
    cfg = MedNeXtV2Config(**{**VALID, "block_counts": [3] * 9, "upsample_expansion_ratios": [4] * 4})
    assert isinstance(cfg.block_counts, tuple) and isinstance(cfg.upsample_expansion_ratios, tuple)


@pytest.mark.parametrize(
    "change",
    [{"in_channels": 0}, {"out_channels": 0}, {"base_channels": 0}, {"block_counts": (3,) * 8},
     {"expansion_ratios": (3,) * 8}, {"downsample_expansion_ratios": (4,) * 3},
     {"upsample_expansion_ratios": (4,) * 3}, {"variant": "large"}],
)
def test_rejects_invalid_schema(change):
    with pytest.raises(ValueError):
        MedNeXtV2Config(**{**VALID, **change})


@pytest.mark.parametrize("field,length", [("block_counts", 9), ("expansion_ratios", 9),
                                          ("downsample_expansion_ratios", 4), ("upsample_expansion_ratios", 4)])
@pytest.mark.parametrize("bad", [0, -1, 1.5, True, False, "2"])
def test_rejects_non_positive_integer_entries(field, length, bad):
    entries = [2] * length
    entries[length // 2] = bad
    with pytest.raises(ValueError, match=field):
        MedNeXtV2Config(**{**VALID, field: entries})


def test_rejects_unknown_variant_and_other_kernels():
    with pytest.raises(ValueError, match="variant"):
        get_mednext_v2_config("large", in_channels=1, out_channels=3)
    with pytest.raises(ValueError, match="kernel_size.*3"):
        replace(small_config(), kernel_size=5)


# --------------------------------------------------------------------- blocks


def test_block_order_and_parameters():
    block = MedNeXtV2Block(in_channels=4, out_channels=4, expansion_ratio=3)
    assert block.depthwise.groups == 4 and block.depthwise.kernel_size == (3, 3, 3)
    assert block.depthwise.padding == (1, 1, 1)
    assert block.expand.out_channels == 12 and block.project.in_channels == 12
    assert isinstance(block.activation, EvalModeGELU) and block.activation.approximate_eval is False
    assert isinstance(block.grn, GlobalResponseNorm3d)
    assert [n for n, _ in block.named_children()] == ["depthwise", "norm", "expand", "activation", "grn", "project"]
    assert block(torch.randn(2, 4, 9, 11, 13)).shape == (2, 4, 9, 11, 13)


def test_resampling_shapes_and_right_edge_padding():
    x = torch.randn(2, 4, 9, 11, 13)
    down = MedNeXtV2DownBlock(in_channels=4, out_channels=8, expansion_ratio=4)
    y = down(x)
    assert y.shape == (2, 8, 5, 6, 7)
    up = MedNeXtV2UpBlock(in_channels=8, out_channels=4, expansion_ratio=8).eval()
    with torch.no_grad():
        z = up(y)
        inner = MedNeXtV2Block.forward(up, y) + up.residual(y)
    assert z.shape == (2, 4, 10, 12, 14)
    torch.testing.assert_close(z[..., :-1, :-1, :-1], inner)  # padding sits at the end
    assert z[..., -1, :, :].abs().max() == 0 and z[..., :, :, -1].abs().max() == 0


@pytest.mark.parametrize(
    "factory,kwargs",
    [(MedNeXtV2Block, dict(in_channels=4, out_channels=4, expansion_ratio=3)),
     (MedNeXtV2DownBlock, dict(in_channels=4, out_channels=8, expansion_ratio=4)),
     (MedNeXtV2UpBlock, dict(in_channels=8, out_channels=4, expansion_ratio=8))],
)
def test_expansion_checkpoint_is_exact(factory, kwargs):
    torch.manual_seed(42)
    ref = factory(**kwargs).double().train()
    for p in ref.grn.parameters():
        torch.nn.init.normal_(p)
    ckpt = copy.deepcopy(ref)
    ckpt.checkpoint_expansion = True
    a = torch.randn(2, kwargs["in_channels"], 5, 7, 9, dtype=torch.double, requires_grad=True)
    b = a.detach().clone().requires_grad_()
    ya, yb = ref(a), ckpt(b)
    ya.square().mean().backward()
    yb.square().mean().backward()
    torch.testing.assert_close(yb, ya, rtol=0, atol=0)
    torch.testing.assert_close(b.grad, a.grad, rtol=0, atol=0)
    for p, q in zip(ref.parameters(), ckpt.parameters(), strict=True):
        torch.testing.assert_close(q.grad, p.grad, rtol=0, atol=0)


# ---------------------------------------------------------------------- model


@pytest.mark.parametrize("variant,count", [("base", 61_969_507), ("wide", 246_536_387)])
def test_published_parameter_counts(variant, count):
    with torch.device("meta"):
        model = getattr(m, f"mednext_v2_{variant}")(in_channels=1, out_channels=3, optimization="reference")
    assert sum(p.numel() for p in model.parameters()) == count


def test_stage_depths_and_ratios():
    with torch.device("meta"):
        model = m.mednext_v2_base(in_channels=1, out_channels=3)
    assert [len(s) for s in model.encoder_stages] == [3, 4, 8, 8]
    assert len(model.bottleneck) == 8
    assert [len(s) for s in model.decoder_stages] == [8, 8, 4, 3]
    for stage, ratio in zip([*model.encoder_stages, model.bottleneck, *model.decoder_stages],
                            [3, 4, 8, 8, 8, 8, 8, 4, 3], strict=True):
        for block in stage:
            assert type(block) is MedNeXtV2Block
            assert block.expand.out_channels == block.expand.in_channels * ratio
    for blocks, kind, ratios in ((model.downsamples, MedNeXtV2DownBlock, [4, 8, 8, 8]),
                                 (model.upsamples, MedNeXtV2UpBlock, [8, 8, 4, 3])):
        for block, ratio in zip(blocks, ratios, strict=True):
            assert type(block) is kind and block.expand.out_channels == block.expand.in_channels * ratio


@pytest.mark.parametrize("shape", [(17, 19, 21), (16, 17, 32), (1, 1, 17)])
def test_any_extent_round_trips(shape):
    model = MedNeXtV2(small_config()).eval()
    with torch.no_grad():
        assert model(torch.randn(1, 1, *shape)).shape == (1, 3, *shape)


@pytest.mark.parametrize("training", [True, False])
def test_batch_one_single_voxel_bottleneck_is_rejected(training):
    model = MedNeXtV2(small_config()).train(training)
    with pytest.raises(ValueError, match="GroupNorm.*batch"):
        model(torch.randn(1, 1, 16, 16, 16))
    assert model(torch.randn(2, 1, 16, 16, 16)).shape == (2, 3, 16, 16, 16)


def test_reconcile_spatial_crops_and_pads_right_edges():
    sample = torch.arange(24.0).reshape(1, 1, 2, 3, 4).requires_grad_()
    out = v2._reconcile_spatial(sample, (3, 2, 5))
    want = torch.zeros(1, 1, 3, 2, 5)
    want[..., :2, :, :4] = sample.detach()[..., :2, :]
    torch.testing.assert_close(out, want)
    out.sum().backward()
    grad = torch.zeros_like(sample)
    grad[..., :2, :] = 1
    torch.testing.assert_close(sample.grad, grad)


@pytest.mark.parametrize("fmt", ["tuple", "list", "stacked"])
def test_deep_supervision_head_order(fmt):
    model = MedNeXtV2(small_config(deep_supervision=True), deep_supervision_output=fmt).train()
    for head, value in zip([model.head, *model.deep_supervision_heads], [0, 4, 3, 2, 1], strict=True):
        torch.nn.init.zeros_(head.conv.weight)
        torch.nn.init.constant_(head.conv.bias, value)
    sample = torch.randn(1, 1, 17, 19, 21)
    out = model(sample)
    if fmt == "stacked":
        assert out.shape == (1, 5, 3, 17, 19, 21)
        outs = out.unbind(1)
    else:
        assert isinstance(out, tuple if fmt == "tuple" else list)
        assert [tuple(o.shape) for o in out] == [(1, 3, 17, 19, 21), (1, 3, 9, 10, 11), (1, 3, 5, 5, 6),
                                                  (1, 3, 3, 3, 3), (1, 3, 2, 2, 2)]
        outs = out
    for value, o in enumerate(outs):
        torch.testing.assert_close(o, torch.full_like(o, value))
    with torch.no_grad():
        assert model.eval()(sample).shape == (1, 3, 17, 19, 21)


def test_stacked_outputs_resize_native_logits():
    model = MedNeXtV2(small_config(deep_supervision=True)).train()
    sample = torch.randn(1, 1, 16, 17, 32)
    with torch.no_grad():
        native = model(sample)
        model.deep_supervision_output = "stacked"
        stacked = model(sample)
    torch.testing.assert_close(stacked, torch.stack([F.interpolate(o, size=(16, 17, 32)) for o in native], 1))


def test_invalid_deep_supervision_output():
    with pytest.raises(ValueError, match="deep_supervision_output"):
        MedNeXtV2(small_config(), deep_supervision_output="tensor")


@pytest.mark.parametrize("style", ["expansion", "block"])
def test_checkpointing_preserves_state_and_gradients(style):
    torch.manual_seed(42)
    ref = MedNeXtV2(small_config(deep_supervision=True)).train()
    ckpt = MedNeXtV2(small_config(deep_supervision=True), checkpointing=CheckpointConfig(style=style, stages=(0, 1))).train()
    ckpt.load_state_dict(ref.state_dict(), strict=True)
    a = torch.randn(1, 1, 17, 19, 21, requires_grad=True)
    b = a.detach().clone().requires_grad_()
    ya, yb = ref(a), ckpt(b)
    sum(o.square().mean() for o in ya).backward()
    sum(o.square().mean() for o in yb).backward()
    torch.testing.assert_close(yb, ya)
    torch.testing.assert_close(b.grad, a.grad)
    assert ckpt.state_dict().keys() == ref.state_dict().keys()
    for name, p in ref.named_parameters():
        torch.testing.assert_close(ckpt.get_parameter(name).grad, p.grad, msg=name)


def test_custom_resampling_ratios():
    model = MedNeXtV2(replace(small_config(), downsample_expansion_ratios=(1, 2, 3, 4),
                              upsample_expansion_ratios=(4, 3, 2, 1)))
    assert [b.expand.out_channels // b.expand.in_channels for b in model.downsamples] == [1, 2, 3, 4]
    assert [b.expand.out_channels // b.expand.in_channels for b in model.upsamples] == [4, 3, 2, 1]


@pytest.mark.parametrize("variant", ["base", "wide"])
def test_factory_installs_adaptive_families_and_keeps_state(monkeypatch, variant):
    monkeypatch.setattr(v2, "get_mednext_v2_config", lambda *a, **kw: small_config())
    factory = getattr(m, f"mednext_v2_{variant}")
    ref = factory(in_channels=1, out_channels=3, optimization="reference")
    auto = factory(in_channels=1, out_channels=3, optimization="auto")
    assert isinstance(auto.stem, AdaptivePointwise3d)
    assert isinstance(auto.encoder_stages[0][0].depthwise, AdaptiveDepthwise3d)
    assert isinstance(auto.encoder_stages[0][0].grn, AdaptiveGlobalResponseNorm3d)
    assert auto.state_dict().keys() == ref.state_dict().keys()
    auto.load_state_dict(ref.state_dict(), strict=True)
    assert auto.stem.model_context.family == "mednext_v2"
    adaptive = (AdaptivePointwise3d, AdaptiveDepthwise3d, AdaptiveGlobalResponseNorm3d)
    assert not any(isinstance(mod, adaptive) for mod in ref.modules())
    x = torch.randn(2, 1, 16, 17, 18, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    want, got = ref(x), auto(y)
    torch.testing.assert_close(got, want)
    want.square().mean().backward()
    got.square().mean().backward()
    torch.testing.assert_close(y.grad, x.grad)
    for name, p in ref.named_parameters():
        torch.testing.assert_close(auto.get_parameter(name).grad, p.grad)
    params = dict(ref.named_parameters())
    v2._configure_optimization(ref, "auto")
    assert all(ref.get_parameter(n) is p for n, p in params.items())


@pytest.mark.parametrize("source", ["torch", "conservative", "autotune"])
def test_removed_optimization_sources(monkeypatch, source):
    monkeypatch.setattr(v2, "get_mednext_v2_config", lambda *a, **kw: small_config())
    with pytest.raises(ValueError, match="was removed"):
        m.mednext_v2_base(in_channels=1, out_channels=3, optimization=source)


def test_report_resolves_each_operator_at_its_input_resolution(monkeypatch):
    model = v2._configure_optimization(MedNeXtV2(small_config(deep_supervision=True)), "auto")
    seen = {}

    def record(role):
        def hook(module, args):
            seen[role] = tuple(args[0].shape[2:])
        return hook

    adaptive = (AdaptiveDepthwise3d, AdaptivePointwise3d, AdaptiveGlobalResponseNorm3d)
    handles = [mod.register_forward_pre_hook(record(r)) for r, mod in model.named_modules() if isinstance(mod, adaptive)]
    with torch.no_grad():
        model(torch.randn(1, 1, 17, 19, 21))
    for h in handles:
        h.remove()
    resolved = {}
    resolver = model._optimization_resolver
    original = resolver.resolve

    def resolve(descriptor, context, phase):
        resolved[descriptor.role] = context.spatial_shape
        return original(descriptor, context, phase)

    monkeypatch.setattr(resolver, "resolve", resolve)
    report = model.explain_optimization(input_shape=(1, 1, 17, 19, 21), dtype="bfloat16", device="cpu")
    for role, shape in seen.items():
        assert resolved[role] == shape, role
    grn = [d for d in report.decisions if d.descriptor.family == "global_response_norm3d"]
    assert len(grn) == 17 and all(d.phase == "training" for d in grn)


def _fake_amd_gpu(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda *a: (9, 5))
    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    monkeypatch.setattr(
        torch.cuda, "get_device_properties",
        lambda *a: SimpleNamespace(total_memory=288 * 2**30, gcnArchName="gfx950:sramecc+:xnack-"),
    )
    from mednext_accel_amd import adaptive

    adaptive._cached_device.cache_clear()


def test_bundled_policy_selects_hip_grn_for_training_and_reference_for_eval(monkeypatch):
    monkeypatch.setattr(v2, "get_mednext_v2_config", lambda *a, **kw: small_config())
    model = m.mednext_v2_base(in_channels=1, out_channels=3)
    _fake_amd_gpu(monkeypatch)
    try:
        report = model.explain_optimization(input_shape=(2, 1, 32, 32, 32), dtype="bfloat16", device="cuda")
        grn = [d for d in report.decisions if d.descriptor.family == "global_response_norm3d"]
        assert len(grn) == 17 and all(d.implementation == "hip_fused_grn" for d in grn)
        fp32 = model.explain_optimization(input_shape=(2, 1, 32, 32, 32), dtype="float32", device="cuda")
        grn32 = [d for d in fp32.decisions if d.descriptor.family == "global_response_norm3d"]
        assert all(d.implementation == "reference" for d in grn32)  # half-precision contract
        evals = model.eval().explain_optimization(input_shape=(2, 1, 32, 32, 32), dtype="bfloat16", device="cuda")
        grn_eval = [d for d in evals.decisions if d.descriptor.family == "global_response_norm3d"]
        assert len(grn_eval) == 17 and all(d.implementation == "reference" for d in grn_eval)
    finally:
        from mednext_accel_amd import adaptive

        adaptive._cached_device.cache_clear()


def test_reference_report_and_input_rank():
    model = MedNeXtV2(small_config())
    report = model.explain_optimization(input_shape=(2, 1, 32, 32, 32), dtype="float32", device="cpu")
    assert report.decisions and all(d.implementation == "reference" for d in report.decisions)
    assert len([d for d in report.decisions if d.descriptor.family == "global_response_norm3d"]) == 17
    with pytest.raises(ValueError, match="rank 5"):
        model.explain_optimization(input_shape=(1, 1, 32, 32), dtype="float32", device="cpu")
