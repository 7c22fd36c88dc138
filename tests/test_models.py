"""MedNeXt v1 model harness on the CPU: architecture KATs, output formats,
checkpointing equivalence, state-dict compatibility (mirrors the reference's
tests/models/test_mednext_v1.py)."""

from __future__ import annotations

import pytest
import torch

from mednext_accel_amd import (
    AdaptiveDepthwise3d,
    AdaptiveGroupNorm3d,
    AdaptivePointwise3d,
    CheckpointConfig,
    MedNeXtV1,
    get_mednext_v1_config,
    mednext_base,
    mednext_large,
    mednext_medium,
    mednext_small,
)
from mednext_accel_amd.mednext_v1 import checkpoint_name, spatial_shape_for_role


@pytest.mark.parametrize("factory", [mednext_small, mednext_base, mednext_medium, mednext_large])
def test_factories_build_declared_variant(factory):
    model = factory(in_channels=1, out_channels=3, base_channels=2)
    assert isinstance(model, MedNeXtV1)
    assert model.config.variant in factory.__name__


def test_base_parameter_count_matches_published():
    """KAT: MedNeXt-B (1 in, 3 out, k3, deep supervision) has 10,529,231 parameters
    (reference tests/models/test_mednext_v1.py:52-55)."""
    model = mednext_base(in_channels=1, out_channels=3, deep_supervision=True)
    assert sum(p.numel() for p in model.parameters()) == 10_529_231


def test_large_k5_parameter_count():
    """MedNeXt-L at k=5 with deep supervision: 62,995,823 parameters, derived by
    counting: each k=5 depthwise weight has 125 taps vs 27 at k=3."""
    model = mednext_large(in_channels=1, out_channels=3, kernel_size=5, deep_supervision=True)
    k3 = mednext_large(in_channels=1, out_channels=3, kernel_size=3, deep_supervision=True)
    n5 = sum(p.numel() for p in model.parameters())
    n3 = sum(p.numel() for p in k3.parameters())
    assert n5 == 62_995_823
    depthwise_channels = sum(m.in_channels for m in model.modules() if isinstance(m, AdaptiveDepthwise3d))
    assert n5 - n3 == depthwise_channels * (125 - 27)


@pytest.mark.parametrize("spatial_dims", [2, 3])
def test_small_eval_returns_primary_logits(spatial_dims):
    model = mednext_small(
        in_channels=1, out_channels=3, spatial_dims=spatial_dims, base_channels=2, deep_supervision=True
    ).eval()
    with torch.no_grad():
        out = model(torch.randn(1, 1, *([32] * spatial_dims)))
    assert isinstance(out, torch.Tensor) and out.shape == (1, 3, *([32] * spatial_dims))


@pytest.mark.parametrize("fmt", ["tuple", "list", "stacked"])
def test_deep_supervision_output_formats(fmt):
    model = mednext_small(
        in_channels=1, out_channels=3, base_channels=2, deep_supervision=True, deep_supervision_output=fmt
    ).train()
    out = model(torch.randn(1, 1, 32, 32, 32))
    if fmt == "stacked":
        assert out.shape == (1, 5, 3, 32, 32, 32)
    else:
        assert isinstance(out, tuple if fmt == "tuple" else list)
        assert [tuple(o.shape) for o in out] == [(1, 3, s, s, s) for s in (32, 16, 8, 4, 2)]


def test_invalid_deep_supervision_output_is_rejected():
    with pytest.raises(ValueError, match="deep_supervision_output"):
        mednext_small(in_channels=1, out_channels=3, deep_supervision_output="tensor")


@pytest.mark.parametrize("style", ["expansion", "block"])
def test_checkpointing_preserves_outputs_and_gradients(style):
    torch.manual_seed(42)
    plain = mednext_small(in_channels=1, out_channels=2, base_channels=2).train()
    ckpt = mednext_small(
        in_channels=1, out_channels=2, base_channels=2, checkpointing=CheckpointConfig(style=style, stages=(0, 1))
    ).train()
    ckpt.load_state_dict(plain.state_dict(), strict=True)
    x = torch.randn(1, 1, 32, 32, 32, requires_grad=True)
    x2 = x.detach().clone().requires_grad_(True)
    a, b = plain(x), ckpt(x2)
    a.square().mean().backward()
    b.square().mean().backward()
    torch.testing.assert_close(b, a)
    torch.testing.assert_close(x2.grad, x.grad)
    for p, q in zip(plain.parameters(), ckpt.parameters(), strict=True):
        torch.testing.assert_close(q.grad, p.grad)


def test_optimization_keeps_state_dict_keys_and_parameters():
    torch.manual_seed(0)
    ref = mednext_base(in_channels=1, out_channels=3, deep_supervision=True, optimization="reference")
    opt = mednext_base(in_channels=1, out_channels=3, deep_supervision=True, optimization="auto")
    assert list(ref.state_dict()) == list(opt.state_dict())
    opt.load_state_dict(ref.state_dict(), strict=True)
    kinds = {type(m) for m in opt.modules()}
    assert {AdaptiveDepthwise3d, AdaptivePointwise3d, AdaptiveGroupNorm3d} <= kinds
    keys = set(ref.state_dict())
    for key in (
        "stem.weight",
        "encoder_stages.0.0.depthwise.weight",
        "encoder_stages.0.0.norm.bias",
        "encoder_stages.3.1.project.weight",
        "downsamples.0.residual.weight",
        "bottleneck.1.expand.bias",
        "upsamples.3.depthwise.weight",
        "decoder_stages.3.1.norm.weight",
        "head.conv.weight",
        "deep_supervision_heads.3.conv.bias",
    ):
        assert key in keys
    assert len(keys) == sum(1 for _ in ref.parameters())  # no buffers: every entry is a Parameter


def test_cpu_model_with_wrappers_matches_reference_model():
    """On the CPU every wrapper takes the native route: identical numbers."""
    torch.manual_seed(5)
    ref = mednext_small(in_channels=1, out_channels=2, base_channels=4, optimization="reference").double().train()
    opt = mednext_small(in_channels=1, out_channels=2, base_channels=4).double().train()
    opt.load_state_dict(ref.state_dict())
    x = torch.randn(1, 1, 32, 32, 32, dtype=torch.double)
    torch.testing.assert_close(opt(x), ref(x))


def test_config_and_checkpoint_validation():
    with pytest.raises(ValueError):
        get_mednext_v1_config("huge", in_channels=1, out_channels=1)
    with pytest.raises(ValueError):
        get_mednext_v1_config("base", in_channels=1, out_channels=1, kernel_size=4)
    with pytest.raises(ValueError):
        get_mednext_v1_config("base", in_channels=1, out_channels=1, compatibility="other")
    assert get_mednext_v1_config("base", in_channels=1, out_channels=1).downsample_expansion_ratios == (3, 4, 4, 4)
    assert get_mednext_v1_config(
        "base", in_channels=1, out_channels=1, compatibility="monai"
    ).downsample_expansion_ratios == (2, 3, 4, 4)
    for bad in ((), (5,), (0, 0), (1.0,)):
        with pytest.raises(ValueError):
            CheckpointConfig(stages=bad)
    with pytest.raises(ValueError):
        CheckpointConfig(style="layer")
    assert CheckpointConfig(stages=(2, 0)).stages == (0, 2)
    assert checkpoint_name(None) == "none"
    assert checkpoint_name(CheckpointConfig()) == "all-expansion"
    assert checkpoint_name(CheckpointConfig(style="block")) == "whole-block"
    assert checkpoint_name(CheckpointConfig(stages=(0, 1))) == "expansion:0,1"
    with pytest.raises(ValueError):
        mednext_small(in_channels=1, out_channels=1, optimization="autotune")


def test_spatial_shape_for_role():
    s = (128, 128, 128)
    assert spatial_shape_for_role("stem", s) == s
    assert spatial_shape_for_role("encoder_stages.2.0.depthwise", s) == (32, 32, 32)
    assert spatial_shape_for_role("downsamples.0.depthwise", s) == s
    assert spatial_shape_for_role("downsamples.0.expand", s) == (64, 64, 64)
    assert spatial_shape_for_role("bottleneck.0.norm", s) == (8, 8, 8)
    assert spatial_shape_for_role("upsamples.0.depthwise", s) == (8, 8, 8)
    assert spatial_shape_for_role("upsamples.0.expand", s) == (15, 15, 15)
    assert spatial_shape_for_role("decoder_stages.3.0.project", s) == s


def test_explain_optimization_on_cpu_is_reference():
    model = mednext_small(in_channels=1, out_channels=2, base_channels=4)
    report = model.explain_optimization(input_shape=(1, 1, 64, 64, 64), dtype=torch.bfloat16, device="cpu")
    assert report.policies == ("reference",)
    assert report.decisions and all(d.implementation == "reference" for d in report.decisions)
    with pytest.raises(ValueError):
        model.explain_optimization(input_shape=(1, 64, 64, 64), dtype="float32", device="cpu")


def test_report_helpers_and_json_form():
    import json

    model = mednext_small(in_channels=1, out_channels=2, base_channels=4)
    report = model.explain_optimization(input_shape=(1, 1, 32, 32, 32), dtype=torch.bfloat16, device="cpu")
    counts = report.implementations()
    assert counts == {"reference": len(report.decisions)}
    assert report.custom() == ()
    data = json.loads(json.dumps(report.to_primitive()))
    assert data["policies"] == ["reference"] and len(data["decisions"]) == len(report.decisions)
    assert data["context"]["spatial_shape"] == [32, 32, 32]


def test_load_policy_sources(tmp_path):
    import json

    import yaml

    from mednext_accel_amd.optimization import load_bundled_policy, load_policy, policy_to_primitive

    bundled = load_bundled_policy("gfx950")
    assert load_policy(bundled) is bundled
    doc = policy_to_primitive(bundled)
    (tmp_path / "p.yaml").write_text(yaml.safe_dump(doc))
    (tmp_path / "p.json").write_text(json.dumps(doc))
    assert load_policy(tmp_path / "p.yaml") == bundled == load_policy(str(tmp_path / "p.json"))
    assert load_policy(doc) == bundled
    with pytest.raises(ValueError, match="suffix"):
        load_policy(tmp_path / "p.txt")
    with pytest.raises(ValueError, match="factory mode"):
        load_policy("auto")
