"""Selection hook on the CPU: wrapper installation, gfx950 policy decisions,
vendor layering, guards and the policy document schema (mirrors the
reference's tests/ops/test_adaptive.py and tests/optimization/*)."""

from __future__ import annotations

import copy
import warnings

import pytest
import torch
from torch import nn

from mednext_accel_amd import tiles
from mednext_accel_amd.adaptive import (
    AdaptiveDepthwise3d,
    AdaptiveGroupNorm3d,
    AdaptivePointwise3d,
    ModelOptimizationContext,
    _conv_descriptor,
    _norm_descriptor,
    execution_context_for_shape,
    install_adaptive_operators,
)
from mednext_accel_amd.optimization import (
    PolicyRegistry,
    PolicyResolver,
    load_bundled_policy,
    parse_policy,
    policy_to_primitive,
)

MC = ModelOptimizationContext("mednext_v1", "base", "none")
STAGES = [(32, 128), (64, 64), (128, 32), (256, 16), (512, 8)]


def ctx(spatial, *, dtype="bfloat16", arch="gfx950", sm=(9, 5), device="cuda", training=True, batch=1):
    return execution_context_for_shape(
        MC, batch_size=batch, spatial_shape=spatial, dtype=dtype, device_type=device, sm=sm,
        total_vram_bytes=288 * 2**30, training=training, arch=arch,
    )


def policy(rules, *, vendor="amd", arch=None, name="test"):
    target = {"vendor": vendor, **({"arch": arch} if arch else {})}
    return parse_policy({"version": 2, "kind": "mednext-accel-policy", "name": name, "target": target, "rules": rules})


def test_installation_preserves_parameters_and_state_dict_keys():
    model = nn.Sequential(nn.Conv3d(32, 32, 3, padding=1, groups=32), nn.GroupNorm(32, 32), nn.Conv3d(32, 64, 1))
    params, keys = tuple(model.parameters()), tuple(model.state_dict())
    count = install_adaptive_operators(model, resolver=PolicyRegistry().resolver(), model_context=MC)
    assert count == 3
    assert tuple(model.parameters()) == params and tuple(model.state_dict()) == keys
    assert isinstance(model[0], AdaptiveDepthwise3d)
    assert isinstance(model[1], AdaptiveGroupNorm3d)
    assert isinstance(model[2], AdaptivePointwise3d)


def test_ineligible_modules_are_left_alone():
    model = nn.Sequential(
        nn.Conv3d(4, 4, 3, padding=0, groups=4),  # not "same" padding
        nn.Conv3d(4, 8, 3, padding=1),  # dense 3x3x3
        nn.GroupNorm(2, 4),  # groups != channels
        nn.Conv3d(4, 4, 2, padding=0, groups=4),  # even kernel
    )
    assert install_adaptive_operators(model, resolver=PolicyRegistry().resolver(), model_context=MC) == 0


def test_cpu_forward_backward_matches_native():
    torch.manual_seed(3)
    ref = nn.Sequential(nn.Conv3d(3, 3, 3, padding=1, groups=3), nn.GroupNorm(3, 3), nn.Conv3d(3, 7, 1)).double()
    cand = copy.deepcopy(ref)
    install_adaptive_operators(cand, resolver=PolicyRegistry().resolver(), model_context=MC)
    x = torch.randn(2, 3, 5, 6, 7, dtype=torch.double, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    a, b = ref(x), cand(y)
    torch.testing.assert_close(b, a)
    g = torch.randn_like(a)
    for got, want in zip(
        torch.autograd.grad(b, (y, *cand.parameters()), g), torch.autograd.grad(a, (x, *ref.parameters()), g), strict=True
    ):
        torch.testing.assert_close(got, want)


@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("bias", [True, False])
def test_per_sample_gemm_matches_convolution(batch, bias):
    torch.manual_seed(37)
    ref = nn.Conv3d(4, 7, 1, bias=bias).double()
    cand = AdaptivePointwise3d(copy.deepcopy(ref), PolicyRegistry().resolver(), MC)
    x = torch.randn(batch, 4, 3, 4, 5, dtype=torch.double, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    a, b = ref(x), cand._gemm(y)
    torch.testing.assert_close(b, a)
    g = torch.randn_like(a)
    for got, want in zip(
        torch.autograd.grad(b, (y, *cand.parameters()), g), torch.autograd.grad(a, (x, *ref.parameters()), g), strict=True
    ):
        torch.testing.assert_close(got, want)


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("channels,size", STAGES)
def test_gfx950_policy_selects_hip_depthwise_with_tile_recipes(channels, size, k):
    """The formula-driven gfx950 layer on its own: HIP everywhere at the stage
    shapes, with the tile recipe of ``tiles.depthwise_recipe``."""
    from mednext_accel_amd.optimization.policies import load_bundled_policy
    from mednext_accel_amd.optimization.policy_resolver import PolicyResolver

    resolver = PolicyResolver((load_bundled_policy("gfx950"),))
    conv = nn.Conv3d(channels, channels, k, padding=k // 2, groups=channels)
    desc = _conv_descriptor(conv, role="encoder_stages.0.0.depthwise")
    c = ctx((size,) * 3)
    for phase, impl, tile_phase in (
        ("forward", "hip_depthwise_fwd", "forward"),
        ("backward_input", "hip_depthwise_dx", "input_grad"),
        ("backward_weight", "hip_split_dw", "weight_grad"),
    ):
        d = resolver.resolve(desc, c, phase)
        assert d.implementation == impl and d.policy == "gfx950" and d.disposition == "custom"
        want = tiles.depthwise_recipe(1, channels, (size,) * 3, k, "bfloat16", tile_phase)
        assert [d.parameters["engine"], d.parameters["tile_w"], d.parameters["depth_chunk"]] == want


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("channels,size", STAGES)
def test_measured_policy_layer_matches_its_evidence(channels, size, k):
    """The bundled registry resolves the MedNeXt-Base 128^3 depthwise contexts
    through the measured exact-context layer, and each selected recipe is the
    fastest valid candidate recorded in that layer's evidence file."""
    import json

    from mednext_accel_amd.optimization.policies import POLICY_DIR

    evidence = json.loads((POLICY_DIR / "gfx950_base128_evidence.json").read_text())["measurements"]
    resolver = PolicyRegistry().resolver()
    conv = nn.Conv3d(channels, channels, k, padding=k // 2, groups=channels)
    desc = _conv_descriptor(conv, role="encoder_stages.0.0.depthwise")
    for phase in ("forward", "backward_input", "backward_weight"):
        d = resolver.resolve(desc, ctx((size,) * 3), phase)
        rows = [m for m in evidence if m["family"] == "depthwise_conv3d" and m["phase"] == phase
                and m["in_channels"] == channels and m["kernel_size"] == k and m["spatial_shape"] == [size] * 3
                and m["valid"]]
        best = min(rows, key=lambda m: m["candidate_ms"])
        assert d.policy == "gfx950-base-128-measured"
        assert d.implementation == best["implementation"]
        if best["parameters"]:
            assert d.parameters == best["parameters"]
        # Every HIP candidate beat native PyTorch at these shapes on MI355X.
        assert d.disposition == "custom"


def test_gfx950_policy_group_norm_and_pointwise():
    resolver = PolicyRegistry().resolver()
    gn = _norm_descriptor(nn.GroupNorm(32, 32), role="encoder_stages.0.0.norm")
    d = resolver.resolve(gn, ctx((128,) * 3), "training")
    assert d.implementation == "hip_group_norm"
    assert d.parameters["splits"] == tiles.group_norm_splits(1, 32, 128**3)
    pw = _conv_descriptor(nn.Conv3d(32, 64, 1), role="encoder_stages.0.0.expand")
    assert resolver.resolve(pw, ctx((128,) * 3), "training").implementation == "hip_pointwise_gemm"
    assert resolver.resolve(pw, ctx((128,) * 3, dtype="float32"), "training").implementation == "reference"


def test_fused_expansion_is_attached_without_touching_parameters():
    from mednext_accel_amd import MedNeXtBlock
    from mednext_accel_amd.adaptive import AdaptiveExpansion

    block = MedNeXtBlock(spatial_dims=3, in_channels=32, out_channels=32, expansion_ratio=2, kernel_size=3)
    params, keys = tuple(block.parameters()), tuple(block.state_dict())
    install_adaptive_operators(block, resolver=PolicyRegistry().resolver(), model_context=MC)
    fused = block.__dict__["fused_expansion"]
    assert isinstance(fused, AdaptiveExpansion) and "fused_expansion" not in dict(block.named_children())
    assert tuple(block.parameters()) == params and tuple(block.state_dict()) == keys
    d = PolicyRegistry().resolver().resolve(fused.descriptor, ctx((128,) * 3), "training")
    assert d.implementation == "hip_fused_expansion"
    assert PolicyRegistry().resolver().resolve(fused.descriptor, ctx((128,) * 3, dtype="float32"), "training").implementation == "reference"
    # On the CPU the block never takes the fused route.
    assert not fused.applies(torch.randn(1, 32, 8, 8, 8))
    copy.deepcopy(block)  # the plain attribute survives deep copies (checkpoint loaders use them)


def test_strided_and_transposed_depthwise_select_hip():
    resolver = PolicyRegistry().resolver()
    down = _conv_descriptor(nn.Conv3d(32, 32, 3, stride=2, padding=1, groups=32), role="downsamples.0.depthwise")
    up = _conv_descriptor(nn.ConvTranspose3d(64, 64, 3, stride=2, padding=1, groups=64), role="upsamples.0.depthwise")
    for desc, impl in ((down, "hip_depthwise_stride2"), (up, "hip_depthwise_transpose2")):
        for phase in ("forward", "backward_input", "backward_weight"):
            assert resolver.resolve(desc, ctx((64,) * 3), phase).implementation == impl
            assert resolver.resolve(desc, ctx((64,) * 3, training=False), phase).implementation == "reference"
    # Geometries the kernels do not take stay native.
    k7 = _conv_descriptor(nn.Conv3d(8, 8, 7, stride=2, padding=3, groups=8), role=None)
    pad0 = _conv_descriptor(nn.Conv3d(8, 8, 3, stride=2, padding=0, groups=8), role=None)
    for desc in (k7, pad0):
        assert resolver.resolve(desc, ctx((32,) * 3), "forward").implementation == "reference"


def test_context_guards():
    resolver = PolicyRegistry().resolver()
    desc = _conv_descriptor(nn.Conv3d(32, 32, 3, padding=1, groups=32), role=None)
    cpu = resolver.resolve(desc, ctx((32,) * 3, device="cpu", arch=None, sm=None), "backward_input")
    assert cpu.implementation == "reference" and cpu.guard_reason is not None
    # An NVIDIA context sees no bundled layer in this build.
    nv = resolver.resolve(desc, ctx((32,) * 3, arch=None, sm=(12, 0)), "backward_input")
    assert nv.implementation == "reference" and nv.rule == "fallback"
    # Inference is guarded (training-only implementations).
    inf = resolver.resolve(desc, ctx((32,) * 3, training=False), "backward_input")
    assert inf.implementation == "reference" and inf.guard_reason == "implementation requires training"
    # Another AMD arch: no exact layer.
    other = resolver.resolve(desc, ctx((32,) * 3, arch="gfx942"), "backward_input")
    assert other.implementation == "reference"


def test_mfma_override_needs_bf16_and_supported_plane():
    ext = policy(
        [{"id": "dw", "when": {"family": "depthwise_conv3d"},
          "use": {"backward_input": {"implementation": "hip_depthwise_dx",
                                     "parameters": {"engine": 1, "tile_w": 64, "depth_chunk": 8}}},
          "confidence": "extrapolated"}],
        arch="gfx950",
    )
    resolver = PolicyResolver((load_bundled_policy("gfx950"),), external=ext)
    desc = _conv_descriptor(nn.Conv3d(32, 32, 3, padding=1, groups=32), role=None)
    good = resolver.resolve(desc, ctx((64,) * 3), "backward_input")
    assert good.policy == "test" and dict(good.parameters) == {"engine": 1, "tile_w": 64, "depth_chunk": 8}
    fp32 = resolver.resolve(desc, ctx((64,) * 3, dtype="float32"), "backward_input")
    # The external selection is guarded; the bundled layer's VALU recipe wins.
    assert fp32.policy == "gfx950" and fp32.parameters["engine"] == tiles.ENGINE_VALU


def test_external_policy_precedes_bundled_and_reference_terminates():
    ext = policy(
        [{"id": "gn-native", "when": {"family": "group_norm3d"}, "use": {"training": {"implementation": "reference"}},
          "confidence": "measured-exact-context"}]
    )
    resolver = PolicyRegistry(external=policy_to_primitive(ext)).resolver()
    gn = _norm_descriptor(nn.GroupNorm(32, 32))
    d = resolver.resolve(gn, ctx((128,) * 3), "training")
    assert d.implementation == "reference" and d.policy == "test" and d.rule == "gn-native"


def test_reference_nvidia_policy_document_parses_and_stays_native():
    """A policy in the reference's own format naming its Triton kernels parses;
    on an NVIDIA context it resolves to the native route with a reason."""
    doc = {
        "version": 2, "kind": "mednext-accel-policy", "name": "sm120", "target": {"vendor": "nvidia", "sm": [12, 0]},
        "scope": {"dtype": "bfloat16"},
        "rules": [{"id": "regular-dx", "when": {"family": "depthwise_conv3d", "direction": "regular",
                                                "kernel_size": [3, 3, 3], "work": {"min": 1500000}},
                   "use": {"backward_input": {"implementation": "triton_depthwise_dx", "parameters": "auto"},
                           "backward_weight": {"implementation": "triton_split_dw", "parameters": {"dw_splits": 64, "dw_block": 1024}}},
                   "confidence": "measured-exact-context"}],
    }
    resolver = PolicyRegistry(external=doc).resolver()
    desc = _conv_descriptor(nn.Conv3d(32, 32, 3, padding=1, groups=32), role=None)
    d = resolver.resolve(desc, ctx((128,) * 3, arch=None, sm=(12, 0)), "backward_input")
    assert d.implementation == "reference" and d.guard_reason == "Triton backend is not part of this build"
    # The same document does not apply to the AMD device.
    amd = resolver.resolve(desc, ctx((128,) * 3), "backward_input")
    assert amd.implementation == "hip_depthwise_dx"


@pytest.mark.parametrize(
    "mutate, message",
    [
        (lambda d: d.update(version=1), "schema-v1"),
        (lambda d: d.update(kind="other"), "kind"),
        (lambda d: d.update(extra=1), "unknown fields"),
        (lambda d: d["rules"].append(dict(d["rules"][0])), "duplicate rule id"),
        (lambda d: d["rules"][0].update(confidence="sure"), "confidence"),
        (lambda d: d["rules"][0]["use"]["training"].update(implementation="fast"), "unknown implementation"),
        (lambda d: d["rules"][0]["use"]["training"].update(parameters={"splits": 0}), "positive integer"),
        (lambda d: d["rules"][0]["when"].update(batch={"min": 0}), "positive integer"),
        (lambda d: d.update(scope={"batch": {"max": 4}}) or d["rules"][0]["when"].update(batch={"max": 8}), "widen"),
    ],
)
def test_policy_schema_rejects_malformed_documents(mutate, message):
    doc = {
        "version": 2, "kind": "mednext-accel-policy", "name": "p", "target": {"vendor": "amd", "arch": "gfx950"},
        "rules": [{"id": "gn", "when": {"family": "group_norm3d"},
                   "use": {"training": {"implementation": "hip_group_norm", "parameters": "auto"}},
                   "confidence": "measured-exact-context"}],
    }
    mutate(doc)
    with pytest.raises(ValueError, match=message):
        parse_policy(doc)


def test_depthwise_parameter_validation():
    base = {"version": 2, "kind": "mednext-accel-policy", "name": "p", "target": {"vendor": "amd"}}
    for params, message in (
        ({"engine": 3}, "engine"),
        ({"engine": 2, "tile_w": 8}, "tile_w"),
        ({"engine": 1, "tile_w": 16}, "tile_w"),
        ({"engine": 0, "tile_w": 128}, "tile_w"),
        ({"depth_chunk": 0}, "positive"),
        ({"block": 128}, "unknown parameters"),
    ):
        doc = dict(base, rules=[{"id": "r", "when": {}, "confidence": "extrapolated",
                                 "use": {"backward_input": {"implementation": "hip_depthwise_dx", "parameters": params}}}])
        with pytest.raises(ValueError, match=message):
            parse_policy(doc)


def test_bundled_policy_round_trips():
    p = load_bundled_policy("gfx950")
    assert p.vendor == "amd" and p.target_arch == "gfx950"
    assert parse_policy(policy_to_primitive(p)) == p


def test_external_target_mismatch_warns_once():
    ext = policy([], arch="gfx942", name="mi300")
    resolver = PolicyResolver((), external=ext)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        assert resolver.warn_for_target("amd", "gfx950") is not None
        resolver.warn_for_target("amd", "gfx950")
    assert len(caught) == 1 and "gfx942" in str(caught[0].message)
    assert resolver.warn_for_target("amd", "gfx942") is None
    assert resolver.warn_for_sm((9, 5)) is None  # vendor mismatch: no warning


def test_decision_for_shape_without_a_gpu():
    wrapper = AdaptiveDepthwise3d(nn.Conv3d(64, 64, 3, padding=1, groups=64), PolicyRegistry().resolver(), MC)
    d = wrapper.decision_for_shape(
        batch_size=2, spatial_shape=(64, 64, 64), dtype="bfloat16", device_type="cuda", sm=(9, 5),
        total_vram_bytes=288 * 2**30, arch="gfx950", phase="backward_weight",
    )
    assert d.implementation == "hip_split_dw"
    assert [d.parameters[k] for k in ("engine", "tile_w", "depth_chunk")] == tiles.depthwise_recipe(
        2, 64, (64,) * 3, 3, "bfloat16", "weight_grad"
    )


def test_missing_library_falls_back_to_native_with_one_warning(monkeypatch):
    """The reference's wrapper runs the native op when its kernel backend
    cannot be imported (reference ops/adaptive.py:273-276). Here: a HIP
    selection on a (simulated) gfx950 device with ``libmednext_hip.so``
    unloadable runs PyTorch's operators, forward and backward, and warns once;
    with MEDNEXT_ACCEL_AMD_REQUIRE_HIP=1 the same call raises."""
    from mednext_accel_amd import _hip, adaptive

    def unloadable():
        raise _hip.HipLibraryError("libmednext_hip.so is not built")

    gfx950 = lambda x, mc, training: ctx(tuple(x.shape[2:]), dtype="float64", batch=x.shape[0])  # noqa: E731
    monkeypatch.setattr(_hip, "load", unloadable)
    monkeypatch.setattr(adaptive, "_context_from_tensor", gfx950)
    monkeypatch.setattr(adaptive, "_backend_state", [])
    monkeypatch.delenv(adaptive.REQUIRE_HIP_ENV, raising=False)

    torch.manual_seed(5)
    ref = nn.Sequential(nn.Conv3d(3, 3, 3, padding=1, groups=3), nn.GroupNorm(3, 3), nn.Conv3d(3, 7, 1)).double()
    cand = copy.deepcopy(ref)
    install_adaptive_operators(cand, resolver=PolicyRegistry().resolver(), model_context=MC)
    decisions = cand[0].phase_decisions(gfx950(torch.empty(2, 3, 4, 5, 6), MC, True))
    assert all(d.implementation != "reference" for d in decisions), decisions
    x = torch.randn(2, 3, 4, 5, 6, dtype=torch.double, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    with pytest.warns(RuntimeWarning, match="HIP kernels are unavailable"):
        b = cand(y)
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # reported once only
        b2 = cand(y)
    a = ref(x)
    torch.testing.assert_close(b, a)
    torch.testing.assert_close(b2, a)
    g = torch.randn_like(a)
    for got, want in zip(
        torch.autograd.grad(b, (y, *cand.parameters()), g), torch.autograd.grad(a, (x, *ref.parameters()), g), strict=True
    ):
        torch.testing.assert_close(got, want)

    monkeypatch.setattr(adaptive, "_backend_state", [])
    monkeypatch.setenv(adaptive.REQUIRE_HIP_ENV, "1")
    with pytest.raises(_hip.HipLibraryError):
        cand(y)


def test_resolution_traces_under_torch_compile_fullgraph():
    """The resolver runs inside the adaptive wrappers' forward, which
    torch.compile(fullgraph=True) traces: a resolution must trace without a
    graph break (reference tests/ops/test_phase_routing.py:142-158 compiles
    the wrapped model the same way)."""
    resolver = PolicyRegistry().resolver()
    desc = _conv_descriptor(nn.Conv3d(32, 32, 3, padding=1, groups=32), role="encoder_stages.0.0.depthwise")
    context = ctx((128,) * 3)

    def pick(x):
        d = resolver.resolve(desc, context, "backward_weight")
        return x + 1 if d.implementation == "hip_split_dw" else x - 1

    torch._dynamo.reset()
    compiled = torch.compile(pick, fullgraph=True, backend="eager")
    x = torch.zeros(3)
    assert torch.equal(compiled(x), pick(x)) and torch.equal(pick(x), x + 1)
