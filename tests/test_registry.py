"""Registry / config API: the reference's contract (upstream tests/test_registry.py)."""

from __future__ import annotations

import pytest
import torch
from pydantic import ValidationError

from ace_kernels import ACEConfig, ace_loss, available_impls, get_impl
from ace_kernels.registry import _REGISTRY, ImplSpec, register


def test_hip_impl_registered_for_cuda_only() -> None:
    spec = get_impl("hip_mi355x")
    for binning in ("hard", "soft"):
        assert spec.supports(binning, "cuda")
        assert not spec.supports(binning, "cpu")


def test_unknown_impl_raises() -> None:
    with pytest.raises(KeyError, match="unknown implementation"):
        get_impl("nope")


def test_duplicate_registration_raises() -> None:
    with pytest.raises(ValueError, match="already registered"):
        register("hip_mi355x", description="dup")(get_impl("hip_mi355x").fn)


def test_unsupported_device_raises() -> None:
    x = torch.rand(1, 2, 4)
    with pytest.raises(ValueError, match="does not support"):
        ace_loss(x, x, ACEConfig(), impl="hip_mi355x")


def test_unsupported_binning_raises(monkeypatch: pytest.MonkeyPatch) -> None:
    def _impl(x, y, c):
        return x.sum()

    spec = ImplSpec("_hard_only_test", _impl, frozenset({"hard"}), frozenset({"cpu"}), "test")
    monkeypatch.setitem(_REGISTRY, spec.name, spec)
    x = torch.rand(1, 2, 4)
    with pytest.raises(ValueError, match="does not support"):
        ace_loss(x, x, ACEConfig(binning="soft"), impl="_hard_only_test")
    assert "_hard_only_test" in {s.name for s in available_impls(binning="hard")}
    assert "_hard_only_test" not in {s.name for s in available_impls(binning="soft")}


def test_config_rejects_unknown_and_invalid_fields() -> None:
    with pytest.raises(ValidationError):
        ACEConfig.model_validate({"num_binz": 20})
    with pytest.raises(ValidationError):
        ACEConfig(num_bins=0)
    with pytest.raises(ValidationError):
        ACEConfig(empty_weight=-1.0)
    with pytest.raises(ValidationError):
        ACEConfig(binning="medium")


def test_config_is_frozen_and_roundtrips() -> None:
    c = ACEConfig(binning="soft", weight=(0.1, 1.0), num_bins=50)
    with pytest.raises(ValidationError):
        c.num_bins = 3
    assert ACEConfig.model_validate_json(c.model_dump_json()) == c


def test_class_weight_validation() -> None:
    from ace_kernels.common import class_weights

    assert class_weights(ACEConfig(), 4) is None
    assert class_weights(ACEConfig(weight=2.0), 3) == [2.0, 2.0, 2.0]
    assert class_weights(ACEConfig(weight=(1.0, 2.0)), 1) is None
    with pytest.raises(ValueError):
        class_weights(ACEConfig(weight=(1.0, 2.0)), 3)
    with pytest.raises(ValueError):
        class_weights(ACEConfig(weight=(1.0, -2.0)), 2)


def test_tables_are_the_reference_linspace() -> None:
    from ace_kernels.common import bin_tables

    eps = torch.finfo(torch.float32).eps
    for k in (1, 20, 50):
        edges, none = bin_tables(k, False, torch.device("cpu"))
        assert none is None
        assert torch.equal(edges, torch.linspace(0.0, 1.0 + eps, k + 1)[1:])
        half, repl = bin_tables(k, True, torch.device("cpu"))
        full = torch.linspace(0.0, 1.0 + eps, 2 * k + 1)
        assert torch.equal(half, full[1:])
        assert repl.numel() == 2 * k + 2 and repl[0] == -1e4 and repl[-1] == 1e4
        assert torch.equal(repl[1:-1:2], full[1::2]) and torch.equal(repl[2:-1:2], full[1::2])


def test_default_impl_resolves_automatically() -> None:
    """``ace_loss(x, y, config)`` with no impl: HIP tensors take hip_mi355x;
    CPU tensors take the first registered CPU entry (the test suite's oracle),
    and with none registered the call raises a clear ValueError."""
    from ace_kernels.registry import resolve_impl

    assert resolve_impl("auto", "hard", "cuda") == "hip_mi355x"
    assert resolve_impl("auto", "soft", "cuda") == "hip_mi355x"
    assert resolve_impl("hip_mi355x_op", "hard", "cuda") == "hip_mi355x_op"
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 5, 4, generator=gen)
    y = torch.randint(0, 3, (2, 1, 5, 4), generator=gen)
    cfg = ACEConfig(to_onehot_y=True, activation="softmax")
    cpu_name = resolve_impl("auto", "hard", "cpu")
    assert get_impl(cpu_name).supports("hard", "cpu")
    assert torch.equal(ace_loss(x, y, cfg), ace_loss(x, y, cfg, impl=cpu_name))


def test_default_impl_without_a_cpu_entry_raises(monkeypatch: pytest.MonkeyPatch) -> None:
    from ace_kernels import registry

    kept = {k: v for k, v in registry._REGISTRY.items() if "cpu" not in v.devices}
    monkeypatch.setattr(registry, "_REGISTRY", kept)
    x = torch.rand(1, 2, 4)
    with pytest.raises(ValueError, match="no registered implementation"):
        ace_loss(x, x, ACEConfig())
