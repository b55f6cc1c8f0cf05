"""Drop-in modules and custom-op packaging, host side (no kernel launched).

Mirrors the reference's module tests (upstream ``tests/test_module.py:18-101``):
the constructor keeps the upstream signature and validation, ``impl="auto"``
picks the HIP implementation for HIP tensors, and a forced implementation is
used as named.  The custom ops' fake kernels give the real kernels' output
shapes (``v6_triton.py:154-167`` upstream), checked here under FakeTensorMode.
"""

from __future__ import annotations

import inspect

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels.impls.hip_mi355x import _dump
from ace_kernels.module import HardL1ACELoss, SoftL1ACELoss

# upstream constructor parameters, in order, with defaults
# (src/ace_kernels/module.py:112-124 and :150-163 of the reference)
HARD_PARAMS = [("num_bins", 20), ("include_background", True), ("to_onehot_y", False),
               ("sigmoid", False), ("softmax", False), ("other_act", None), ("reduction", "mean"),
               ("weight", None), ("right", False), ("ignore_empty_classes", True), ("impl", "auto")]
SOFT_PARAMS = HARD_PARAMS[:8] + [("empty_weight", 0.01)] + HARD_PARAMS[8:]


@pytest.mark.parametrize("cls, expected", [(HardL1ACELoss, HARD_PARAMS), (SoftL1ACELoss, SOFT_PARAMS)])
def test_upstream_signature(cls, expected) -> None:
    params = list(inspect.signature(cls.__init__).parameters.values())[1:]
    assert [(p.name, p.default) for p in params] == expected
    assert params[-1].kind is inspect.Parameter.KEYWORD_ONLY  # impl


def test_validation() -> None:
    with pytest.raises(ValueError, match="Incompatible values"):
        HardL1ACELoss(sigmoid=True, softmax=True)
    with pytest.raises(TypeError, match="other_act"):
        HardL1ACELoss(other_act=3)
    with pytest.raises(KeyError, match="unknown implementation"):
        SoftL1ACELoss(impl="nope")
    with pytest.raises(ValueError, match="Unsupported reduction"):
        HardL1ACELoss(reduction="max")


def test_config_mapping() -> None:
    class Reduction:  # an enum-like reduction (MONAI's LossReduction has .value)
        value = "sum"

    m = SoftL1ACELoss(num_bins=7, to_onehot_y=True, softmax=True, include_background=False,
                      reduction=Reduction(), weight=torch.tensor([1.0, 2.0, 3.0]), empty_weight=0.5,
                      right=True, ignore_empty_classes=False)
    assert m.config == ACEConfig(binning="soft", num_bins=7, activation="softmax", to_onehot_y=True,
                                 include_background=False, reduction="sum", weight=(1.0, 2.0, 3.0),
                                 empty_weight=0.5, right=True, ignore_empty_classes=False)
    assert HardL1ACELoss(sigmoid=True, weight=2).config.activation == "sigmoid"
    assert HardL1ACELoss(weight=2).config.weight == 2.0
    assert HardL1ACELoss().config.activation == "none"


def test_impl_resolution() -> None:
    m = HardL1ACELoss(softmax=True)
    assert m.resolve_impl(torch.device("cuda")) == "hip_mi355x"
    with pytest.raises(ValueError, match="no implementation"):
        m.resolve_impl(torch.device("cpu"))
    assert HardL1ACELoss(impl="hip_mi355x_op").resolve_impl(torch.device("cpu")) == "hip_mi355x_op"


def test_forced_impl_runs_through_the_registry() -> None:
    """The module forwards to the named registry implementation (here the
    test oracle, registered by conftest for the CPU)."""
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 6, 5, generator=gen)
    y = torch.randint(0, 3, (2, 1, 6, 5), generator=gen)
    for cls in (HardL1ACELoss, SoftL1ACELoss):
        m = cls(num_bins=5, to_onehot_y=True, softmax=True, impl="reference")
        assert torch.equal(m(x, y), ace_loss(x, y, m.config, impl="reference"))
    # other_act is applied before the loss
    m = HardL1ACELoss(num_bins=5, to_onehot_y=True, other_act=lambda t: torch.softmax(t, 1),
                      impl="reference")
    ref = ace_loss(torch.softmax(x, 1), y, ACEConfig(num_bins=5, to_onehot_y=True, activation="none"),
                   impl="reference")
    assert torch.equal(m(x, y), ref)


@pytest.mark.parametrize("reduction", ["mean", "none"])
@pytest.mark.parametrize("include_background", [True, False])
def test_custom_op_fake_shapes(reduction, include_background) -> None:
    from torch._subclasses.fake_tensor import FakeTensorMode

    cfg = ACEConfig(binning="soft", num_bins=7, reduction=reduction,
                    include_background=include_background, to_onehot_y=True)
    with FakeTensorMode():
        x = torch.empty(2, 4, 8, 8, 3, device="cuda")
        y = torch.empty(2, 1, 8, 8, 3, dtype=torch.int64, device="cuda")
        loss, coef, d, jac = torch.ops.ace_kernels.hip_forward(x, y, _dump(cfg))
        cl = 4 if include_background else 3
        assert tuple(loss.shape) == ((2, cl, 1, 1, 1) if reduction == "none" else ())
        assert tuple(coef.shape) == (2, cl, 7)
        assert tuple(d.shape) == (2, 2, cl, 7)  # soft float32: d and its remainder
        assert tuple(jac.shape) == (2, cl)
        go = torch.empty(loss.shape, device="cuda")
        dx = torch.ops.ace_kernels.hip_backward(x, y, coef, d, jac, go, _dump(cfg))
        assert dx.shape == x.shape and dx.dtype == x.dtype
