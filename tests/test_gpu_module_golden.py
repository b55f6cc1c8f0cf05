"""The drop-in modules on the device against the reference's golden vectors.

Upstream ``tests/test_module.py:52-70`` runs all 43 cases through its
``HardL1ACELoss`` / ``SoftL1ACELoss`` and checks ``other_act``; here the
modules, built from each case's config with the upstream keyword arguments
(``tests/test_module.py:29-43``: sigmoid / softmax flags, reduction, weight,
right, ignore_empty_classes, and empty_weight for soft binning), run on the
HIP device through ``impl="auto"`` and are checked against the stored loss
and gradient at the reference's tolerances (loss rtol 1e-5 / atol 1e-6,
gradient rtol 1e-4 / atol 1e-7).  ``other_act`` (a softmax applied by torch
before the loss, the module then binning probabilities) is checked against
the CPU reference given the same activation."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
from ace_kernels.module import HardL1ACELoss, SoftL1ACELoss
from golden_cases import load_golden
from gpu_helpers import GRAD_ATOL, GRAD_RTOL, LOSS_ATOL, LOSS_RTOL, assert_grad_close, say

pytestmark = pytest.mark.gpu
GOLDEN = load_golden()


def _module(config: ACEConfig, **extra):
    kwargs = {
        "num_bins": config.num_bins,
        "include_background": config.include_background,
        "to_onehot_y": config.to_onehot_y,
        "sigmoid": config.activation == "sigmoid",
        "softmax": config.activation == "softmax",
        "reduction": config.reduction,
        "weight": config.weight,
        "right": config.right,
        "ignore_empty_classes": config.ignore_empty_classes,
    }
    kwargs.update(extra)
    if config.binning == "soft":
        return SoftL1ACELoss(empty_weight=config.empty_weight, **kwargs)
    return HardL1ACELoss(**kwargs)


def _run(module, x, y):
    leaf = x.detach().clone().requires_grad_(True)
    loss = module(leaf, y)
    (g,) = torch.autograd.grad(loss.sum(), leaf)
    return loss.detach(), g


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_module_matches_golden(name: str) -> None:
    case = GOLDEN[name]
    config = ACEConfig.model_validate(case.config)
    module = _module(config)
    assert module.config == config
    assert module.resolve_impl(torch.device("cuda")) == "hip_mi355x"
    say(f"module golden {name}")
    loss, grad = _run(module, case.input.cuda(), case.target.cuda())
    torch.testing.assert_close(loss.cpu(), case.loss, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    torch.testing.assert_close(grad.cpu(), case.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_module_other_act(binning: str) -> None:
    from oracle.reference import reference_ace

    case = GOLDEN[f"paper-3d-{binning}"]
    act = torch.nn.Softmax(dim=1)
    cls = HardL1ACELoss if binning == "hard" else SoftL1ACELoss
    module = cls(to_onehot_y=True, other_act=act)
    assert module.config.activation == "none"
    say(f"module other_act {binning}")
    loss, grad = _run(module, case.input.cuda(), case.target.cuda())
    leaf = case.input.clone().requires_grad_(True)
    ref = reference_ace(act(leaf), case.target, module.config)
    (ref_grad,) = torch.autograd.grad(ref.sum(), leaf)
    torch.testing.assert_close(loss.cpu(), ref.detach(), rtol=LOSS_RTOL, atol=LOSS_ATOL)
    # the device's softmax and torch's CPU softmax may differ by an ulp, so a
    # voxel within 1e-6 of a bin boundary may fall on the other side
    assert_grad_close(grad, ref_grad, case.input, module.config.model_copy(update={"activation": "softmax"}))
