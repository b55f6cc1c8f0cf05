"""HIP implementation vs the reference's 43 golden cases (loss and gradient).

Tolerances: the reference's own (``tests/helpers.py:15-21`` upstream): loss
rtol 1e-5 / atol 1e-6; gradient rtol 1e-4 / atol 1e-7 (the north star's bar).
"""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
from golden_cases import load_golden
from gpu_helpers import GRAD_ATOL, GRAD_RTOL, LOSS_ATOL, LOSS_RTOL, run, say

pytestmark = pytest.mark.gpu
GOLDEN = load_golden()


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_hip_matches_golden(name: str) -> None:
    case = GOLDEN[name]
    config = ACEConfig.model_validate(case.config)
    say(f"golden {name}: x{tuple(case.input.shape)} {config.binning} K={config.num_bins}")
    loss, grad = run("hip_mi355x", case.input.cuda(), case.target.cuda(), config)
    torch.testing.assert_close(loss.cpu(), case.loss, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    torch.testing.assert_close(grad.cpu(), case.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)
