"""The end-to-end training step (``ace_kernels.e2e``) on MI355X: the mL1-ACE
term through ``ace_loss(impl="hip_mi355x")`` per level, or through
``ace_loss_levels`` in one launch per direction, inside a deep-supervision
training step with fp16 autocast (the reference's ``src/ace_bench/e2e.py``
step, MONAI-free).  The two ACE routes give the same first-step loss and ACE
term (each level bit-identical, summed in the same order), the step without
the ACE term differs from them by exactly 0.33 x the weighted ACE sum, and
every loss is finite."""

from __future__ import annotations

import math

import pytest
import torch

from ace_kernels import e2e
from gpu_helpers import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_training_steps_with_the_hip_loss(binning: str) -> None:
    results = {}
    for ace in ("hip_mi355x", "levels", "none"):
        cfg = e2e.E2EConfig(binning=binning, ace=ace, batch=2, patch=(32, 32, 32),
                            init_filters=8, steps=3, skip_steps=1)
        say(f"e2e {binning} ace={ace}: 3 steps at 32^3")
        res = e2e.train(cfg)
        assert all(math.isfinite(v) for v in res.losses), res.losses
        results[ace] = res
    a, b, none = results["hip_mi355x"], results["levels"], results["none"]
    assert a.aces[0] > 0 and b.aces[0] == a.aces[0]
    assert math.isclose(a.losses[0], b.losses[0], rel_tol=1e-6)
    assert math.isclose(a.losses[0] - none.losses[0], 0.33 * a.aces[0], rel_tol=1e-4, abs_tol=1e-6)
