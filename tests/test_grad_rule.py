"""The boundary-voxel rule of the GPU gradient comparisons, on the CPU: a
difference at a voxel whose probability sits on a bin boundary passes, one
elsewhere fails, and more than a few boundary voxels fail."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
from gpu_helpers import assert_grad_close, near_boundary_voxels


def _inputs(binning):
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    gen = torch.Generator().manual_seed(3)
    x = torch.randn((2, 2, 40), generator=gen)
    # voxel (0, 5): p0 exactly on a boundary (0.5 is an edge of 20 hard bins
    # and a half boundary of 20 soft bins)
    x[0, :, 5] = 0.0
    return cfg, x


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_boundary_voxel_may_differ(binning):
    cfg, x = _inputs(binning)
    near = near_boundary_voxels(x, cfg)
    assert near[0, 5]
    g = torch.randn_like(x)
    h = g.clone()
    h[0, :, 5] += 1.0
    bad = assert_grad_close(h, g, x, cfg)
    assert bad[0, 5] and int(bad.sum()) == 1


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_difference_elsewhere_fails(binning):
    cfg, x = _inputs(binning)
    far = int((~near_boundary_voxels(x, cfg))[1].nonzero()[0])
    g = torch.randn_like(x)
    h = g.clone()
    h[1, 0, far] *= 1.0 + 1e-3
    with pytest.raises(AssertionError, match="away from bin boundaries"):
        assert_grad_close(h, g, x, cfg)


def test_many_boundary_voxels_fail():
    cfg, x = _inputs("soft")
    x[:, :, :4] = 0.0
    g = torch.randn_like(x)
    h = g.clone()
    h[:, :, :4] += 1.0
    with pytest.raises(AssertionError, match="boundary voxels differ"):
        assert_grad_close(h, g, x, cfg)
