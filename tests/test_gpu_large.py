"""Maximum sizes: 2^31 voxels per channel row, built by tiling a small volume
T = 2^16 times along the voxels.  With hard binning every count and sum of
the tiled volume is T times the small one's (T a power of two, fixed-point
sums exact), so its loss is bit-identical to the small volume's and its
gradient is exactly the small volume's divided by T.  That is an exact check
of the kernels' 64-bit index paths at a size no CPU oracle reaches.  Soft
binning follows the same scaling up to the rounding of the per-copy sums of
squares before they enter the final sums (the shift grows with N): within
1e-6.  The small volume itself is checked against the oracle.
"""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
from gpu_helpers import LOSS_ATOL, LOSS_RTOL, assert_grad_close, run, say

pytestmark = pytest.mark.gpu

SMALL = 1 << 15
TILES = 1 << 16  # SMALL * TILES = 2^31 voxels


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_tiled_volume_of_2_pow_31_voxels(binning) -> None:
    if torch.cuda.get_device_properties(0).total_memory < 160 * 2**30:
        pytest.skip("needs ~100 GiB of device memory")
    from oracle.reference import register_reference

    register_reference()
    c = 2
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    gen = torch.Generator().manual_seed(31)
    xs = torch.randn((1, c, SMALL), generator=gen) * 2.0
    ys = torch.randint(0, c, (1, 1, SMALL), generator=gen)
    say(f"large: {binning} small volume ({SMALL} voxels)")
    ls, gs = run("hip_mi355x", xs.cuda(), ys.cuda(), cfg)
    lr, gr = run("reference", xs, ys, cfg)
    torch.testing.assert_close(ls.cpu(), lr, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    assert_grad_close(gs, gr, xs, cfg)

    say(f"large: {binning} tiled volume ({SMALL * TILES} voxels)")
    xb = xs.cuda().repeat(1, 1, TILES)
    yb = ys.cuda().repeat(1, 1, TILES)
    lb, gb = run("hip_mi355x", xb, yb, cfg)
    del xb, yb
    expect = (gs / TILES).view(1, c, 1, SMALL)
    got = gb.view(1, c, TILES, SMALL)
    if binning == "hard":
        assert torch.equal(lb, ls), (float(lb), float(ls))
        assert bool((got == expect).all())
    else:
        torch.testing.assert_close(lb, ls, rtol=1e-6, atol=0.0)
        err = (got - expect).abs().amax()
        assert float(err) <= 1e-6 * float(expect.abs().amax()), float(err)
