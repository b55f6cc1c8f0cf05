"""Problems larger than the last-level cache: the backward writes the
gradient with nontemporal stores (``stream_problem`` in
``ace_geometry.hpp``: logits, targets and gradient above 224 MB).  The cache
policy changes no arithmetic, so a streaming backward must give the same bits
as a backward that does not stream.

With ``reduction="sum"`` every batch index's coefficients and gradient are
its own (no 1/B in the Jacobian), so the gradient of a B = 2 call at
2 x 4 x 128 x 128 x 256 fp32 (302 MB: streams) equals, bit for bit, the
backward of each B = 1 half (151 MB: does not stream) given that call's own
coef, d and jac; the same at 2 x 4 x 128 x 128 x 512 bf16 (335 MB against
168 MB), whose gradient stores are 8 bytes wide.  (The halves' own forwards
agree with it only to float64 rounding: a batch index is tiled differently
at B = 1 and B = 2, and the soft moments' per-copy sums of u^2 are rounded
per copy, which d's float64 remainder carries; so the halves' losses are
compared to rtol 1e-6.)
"""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
from ace_kernels.impls import hip_mi355x as hip
from gpu_helpers import run, say

pytestmark = pytest.mark.gpu

STREAM_BYTES = 224 << 20


def problem_bytes(x: torch.Tensor, y: torch.Tensor) -> int:
    return 2 * x.numel() * x.element_size() + y.numel() * y.element_size()


@pytest.mark.parametrize("dtype,depth", [(torch.float32, 256), (torch.bfloat16, 512)])
@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_streaming_backward_matches_the_halves(binning, dtype, depth) -> None:
    gen = torch.Generator().manual_seed(11)
    x = (torch.randn((2, 4, 128, 128, depth), generator=gen) * 1.5).to(dtype).cuda()
    y = torch.randint(0, 4, (2, 1, 128, 128, depth), generator=gen).cuda()
    assert problem_bytes(x, y) > STREAM_BYTES >= problem_bytes(x[:1], y[:1])
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax", reduction="sum")
    say(f"streaming backward {binning} {dtype}: B=2 (streams) against two B=1 backwards")
    loss, grad = run("hip_mi355x", x, y, cfg)
    pl = hip.make_plan(x, y, cfg)
    _, coef, d, jac, _, _ = hip.hip_forward(pl, cfg)
    for b in range(2):
        half = hip.make_plan(x[b:b + 1].contiguous(), y[b:b + 1].contiguous(), cfg)
        db = (d[:, b:b + 1] if d.dim() == 4 else d[b:b + 1]).contiguous()
        g = hip.hip_backward(half, coef[b:b + 1].contiguous(), db, jac[b:b + 1].contiguous(),
                             torch.ones((), device=x.device))
        torch.cuda.synchronize()
        assert torch.equal(grad[b:b + 1], g), f"batch index {b}"
    halves = [run("hip_mi355x", x[b:b + 1].contiguous(), y[b:b + 1].contiguous(), cfg)[0] for b in range(2)]
    torch.testing.assert_close(loss, halves[0] + halves[1], rtol=1e-6, atol=0.0)
