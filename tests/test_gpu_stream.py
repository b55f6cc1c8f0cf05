"""Problems larger than the last-level cache: the backward writes the
gradient with nontemporal stores (``stream_problem`` in
``ace_geometry.hpp``: logits, targets and gradient above 224 MB).  The cache
policy changes no arithmetic, so a streaming call must give the same bits as
calls that do not stream.

With ``reduction="sum"`` every batch index's statistics, coefficients and
gradient are its own (no 1/B in the Jacobian), so the gradient of a B = 2
call at 2 x 4 x 128 x 128 x 256 fp32 (302 MB: streams) equals, bit for bit,
the gradients of its two B = 1 halves (151 MB: do not stream), and its loss
is the sum of theirs; the same at 2 x 4 x 128 x 128 x 512 bf16 (335 MB
against 168 MB), whose gradient stores are 8 bytes wide.
"""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
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
    say(f"streaming backward {binning} {dtype}: B=2 (streams) against two B=1 calls")
    loss, grad = run("hip_mi355x", x, y, cfg)
    halves = [run("hip_mi355x", x[b:b + 1].contiguous(), y[b:b + 1].contiguous(), cfg)
              for b in range(2)]
    torch.cuda.synchronize()
    for b, (_, g) in enumerate(halves):
        assert torch.equal(grad[b:b + 1], g), f"batch index {b}"
    total = halves[0][0] + halves[1][0]
    torch.testing.assert_close(loss, total, rtol=1e-6, atol=0.0)
