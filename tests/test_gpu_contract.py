"""The reference's contract checks of a fused implementation, on the HIP path.

- Launches: one forward + backward issues exactly the two HIP kernels (the
  forward with its fused epilogue, the backward) plus torch's glue, within
  the reference's bound of 8 device kernels (``tests/test_triton.py:453-471``).
- Saved bytes: the autograd node keeps, beyond its inputs, exactly coef and d
  (float32 [B, C', K]; soft binning also keeps d's float32 remainder) and jac
  (float32 [B, C']): 2 B C' K 4 + B C' 4 bytes hard, 3 B C' K 4 + B C' 4
  soft (``tests/test_triton.py:331-346``, which allows up to 1 KB more;
  ``tests/test_saved_tensors.py``).
- torch.compile: the reference's pattern, ``torch.compile(step,
  fullgraph=True)`` with the default backend, where ``step`` is a network
  plus ``ace_loss(..., impl=...)`` through the custom ops; loss and weight
  gradient equal eager within the reference's bars
  (``tests/test_triton.py:474-495``).
"""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels import measure as m
from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _inputs(shape, seed=0):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=gen) * 2.0).cuda()
    y = torch.randint(0, shape[1], (shape[0], 1, *shape[2:]), generator=gen).cuda()
    return x, y


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_two_hip_kernels_per_forward_backward(binning) -> None:
    from torch.profiler import ProfilerActivity, profile

    cfg = ACEConfig(binning=binning, to_onehot_y=True)
    x, y = _inputs((2, 4, 32, 32, 32), 1)
    x.requires_grad_(True)
    for _ in range(2):  # tables, workspace and class weights cached outside the profile
        torch.autograd.backward(ace_loss(x, y, cfg, impl="hip_mi355x"))
    torch.cuda.synchronize()
    say(f"launches {binning}")
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        torch.autograd.backward(ace_loss(x, y, cfg, impl="hip_mi355x"))
        torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type.name == "CUDA"]
    ours = [k for k in kernels if "ace::" in k]
    say(f"  {len(kernels)} device kernels: {kernels}")
    assert len(ours) == 2, kernels
    assert any("fwd_kernel" in k for k in ours) and any("bwd_kernel" in k for k in ours)
    assert len(kernels) <= 8, kernels


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("include_background", [True, False])
@pytest.mark.parametrize("impl", ["hip_mi355x", "hip_mi355x_op"])
def test_saved_extra_bytes_are_the_per_bin_outputs(binning, include_background, impl) -> None:
    cfg = ACEConfig(binning=binning, to_onehot_y=True, include_background=include_background)
    b, c, k = 2, 4, cfg.num_bins
    cl = c - (0 if include_background else 1)
    x, y = _inputs((b, c, 16, 16, 16), 2)
    x.requires_grad_(True)
    say(f"saved bytes {impl} {binning} background={include_background}")
    extra = m.saved_extra_bytes(lambda: ace_loss(x, y, cfg, impl=impl), exclude=[x, y])
    # coef and d per bin (soft: d and its float32 remainder), jac per class
    per_bin = 3 if binning == "soft" else 2
    assert extra == per_bin * b * cl * k * 4 + b * cl * 4, extra


@pytest.mark.timeout(600)
@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_torch_compile_default_backend(binning) -> None:
    torch._dynamo.reset()
    cfg = ACEConfig(binning=binning, to_onehot_y=True)
    x, y = _inputs((2, 4, 16, 16, 16), 3)
    net = torch.nn.Conv3d(4, 4, 3, padding=1).cuda()

    def step(inp):
        return ace_loss(net(inp), y, cfg, impl="hip_mi355x_op")

    say(f"torch.compile (default backend) {binning}")
    results = []
    for fn in (step, torch.compile(step, fullgraph=True)):
        net.zero_grad()
        loss = fn(x)
        torch.autograd.backward(loss)
        assert net.weight.grad is not None
        results.append((loss.detach(), net.weight.grad.clone()))
    torch.testing.assert_close(results[1][0], results[0][0], rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(results[1][1], results[0][1], rtol=1e-3, atol=1e-6)
