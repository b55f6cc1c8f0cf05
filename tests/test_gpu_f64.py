"""float64 logits on the HIP path (ace_forward_f64 / ace_backward_f64).

The reference sends float64 input to its handwritten "recompute" backward in
torch (``src/ace_kernels/impls/v6_triton.py:226-227``); its tests check that
path with ``gradcheck`` on six configurations x two binnings
(``tests/test_v2.py:14-56``: eps 1e-7, atol 1e-6, rtol 1e-4) and against
autograd in float64 on random small problems (``tests/test_v2.py:59-99``).
Here the same gradchecks run through ``impl="hip_mi355x"`` on the device, and
loss, gradient and the float64 bin statistics are compared with the oracle's
float64 restatement of that path (``oracle/v2.py``) on the CPU: loss rtol 1e-10,
gradient rtol 1e-9 / atol 1e-13 (float64 rounding in a different order; the
bins agree).  Results are also bit-identical run to run."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels import measure as m
from ace_kernels.impls import hip_mi355x as hip
from gpu_helpers import say

pytestmark = pytest.mark.gpu

# tests/test_v2.py:14-28
CONFIGS = {
    "paper": {"to_onehot_y": True},
    "no-background-weights": {"to_onehot_y": True, "include_background": False,
                              "weight": (2.0, 0.5, 1.0)},
    "reduction-none": {"to_onehot_y": True, "reduction": "none"},
    "reduction-sum-kept-empty": {"to_onehot_y": True, "reduction": "sum",
                                 "ignore_empty_classes": False},
    "sigmoid": {"activation": "sigmoid"},
    "onehot-target": {},
}
LOSS_RTOL, LOSS_ATOL = 1e-10, 1e-13
GRAD_RTOL, GRAD_ATOL = 1e-9, 1e-13


def _inputs(config: ACEConfig, b, c, spatial, seed, scale=2.0, bias=1.0):
    shape = m.ShapeSpec("f64", b, c, tuple(spatial), logit_scale=scale, target_bias=bias)
    x, y = m.make_inputs(shape, config, "cpu", seed=seed)
    return x.double(), y


def _oracle(x, y, config, upstream=None):
    from oracle.v2 import v2_ace

    leaf = x.detach().clone().requires_grad_(True)
    loss = v2_ace(leaf, y, config)
    go = torch.ones_like(loss) if upstream is None else upstream.view_as(loss)
    (g,) = torch.autograd.grad(loss, leaf, go)
    return loss.detach(), g


def _device(x, y, config, upstream=None):
    leaf = x.detach().clone().cuda().requires_grad_(True)
    loss = ace_loss(leaf, y.cuda(), config, impl="hip_mi355x")
    assert loss.dtype == torch.float64
    go = torch.ones_like(loss) if upstream is None else upstream.cuda().view_as(loss)
    (g,) = torch.autograd.grad(loss, leaf, go)
    assert g.dtype == torch.float64
    return loss.detach().cpu(), g.cpu()


def _check(x, y, config, upstream=None):
    want_loss, want_g = _oracle(x, y, config, upstream)
    loss, g = _device(x, y, config, upstream)
    torch.testing.assert_close(loss, want_loss, rtol=LOSS_RTOL, atol=LOSS_ATOL, equal_nan=True)
    torch.testing.assert_close(g, want_g, rtol=GRAD_RTOL, atol=GRAD_ATOL)
    return loss, g


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_gradcheck_float64(name: str, binning: str) -> None:
    """tests/test_v2.py:41-56 with the HIP impl: analytic == finite differences."""
    config = ACEConfig.model_validate({"binning": binning, **CONFIGS[name]})
    channels = 1 if name == "sigmoid" else 4
    x, y = _inputs(config, 2, channels, (5, 5, 4), 7)
    xd = x.cuda().requires_grad_(True)
    yd = y.cuda()
    say(f"f64 gradcheck {name} {binning}")
    assert torch.autograd.gradcheck(lambda inp: ace_loss(inp, yd, config, impl="hip_mi355x"),
                                    (xd,), eps=1e-7, atol=1e-6, rtol=1e-4)
    _check(x, y, config)


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_configs_against_the_float64_oracle(name: str, binning: str) -> None:
    config = ACEConfig.model_validate({"binning": binning, **CONFIGS[name]})
    channels = 1 if name == "sigmoid" else 4
    x, y = _inputs(config, 2, channels, (24, 20, 16), 11)
    say(f"f64 oracle {name} {binning}")
    _check(x, y, config)


def test_random_problems_against_the_float64_oracle() -> None:
    """tests/test_v2.py:59-99's ranges: channels 2-5, voxels 1-200, bins 1-25,
    background in or out, both binnings; plus right edges and upstream
    gradients per class."""
    gen = torch.Generator().manual_seed(2024)
    for case in range(40):
        r = torch.randint(0, 1 << 30, (8,), generator=gen).tolist()
        binning = "hard" if r[0] % 2 else "soft"
        channels = 2 + r[1] % 4
        voxels = 1 + r[2] % 200
        bins = 1 + r[3] % 25
        config = ACEConfig(binning=binning, num_bins=bins, to_onehot_y=True,
                           include_background=bool(r[4] % 2), right=bool(r[5] % 3 == 0),
                           reduction="none" if r[6] % 4 == 0 else "mean")
        x, y = _inputs(config, 1 + r[7] % 3, channels, (voxels,), case, scale=1.0 + (r[7] % 3))
        upstream = None
        if config.reduction == "none":
            cl = channels - (0 if config.include_background else 1)
            upstream = torch.randn((x.shape[0], cl, 1), generator=gen, dtype=torch.float64)
        say(f"f64 random {case}: {binning} C={channels} N={voxels} K={bins} B={x.shape[0]}")
        _check(x, y, config, upstream)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_statistics_and_determinism(binning: str) -> None:
    from oracle import v2

    config = ACEConfig(binning=binning, to_onehot_y=True, include_background=False)
    x, y = _inputs(config, 2, 4, (40, 36, 32), 5)
    pl = hip.make_plan(x.cuda(), y.cuda(), config)
    say(f"f64 stats {binning}")
    out1 = hip.hip_forward(pl, config, stats=True)
    out2 = hip.hip_forward(pl, config, stats=True)
    for a, b in zip(out1, out2):
        assert torch.equal(a, b)
    prep = v2.prepare(x, y, config)
    st = v2.bin_stats(prep, config)
    want = torch.stack((st.weight, st.sum_p, st.sum_gt))
    torch.testing.assert_close(out1[5].cpu(), want, rtol=1e-11, atol=1e-12)
    f, present, coef, d = v2.coefficients(st)
    torch.testing.assert_close(out1[2].cpu(), d, rtol=1e-9, atol=1e-13)
    torch.testing.assert_close(out1[1].cpu(), coef, rtol=1e-9, atol=1e-15)


def test_benchmark_shape_against_the_float64_oracle() -> None:
    """Configuration 2's layout at 64^3 per batch index (both binnings)."""
    for binning in ("hard", "soft"):
        config = ACEConfig(binning=binning, to_onehot_y=True)
        x, y = _inputs(config, 2, 4, (64, 64, 64), 3, scale=1.5, bias=2.5)
        say(f"f64 64^3 {binning}")
        _check(x, y, config)


def test_onehot_and_probability_inputs() -> None:
    """Float one-hot targets (read as float64) and activation "none" on
    probabilities, hard and soft."""
    for binning in ("hard", "soft"):
        for act in ("none", "softmax"):
            config = ACEConfig(binning=binning, activation=act, to_onehot_y=False)
            x, y = _inputs(config, 2, 3, (10, 9, 8), 17)
            if act == "none":
                x = torch.softmax(x, 1)
            say(f"f64 onehot {binning} {act}")
            _check(x, y, config)
