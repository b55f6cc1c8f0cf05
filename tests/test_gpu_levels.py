"""Several levels of one loss in one launch per direction (``ace_loss_levels``):
each level's loss and gradient are bit-identical to a separate
``ace_loss(..., impl="hip_mi355x")`` call on that level (same blocks, same
integer sums), for hard and soft binning, every fast channel count,
background dropped, the three reductions, per-class upstream gradients, an
empty level, and configurations without a fast kernel rejected.  Each case
runs twice: the first call of a levels signature takes the Python autograd
Function, the second the C++ node (``AceLevelsBackward``)."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels.levels import ace_loss_levels
from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _levels(b, c, sizes, seed):
    gen = torch.Generator().manual_seed(seed)
    xs, ys = [], []
    for s in sizes:
        shape = (b, c, *s)
        xs.append((torch.randn(shape, generator=gen) * 2.0).cuda())
        ys.append(torch.randint(0, c, (b, 1, *s), generator=gen).cuda())
    return xs, ys


def _separate(xs, ys, cfg, ups):
    out = []
    for x, y, up in zip(xs, ys, ups):
        leaf = x.clone().requires_grad_(True)
        loss = ace_loss(leaf, y, cfg, impl="hip_mi355x")
        (g,) = torch.autograd.grad(loss, leaf, up.view_as(loss))
        out.append((loss.detach(), g))
    return out


def _together(xs, ys, cfg, ups, node=None):
    leaves = [x.clone().requires_grad_(True) for x in xs]
    losses = ace_loss_levels(leaves, ys, cfg)
    if node is not None:
        assert losses[0].grad_fn.name().endswith(node), losses[0].grad_fn.name()
    grads = torch.autograd.grad(losses, leaves, [u.view_as(l) for u, l in zip(ups, losses)])
    return [(l.detach(), g) for l, g in zip(losses, grads)]


def _twice(xs, ys, cfg, ups):
    """The first call (Python Function) and a second one (C++ node)."""
    first = _together(xs, ys, cfg, ups)
    second = _together(xs, ys, cfg, ups, node="AceLevelsBackward")
    return first, second


SIZES = [(32, 32, 32), (16, 16, 16), (8, 8, 8), (4, 4, 4)]


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("c,kw", [
    (4, {}),
    (4, {"reduction": "sum"}),
    (4, {"reduction": "none", "include_background": False}),
    (2, {"num_bins": 7, "right": True}),
    (3, {"weight": [0.5, 2.0, 1.0]}),
    (16, {}),
])
def test_levels_match_separate_calls(binning, c, kw) -> None:
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax", **kw)
    xs, ys = _levels(2, c, SIZES, seed=51 + c)
    cl = c - (0 if cfg.include_background else 1)
    gen = torch.Generator().manual_seed(7)
    ups = [torch.rand((2, cl) if cfg.reduction == "none" else (), generator=gen).cuda() + 0.5
           for _ in SIZES]
    say(f"levels {binning} C={c} {kw}")
    want = _separate(xs, ys, cfg, ups)
    for got in _twice(xs, ys, cfg, ups):
        for (lw, gw), (lg, gg) in zip(want, got):
            assert torch.equal(lg, lw)
            assert torch.equal(gg, gw)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_levels_with_an_empty_level_and_two_levels(binning) -> None:
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    for sizes in ([(24, 20, 16), (0, 5)], [(9, 7, 5)]):
        xs, ys = _levels(3, 4, sizes, seed=61)
        ups = [torch.ones(()).cuda() for _ in sizes]
        say(f"levels {binning} {sizes}")
        want = _separate(xs, ys, cfg, ups)
        for got in _twice(xs, ys, cfg, ups):
            for (lw, gw), (lg, gg) in zip(want, got):
                torch.testing.assert_close(lg, lw, rtol=0, atol=0, equal_nan=True)
                assert torch.equal(gg, gw)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_levels_gradient_of_one_level_only(binning) -> None:
    """Only the first level's loss reaches the gradient: the other levels'
    upstream gradients are zero (the node fills them), and inputs that need
    no gradient get none."""
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    xs, ys = _levels(2, 4, SIZES[:3], seed=71)
    ups = [torch.ones(()).cuda() for _ in SIZES[:3]]
    want0 = _separate(xs[:1], ys[:1], cfg, ups[:1])[0][1]
    for _ in range(2):
        leaves = [x.clone().requires_grad_(i != 2) for i, x in enumerate(xs)]
        losses = ace_loss_levels(leaves, ys, cfg)
        grads = torch.autograd.grad(losses[0], leaves[:2])
        assert torch.equal(grads[0], want0)
        assert not grads[1].any()
    assert losses[0].grad_fn.name() == "AceLevelsBackward"


def test_levels_reject_configurations_without_a_fast_kernel() -> None:
    xs, ys = _levels(2, 5, [(8, 8, 8), (4, 4, 4)], seed=3)
    cfg = ACEConfig(binning="hard", to_onehot_y=True, activation="softmax")
    say("levels: C=5 rejected")
    with pytest.raises(Exception, match="unsupported"):
        ace_loss_levels(xs, ys, cfg)
    xs, ys = _levels(2, 4, [(8, 8, 8)], seed=3)
    with pytest.raises(ValueError):
        ace_loss_levels(xs, ys, ACEConfig(binning="hard", to_onehot_y=True, activation="sigmoid"))


def _oracle_levels(xs_cpu, ys_cpu, cfg):
    """Per level: the float32 CPU reference's (loss, grad) and the float64
    v2 restatement's (loss, grad) of one loss call per level."""
    from oracle.reference import register_reference
    from oracle.v2 import register_v2

    register_reference()
    register_v2()
    out = []
    for x, y in zip(xs_cpu, ys_cpu):
        leaf = x.clone().requires_grad_(True)
        loss = ace_loss(leaf, y, cfg, impl="reference")
        (g,) = torch.autograd.grad(loss.sum(), leaf)
        leaf64 = x.double().requires_grad_(True)
        loss64 = ace_loss(leaf64, y, cfg, impl="v2_recompute")
        (g64,) = torch.autograd.grad(loss64.sum(), leaf64)
        out.append((loss.detach(), g, loss64.detach(), g64))
    return out


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("shape", ["ds", "b2"])
def test_levels_against_the_oracle(binning, shape) -> None:
    """ace_loss_levels against the CPU reference and a float64 truth: the
    deep-supervision levels of the benchmark (128^3 ... 16^3, B = 1, the
    distribution of configuration 2) and a B = 2 set of levels.  Loss within
    rtol 1e-5 of the reference and no further from the truth than twice the
    reference's own distance; gradients element by element within rtol 1e-4
    / atol 1e-7 outside the reference's near-boundary exemption."""
    from ace_kernels.measure import rel_err
    from ace_kernels.workloads import deep_supervision
    from gpu_helpers import assert_grad_close

    if shape == "ds":
        levels = deep_supervision(binning)
        data = [wl.make("cpu") for wl in levels]
        xs_cpu = [d[0] for d in data]
        ys_cpu = [d[1] for d in data]
        cfg = levels[0].config
    else:
        cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
        gen = torch.Generator().manual_seed(1234)
        xs_cpu, ys_cpu = [], []
        for s in (48, 24, 12, 6):
            xs_cpu.append(torch.randn((2, 4, s, s, s), generator=gen) * 1.5)
            ys_cpu.append(torch.randint(0, 4, (2, 1, s, s, s), generator=gen))
    say(f"levels vs oracle {binning} {shape}: HIP")
    ups = [torch.ones(()).cuda() for _ in xs_cpu]
    got = _together([x.cuda() for x in xs_cpu], [y.cuda() for y in ys_cpu], cfg, ups)
    say(f"levels vs oracle {binning} {shape}: CPU reference and float64 truth")
    want = _oracle_levels(xs_cpu, ys_cpu, cfg)
    for lvl, ((loss, grad), (loss_ref, grad_ref, loss64, grad64), x) in enumerate(
            zip(got, want, xs_cpu)):
        loss, grad = loss.cpu(), grad.cpu()
        e_ref = rel_err(loss, loss_ref)
        e64, e64_ref = rel_err(loss, loss64), rel_err(loss_ref, loss64)
        say(f"  level {lvl} {tuple(x.shape)}: loss vs ref {e_ref:.2e}, vs f64 {e64:.2e} "
            f"(ref {e64_ref:.2e})")
        assert e_ref < 1e-5
        assert e64 <= max(2 * e64_ref, 1e-6)
        assert_grad_close(grad, grad_ref, x, cfg, truth=grad64)
