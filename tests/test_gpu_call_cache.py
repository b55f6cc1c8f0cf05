"""The remembered call signatures of ``hip_mi355x`` (``_CALLS``): a repeated
call of one signature (configuration, shapes, dtypes, devices, stream) runs
in C++ (``_ace_autograd``: the forward launch and a C++ backward node) and
must give bit-identical results to the general path (``make_plan`` +
``hip_forward`` / ``hip_backward``) on the same inputs; calls no signature
covers (converted or strided inputs, float64) take the general path; the
C++ node keeps autograd's checks (an in-place change of a saved input, a
second backward through a freed graph)."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels.impls import hip_mi355x as hip
from ace_kernels.impls.hip_mi355x import _CALLS
from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _inputs(b=2, c=4, spatial=(9, 33), dtype=torch.float32, seed=0):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn((b, c, *spatial), generator=gen) * 2).to(dtype)
    y = torch.randint(0, c, (b, 1, *spatial), generator=gen)
    return x.cuda(), y.cuda()


def _general(x, y, cfg):
    """(loss, grad) from the general path: a fresh Plan each call."""
    pl = hip.make_plan(x, y, cfg)
    loss, coef, d, jac, _, _ = hip.hip_forward(pl, cfg)
    go = torch.ones_like(loss)
    dx = hip.hip_backward(pl, coef, d, jac, go)
    return loss, dx


def _cached(x, y, cfg):
    leaf = x.detach().clone().requires_grad_(True)
    loss = ace_loss(leaf, y, cfg, impl="hip_mi355x")
    (g,) = torch.autograd.grad(loss, leaf, torch.ones_like(loss))
    return loss.detach(), g


CONFIGS = [
    dict(binning="hard", num_bins=20),
    dict(binning="soft", num_bins=20),
    dict(binning="hard", num_bins=7, reduction="none", include_background=False),
    dict(binning="soft", num_bins=33, reduction="sum", weight=(0.5, 1.0, 2.0, 1.5), right=True),
    dict(binning="soft", num_bins=12, reduction="none"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kw", CONFIGS, ids=lambda kw: "-".join(f"{k}={v}" for k, v in kw.items()))
def test_cached_calls_match_general_path(kw, dtype) -> None:
    cfg = ACEConfig(to_onehot_y=True, activation="softmax", **kw)
    say(f"call cache: {kw} {dtype}")
    x, y = _inputs(dtype=dtype)
    want_loss, want_grad = _general(x, y, cfg)
    for i in range(3):  # the first call is remembered, the rest run in C++
        loss, g = _cached(x, y, cfg)
        assert torch.equal(loss, want_loss.view_as(loss)), i
        assert torch.equal(g, want_grad), i
    leaf = x.detach().clone().requires_grad_(True)
    assert ace_loss(leaf, y, cfg, impl="hip_mi355x").grad_fn.name() == "AceLossBackward"
    key_cfgs = [k[0] for k, v in _CALLS.items() if v is not None]
    assert cfg in key_cfgs
    # an equal configuration built anew hits the same entry
    n = len(_CALLS)
    loss, g = _cached(x, y, ACEConfig(**cfg.model_dump()))
    assert len(_CALLS) == n
    assert torch.equal(g, want_grad)


def test_no_grad_forward_matches() -> None:
    cfg = ACEConfig(binning="soft", num_bins=20, to_onehot_y=True)
    x, y = _inputs(seed=3)
    want = _general(x, y, cfg)[0]
    for _ in range(2):
        with torch.no_grad():
            assert torch.equal(ace_loss(x, y, cfg, impl="hip_mi355x"), want)
        assert torch.equal(ace_loss(x, y, cfg, impl="hip_mi355x"), want)  # needs no grad


def test_strided_and_converted_inputs_take_the_general_path() -> None:
    cfg = ACEConfig(binning="hard", num_bins=20, to_onehot_y=True)
    x, y = _inputs(spatial=(16, 16), seed=5)
    want_loss, want_grad = _cached(x, y, cfg)
    # the same signature with a transposed (non-contiguous) input
    xt = x.transpose(2, 3).contiguous().transpose(2, 3)
    assert not xt.is_contiguous()
    loss, g = _cached(xt, y, cfg)
    assert torch.equal(loss, want_loss) and torch.equal(g, want_grad)
    # int32 labels are converted: never cached
    loss, g = _cached(x, y.int(), cfg)
    assert torch.equal(loss, want_loss) and torch.equal(g, want_grad)
    key = (cfg, x.shape, x.dtype, y.shape, torch.int32, x.get_device(), y.get_device(),
           hip._stream(x.device))
    assert key in _CALLS and _CALLS[key] is None


def test_other_stream_has_its_own_entry() -> None:
    cfg = ACEConfig(binning="soft", num_bins=20, to_onehot_y=True)
    x, y = _inputs(seed=7)
    want_loss, want_grad = _cached(x, y, cfg)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            loss, g = _cached(x, y, cfg)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(loss, want_loss) and torch.equal(g, want_grad)
    streams = {k[-1] for k in _CALLS if k[0] == cfg and k[1] == x.shape}
    assert len(streams) >= 2


def test_in_place_change_of_saved_input_is_detected() -> None:
    cfg = ACEConfig(binning="soft", num_bins=20, to_onehot_y=True)
    x, y = _inputs(seed=9)
    _cached(x, y, cfg)
    leaf = x.detach().clone().requires_grad_(True)
    z = leaf * 1.0
    loss = ace_loss(z, y, cfg, impl="hip_mi355x")
    z.add_(1.0)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        torch.autograd.grad(loss, leaf)


def test_float64_takes_its_own_entry_points() -> None:
    cfg = ACEConfig(binning="soft", num_bins=10, to_onehot_y=True)
    x, y = _inputs(dtype=torch.float64, seed=11)
    first = _cached(x, y, cfg)
    second = _cached(x, y, cfg)
    assert first[0].dtype == torch.float64
    assert torch.equal(first[0], second[0]) and torch.equal(first[1], second[1])


def test_backward_twice_and_retain_graph() -> None:
    cfg = ACEConfig(binning="soft", num_bins=20, to_onehot_y=True)
    x, y = _inputs(seed=13)
    want = _general(x, y, cfg)[1]
    _cached(x, y, cfg)
    leaf = x.detach().clone().requires_grad_(True)
    loss = ace_loss(leaf, y, cfg, impl="hip_mi355x")
    assert loss.grad_fn.name() == "AceLossBackward"
    loss.backward(retain_graph=True)
    loss.backward()  # accumulates a second time
    assert torch.equal(leaf.grad, want + want)
    with pytest.raises(RuntimeError, match="backward through the graph a second time"):
        loss.backward()


def test_upstream_gradient_through_the_node() -> None:
    """reduction "none" with a strided upstream gradient (the sum's expand) and
    a scaled scalar one."""
    for kw in (dict(reduction="none"), dict(reduction="mean")):
        cfg = ACEConfig(binning="hard", num_bins=20, to_onehot_y=True, **kw)
        x, y = _inputs(seed=17)
        pl = hip.make_plan(x, y, cfg)
        loss, coef, d, jac, _, _ = hip.hip_forward(pl, cfg)
        up = torch.full_like(loss, 3.0)
        want = hip.hip_backward(pl, coef, d, jac, up)
        for _ in range(2):
            leaf = x.detach().clone().requires_grad_(True)
            out = ace_loss(leaf, y, cfg, impl="hip_mi355x")
            (3.0 * out).sum().backward()
            assert torch.equal(leaf.grad, want)


def test_target_that_needs_a_gradient_gets_none() -> None:
    """A float one-hot target that requires grad: the loss records autograd
    history even when the input needs no gradient, and the target's gradient
    is None, as from the reference's autograd Function
    (``impls/v6_triton.py:107-111``); with an input that needs one, the
    input's gradient is the usual one."""
    cfg = ACEConfig(binning="soft", num_bins=20, to_onehot_y=False)
    gen = torch.Generator().manual_seed(21)
    x = (torch.randn((2, 4, 9, 33), generator=gen) * 2).cuda()
    lab = torch.randint(0, 4, (2, 9, 33), generator=gen)
    y = torch.nn.functional.one_hot(lab, 4).permute(0, 3, 1, 2).float().cuda()
    want = _general(x, y, cfg)[1]
    for _ in range(3):  # the signature is remembered after the first call
        t = y.clone().requires_grad_(True)
        loss = ace_loss(x, t, cfg, impl="hip_mi355x")
        assert loss.requires_grad
        loss.backward()
        assert t.grad is None
        leaf = x.clone().requires_grad_(True)
        t = y.clone().requires_grad_(True)
        loss = ace_loss(leaf, t, cfg, impl="hip_mi355x")
        loss.backward()
        assert t.grad is None and torch.equal(leaf.grad, want)


def test_soft_d_without_its_remainder() -> None:
    """The soft forward's d is [2, B, C', K]: its float32 rounding and the
    remainder, which the backward adds.  A plain [B, C', K] float32 d (no
    remainder) gives the same gradient as the two-part d with a zero
    remainder, within float32 rounding of the full one; a d of any other
    size is refused before a launch."""
    cfg = ACEConfig(binning="soft", num_bins=20, to_onehot_y=True)
    x, y = _inputs(seed=23)
    pl = hip.make_plan(x, y, cfg)
    loss, coef, d, jac, _, _ = hip.hip_forward(pl, cfg)
    assert d.shape == (2, pl.B, pl.CL, pl.K)
    go = torch.ones_like(loss)
    full = hip.hip_backward(pl, coef, d, jac, go)
    plain = hip.hip_backward(pl, coef, d[0].clone(), jac, go)
    zero_lo = torch.stack([d[0], torch.zeros_like(d[0])]).contiguous()
    assert torch.equal(plain, hip.hip_backward(pl, coef, zero_lo, jac, go))
    torch.testing.assert_close(plain, full, rtol=1e-4, atol=1e-7)
    with pytest.raises(ValueError, match="d must be"):
        hip.hip_backward(pl, coef, d[:, :1].contiguous(), jac, go)
