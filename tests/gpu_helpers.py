"""Shared helpers of the GPU tests: running the HIP impl and the oracle."""

from __future__ import annotations

import sys
import warnings

import numpy as np
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels.impls import hip_mi355x as hip

LOSS_RTOL, LOSS_ATOL = 1e-5, 1e-6
GRAD_RTOL, GRAD_ATOL = 1e-4, 1e-7


def say(msg: str) -> None:
    """Name the case on stdout before a GPU step (a fault ends the run)."""
    print(msg, flush=True)
    sys.stdout.flush()


def run(impl: str, x: torch.Tensor, y: torch.Tensor, config: ACEConfig, upstream=None):
    leaf = x.detach().clone().requires_grad_(True)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", UserWarning)
        loss = ace_loss(leaf, y, config, impl=impl)
    go = torch.ones_like(loss) if upstream is None else upstream.to(loss.device).view_as(loss)
    (grad,) = torch.autograd.grad(loss, leaf, go)
    return loss.detach(), grad


_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}  # ACE_F32, ACE_BF16, ACE_F16


def kernel_probs(x: torch.Tensor, config: ACEConfig) -> torch.Tensor:
    """The kernels' own float32 probabilities of logits x, on the CPU:
    ``ace_probabilities`` runs the activation that every forward and backward
    kernel applies (softmax: max, exp, the sum in channel order, the IEEE
    quotient; it differs from torch's CPU softmax by an ulp on a few per cent
    of the probabilities)."""
    from ace_kernels import _lib

    xc = x.detach().cuda().contiguous()
    c = xc.shape[1]
    act = {"softmax": _lib.ACT_SOFTMAX if c > 1 else _lib.ACT_NONE,
           "sigmoid": _lib.ACT_SIGMOID}.get(config.activation, _lib.ACT_NONE)
    p = torch.empty(xc.shape, dtype=torch.float32, device=xc.device)
    n = xc[0, 0].numel()
    rc = _lib.lib().ace_probabilities(xc.data_ptr(), _DTYPES[xc.dtype], xc.shape[0], c, n, act,
                                      p.data_ptr(), hip._stream(xc.device))
    _lib.check(rc, "ace_probabilities")
    return p.cpu()


def truth64(x: torch.Tensor, y: torch.Tensor, config: ACEConfig, upstream=None):
    """(loss, grad) in float64 throughout: the oracle's v2 path (the
    handwritten gradient of ``impls/v2_autograd.py``) on float64 logits on
    the CPU.  The reference loss itself is no float64 result on float64
    logits: it casts the probabilities to float32 before binning
    (``hardl1ace.py:84-85``, ``softl1ace.py:84-85``), so its sums and its
    autograd backward run in float32."""
    from oracle.v2 import register_v2

    register_v2()
    return run("v2_recompute", x.detach().cpu().double(), y.detach().cpu(), config, upstream)


def hip_stats(x: torch.Tensor, y: torch.Tensor, config: ACEConfig):
    """(loss, coef, d, jac, per_class, stats[3,B,C',K] float64) of one forward."""
    pl = hip.make_plan(x, y, config)
    return hip.hip_forward(pl, config, stats=True)


def cpu_probs(x: torch.Tensor, config: ACEConfig) -> torch.Tensor:
    """Probabilities as the reference computes them (torch on the CPU)."""
    x = x.detach().cpu().float()
    if config.activation == "sigmoid":
        return torch.sigmoid(x)
    if config.activation == "softmax" and x.shape[1] > 1:
        return torch.softmax(x, 1)
    return x


def onehot_np(y: torch.Tensor, channels: int, config: ACEConfig) -> np.ndarray:
    y = y.detach().cpu()
    if config.to_onehot_y and channels > 1:
        lab = y.reshape(y.shape[0], -1).numpy()
        return np.stack([(lab == c).astype(np.float64) for c in range(channels)], 1)
    return y.reshape(y.shape[0], channels, -1).double().numpy()


def near_boundary_voxels(x: torch.Tensor, config: ACEConfig, window: float = 1e-6) -> torch.Tensor:
    """[B, N] bool: some channel's probability lies within ``window`` of a
    boundary where its bin assignment changes (hard: upper bin edges; soft:
    the half boundaries, centres included, where the two bins of a voxel and
    the sign of a weight's derivative change) -- the reference's criterion
    (tests/test_triton.py:250-261)."""
    from oracle import v2

    p = cpu_probs(x, config).flatten(2)
    if config.binning == "hard":
        bounds = v2.hard_edges(config.num_bins)
    else:
        bounds = v2.soft_half_boundaries(config.num_bins)[1:]
    dist = (p.unsqueeze(-1) - bounds).abs().amin(-1)
    return (dist < window).any(1)


def assert_grad_close(grad: torch.Tensor, grad_ref: torch.Tensor, x: torch.Tensor,
                      config: ACEConfig, rtol: float = GRAD_RTOL, atol: float = GRAD_ATOL,
                      truth: torch.Tensor = None) -> torch.Tensor:
    """Gradients equal to (rtol, atol) except at voxels whose probability is
    within 1e-6 of a bin boundary, and those rare (at most one voxel or 1e-3
    of them): a one-ulp difference between the kernel's softmax and torch's
    can put such a voxel on the other side (the reference's own rule,
    tests/test_triton.py:264-296).  With ``truth`` (the float64 result), an
    element also passes when it is at least as close to it as the float32
    reference (to rtol, atol): elements that are small differences of large
    terms carry the reference's own rounding.  Returns the [B, N] mask of
    voxels that differ."""
    g = grad.detach().cpu().float().flatten(2)
    r = grad_ref.detach().cpu().float().flatten(2)
    ok = torch.isclose(g, r, rtol=rtol, atol=atol)
    if truth is not None:
        t = truth.detach().cpu().double().flatten(2)
        err = (g.double() - t).abs()
        ok |= err <= (r.double() - t).abs() + rtol * t.abs() + atol
    bad = (~ok).any(1)
    if bad.any():
        near = near_boundary_voxels(x, config)
        far = bad & ~near
        assert not far.any(), (
            f"gradient differs away from bin boundaries at {far.nonzero()[:4].tolist()}: "
            f"max |diff| {float((g - r).abs().max()):.3e}"
        )
        assert int(bad.sum()) <= max(1, int(1e-3 * bad.numel())), f"{int(bad.sum())} boundary voxels differ"
    return bad


def assert_lowp_grad_close(grad: torch.Tensor, grad_ref: torch.Tensor, x: torch.Tensor,
                           config: ACEConfig, atol: float = GRAD_ATOL,
                           truth: torch.Tensor = None, own: torch.Tensor = None) -> torch.Tensor:
    """dx in bfloat16 / float16 (the logits' type): every element within one
    unit in the last place of the reference's float32 gradient rounded to
    that type, plus the north star's atol -- both sides round a float32 value
    to nearest even, so they differ by a unit only where the two float32
    values straddle a rounding boundary, and by more only in elements that
    are small differences of large terms, which atol covers -- except at
    voxels whose probability is within 1e-6 of a bin boundary, and those
    rare (the rule of ``assert_grad_close``).  With ``truth`` (the float64
    gradient) an element also passes when it is at least as close to the
    truth, rounded to the same type, as the reference is.  With ``own`` (the
    float64 gradient at the kernels' own float32 probabilities) an element
    also passes within one unit of it rounded to the same type: in bins of a
    few soft voxels the gradient follows the probabilities' last bit, where
    the kernels' correctly rounded softmax and torch's may differ by an ulp.
    Returns the [B, N] mask of voxels that do not pass."""
    dt = grad.dtype
    assert dt in (torch.bfloat16, torch.float16), dt
    mant = 7 if dt == torch.bfloat16 else 10
    g = grad.detach().cpu().float().flatten(2)
    r = grad_ref.detach().cpu().float().to(dt).float().flatten(2)
    # the spacing of dt at |r| (the smallest normal's spacing below it)
    e = torch.floor(torch.log2(torch.clamp(r.abs(), min=torch.finfo(dt).tiny)))
    ok = (g - r).abs() <= torch.exp2(e - mant) + atol
    if truth is not None:
        t = truth.detach().cpu().double().to(dt).double().flatten(2)
        ok |= (g.double() - t).abs() <= (r.double() - t).abs()
    if own is not None:
        o = own.detach().cpu().double().to(dt).double().flatten(2)
        eo = torch.floor(torch.log2(torch.clamp(o.abs(), min=torch.finfo(dt).tiny)))
        ok |= (g.double() - o).abs() <= torch.exp2(eo - mant) + atol
    bad = (~ok).any(1)
    if bad.any():
        near = near_boundary_voxels(x, config)
        far = bad & ~near
        assert not far.any(), (
            f"{dt} gradient more than one unit from the reference away from bin boundaries at "
            f"{far.nonzero()[:4].tolist()}: max |diff| {float((g - r).abs().max()):.3e}"
        )
        assert int(bad.sum()) <= max(1, int(1e-3 * bad.numel())), f"{int(bad.sum())} boundary voxels differ"
    return bad
