"""Vectorised per-bin statistics and the handwritten ("v2") backward (TEST ORACLE).

Restates, in torch (float32 or float64, any device):

- input handling ``prepare`` / ``activate``: ``src/ace_kernels/common.py:85-140``
- class weights / reduction: ``common.py:162-207``
- soft assignment: ``common.py:43-61``
- per-bin sums W, P, G: ``src/ace_kernels/binning.py:54-124``
- class presence, d = P/W - G/W, per-bin error: ``binning.py:127-147``
- ``coefficients`` (coef = sign(d) / (K_ne W)): ``impls/v2_autograd.py:66-76``
- dL/dp: ``v2_autograd.py:88-104``; activation backward ``:107-118``;
  reduction jacobian ``:138-151``; the autograd.Function ``:196-236``
- the mathematics: ``docs/derivation.md:22-84``

It is the float64 ground truth for gradients (pinned by ``gradcheck``) and the
oracle the GPU backward is compared against.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

EPS32 = torch.finfo(torch.float32).eps


# ---------------------------------------------------------------- tables

def hard_edges(num_bins: int) -> torch.Tensor:
    """Upper bin edges: float32 ``linspace(0, 1 + eps32, K + 1)[1:]`` (common.py:17-20)."""
    return torch.linspace(0.0, 1.0 + EPS32, num_bins + 1)[1:]


def soft_half_boundaries(num_bins: int) -> torch.Tensor:
    """Centres and edges interleaved: ``linspace(0, 1 + eps32, 2K + 1)`` (common.py:23-25)."""
    return torch.linspace(0.0, 1.0 + EPS32, 2 * num_bins + 1)


# ---------------------------------------------------------------- prepare

@dataclass
class Prepared:
    probs: torch.Tensor  # [B, C', N]
    onehot: Optional[torch.Tensor]  # [B, C', N] or None
    labels: Optional[torch.Tensor]  # [B, N] shifted (-1: no loss channel) or None
    spatial_ndim: int


def compute_dtype(x: torch.Tensor) -> torch.dtype:
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def activate(x: torch.Tensor, activation: str) -> torch.Tensor:
    if activation == "sigmoid":
        return torch.sigmoid(x)
    if activation == "softmax" and x.shape[1] > 1:
        return torch.softmax(x, 1)
    return x


def prepare(input: torch.Tensor, target: torch.Tensor, config) -> Prepared:
    """Activation, label / one-hot handling and background removal (common.py:93-140)."""
    if input.dim() < 3:
        raise ValueError(f"input must be [B, C, *spatial], got {tuple(input.shape)}")
    probs = activate(input, config.activation)
    dtype = compute_dtype(input)
    n_ch = input.shape[1]
    drop_bg = not config.include_background and n_ch > 1
    if config.to_onehot_y and n_ch > 1:
        labels = target.reshape(target.shape[0], -1).long()
        if drop_bg:
            labels = labels - 1
            probs = probs[:, 1:]
        if labels.shape[-1] != probs[0, 0].numel():
            raise AssertionError("target and input spatial sizes differ")
        return Prepared(probs.flatten(2).to(dtype), None, labels, input.dim() - 2)
    onehot = target.to(dtype)
    if drop_bg:
        probs, onehot = probs[:, 1:], onehot[:, 1:]
    if onehot.shape != probs.shape:
        raise AssertionError(
            f"ground truth has different shape ({tuple(onehot.shape)}) from input "
            f"({tuple(probs.shape)})"
        )
    return Prepared(probs.flatten(2).to(dtype), onehot.flatten(2), None, input.dim() - 2)


def true_target(prep: Prepared) -> torch.Tensor:
    """``[B, C', N]`` y in the probabilities' dtype."""
    if prep.onehot is not None:
        return prep.onehot
    channels = torch.arange(prep.probs.shape[1], device=prep.probs.device)
    return (prep.labels.unsqueeze(1) == channels.view(1, -1, 1)).to(prep.probs.dtype)


# ---------------------------------------------------------------- binning

@dataclass
class SoftAssignment:
    left_idx: torch.Tensor
    right_idx: torch.Tensor
    left_w: torch.Tensor
    right_w: torch.Tensor
    span: torch.Tensor


def soft_assign(p: torch.Tensor, num_bins: int, right: bool) -> SoftAssignment:
    """Two neighbouring bins and interpolation weights (common.py:43-61)."""
    half = soft_half_boundaries(num_bins).to(device=p.device, dtype=p.dtype)
    h = torch.bucketize(p, half[1:], right=right)
    left = torch.clamp(h - 1, min=0) // 2
    rght = torch.clamp(h + 1, max=2 * num_bins - 1) // 2
    sentinel = half.new_full((1,), 10000.0)
    repl = torch.cat((-sentinel, half[1::2].repeat_interleave(2), sentinel))
    ld = p - repl[h]
    rd = repl[h + 2] - p
    span = ld + rd
    return SoftAssignment(left, rght, rd / span, ld / span, span)


def hard_bin_index(p: torch.Tensor, config) -> torch.Tensor:
    edges = hard_edges(config.num_bins).to(device=p.device, dtype=p.dtype)
    return torch.bucketize(p, edges, right=config.right)


@dataclass
class BinStats:
    weight: torch.Tensor  # W [B, C', K]
    sum_p: torch.Tensor  # P
    sum_gt: torch.Tensor  # G
    empty: torch.Tensor


def _rows(p: torch.Tensor) -> torch.Tensor:
    b, c = p.shape[:2]
    return torch.arange(b * c, device=p.device).view(b, c, 1)


def _true_class(prep: Prepared):
    b, c = prep.probs.shape[:2]
    valid = (prep.labels >= 0).unsqueeze(1).to(prep.probs.dtype)
    channel = prep.labels.clamp_min(0).unsqueeze(1)
    batch = torch.arange(b, device=channel.device).view(b, 1, 1)
    return channel, batch * c + channel, valid


def hard_stats(prep: Prepared, config) -> BinStats:
    """binning.py:54-71: one flat scatter_add per statistic."""
    p = prep.probs
    b, c, _ = p.shape
    k = config.num_bins
    idx = hard_bin_index(p, config)
    flat = (idx + _rows(p) * k).flatten()
    zeros = p.new_zeros(b * c * k)
    counts = zeros.scatter_add(0, flat, p.new_ones(()).expand(flat.shape))
    sum_p = zeros.scatter_add(0, flat, p.flatten())
    if prep.onehot is not None:
        sum_gt = zeros.scatter_add(0, flat, prep.onehot.flatten())
    else:
        channel, row, valid = _true_class(prep)
        true_idx = idx.gather(1, channel)
        sum_gt = zeros.scatter_add(0, (true_idx + row * k).flatten(), valid.flatten())
    shape = (b, c, k)
    counts = counts.view(shape)
    return BinStats(counts, sum_p.view(shape), sum_gt.view(shape), counts == 0)


def soft_stats(prep: Prepared, config) -> BinStats:
    """binning.py:74-116: left and right contributions scattered separately."""
    p = prep.probs
    b, c, _ = p.shape
    k = config.num_bins
    a = soft_assign(p, k, config.right)
    offsets = _rows(p) * k
    left = (a.left_idx + offsets).flatten()
    rght = (a.right_idx + offsets).flatten()
    zeros = p.new_zeros(b * c * k)

    def scatter(il, vl, ir, vr):
        return zeros.scatter_add(0, il, vl).scatter_add(0, ir, vr)

    weights = scatter(left, a.left_w.flatten(), rght, a.right_w.flatten())
    sum_p = scatter(left, (a.left_w * p).flatten(), rght, (a.right_w * p).flatten())
    if prep.onehot is not None:
        y = prep.onehot
        sum_gt = scatter(left, (a.left_w * y).flatten(), rght, (a.right_w * y).flatten())
    else:
        channel, row, valid = _true_class(prep)
        sum_gt = scatter(
            (a.left_idx.gather(1, channel) + row * k).flatten(),
            (a.left_w.gather(1, channel) * valid).flatten(),
            (a.right_idx.gather(1, channel) + row * k).flatten(),
            (a.right_w.gather(1, channel) * valid).flatten(),
        )
    shape = (b, c, k)
    weights = weights.view(shape)
    return BinStats(weights, sum_p.view(shape), sum_gt.view(shape), weights < config.empty_weight)


def bin_stats(prep: Prepared, config) -> BinStats:
    return hard_stats(prep, config) if config.binning == "hard" else soft_stats(prep, config)


def class_present(stats: BinStats) -> torch.Tensor:
    return stats.sum_gt.sum(-1) > 0


def bin_difference(stats: BinStats) -> torch.Tensor:
    safe = torch.where(stats.empty, torch.ones_like(stats.weight), stats.weight)
    diff = stats.sum_p / safe - stats.sum_gt / safe
    return torch.where(stats.empty, torch.zeros_like(diff), diff)


def per_bin_error(stats: BinStats) -> torch.Tensor:
    error = bin_difference(stats).abs()
    return torch.where(stats.empty, torch.full_like(error, torch.nan), error)


def coefficients(stats: BinStats):
    """(f [B,C'], present [B,C'], coef [B,C',K], d [B,C',K]) (v2_autograd.py:66-76)."""
    d = bin_difference(stats)
    f = torch.nanmean(per_bin_error(stats), dim=-1)
    nonempty = ~stats.empty
    k_ne = nonempty.sum(-1, keepdim=True).clamp_min(1).to(d.dtype)
    safe_w = torch.where(nonempty, stats.weight, torch.ones_like(stats.weight))
    coef = torch.where(nonempty, torch.sign(d) / (k_ne * safe_w), torch.zeros_like(d))
    return f, class_present(stats), coef, d


# ---------------------------------------------------------------- reduction

def class_weights(config, n_ch: int) -> Optional[List[float]]:
    """common.py:162-181."""
    if config.weight is None or n_ch == 1:
        return None
    weights = [config.weight] * n_ch if isinstance(config.weight, float) else list(config.weight)
    if len(weights) != n_ch:
        raise ValueError(
            "the length of the `weight` sequence should be the same as the number of classes"
        )
    if min(weights) < 0:
        raise ValueError("the value/values of the `weight` should be no less than 0.")
    return weights


def reduce_classes(f: torch.Tensor, spatial_ndim: int, config, present: torch.Tensor) -> torch.Tensor:
    """common.py:184-207 with ``present`` from the bin statistics."""
    if config.ignore_empty_classes:
        f = f * present.to(f.dtype)
    weights = class_weights(config, f.shape[1])
    if weights is not None:
        f = torch.cat([f[:, i : i + 1] * w for i, w in enumerate(weights)], dim=1)
    if config.reduction == "mean":
        return f.mean()
    if config.reduction == "sum":
        return f.sum()
    return f.view(*f.shape[:2], *([1] * spatial_ndim))


def reduction_jacobian(f: torch.Tensor, spatial_ndim: int, config, present: torch.Tensor) -> torch.Tensor:
    """d(sum of loss outputs)/d f  [B, C'] (v2_autograd.py:138-151)."""
    with torch.enable_grad():
        f_var = torch.zeros_like(f, requires_grad=True)
        out = reduce_classes(f_var, spatial_ndim, config, present)
        (jac,) = torch.autograd.grad(out.sum(), f_var)
    return jac


# ---------------------------------------------------------------- backward

def df_dprobs(prep: Prepared, coef: torch.Tensor, d: torch.Tensor, config) -> torch.Tensor:
    """``[B, C', N]`` d f_bc / d p_bci (v2_autograd.py:88-104, derivation.md:57-73)."""
    if config.binning == "hard":
        return coef.gather(2, hard_bin_index(prep.probs, config))
    p = prep.probs
    a = soft_assign(p, config.num_bins, config.right)
    inv_span = 1.0 / a.span
    resid = p - true_target(prep)
    left = coef.gather(2, a.left_idx) * (a.left_w - inv_span * (resid - d.gather(2, a.left_idx)))
    rght = coef.gather(2, a.right_idx) * (a.right_w + inv_span * (resid - d.gather(2, a.right_idx)))
    return left + rght


def activation_backward(input: torch.Tensor, grad_probs: torch.Tensor, activation: str) -> torch.Tensor:
    """v2_autograd.py:107-118."""
    dtype = compute_dtype(input)
    if activation == "sigmoid":
        p = torch.sigmoid(input).to(dtype)
        return grad_probs * p * (1 - p)
    if activation == "softmax" and input.shape[1] > 1:
        p = torch.softmax(input, 1).to(dtype)
        return p * (grad_probs - (grad_probs * p).sum(1, keepdim=True))
    return grad_probs


def forward_stats(input: torch.Tensor, target: torch.Tensor, config):
    """(loss, coef, d, jac, stats) with the reference's float semantics."""
    prep = prepare(input, target, config)
    stats = bin_stats(prep, config)
    f, present, coef, d = coefficients(stats)
    loss = reduce_classes(f, prep.spatial_ndim, config, present)
    jac = reduction_jacobian(f, prep.spatial_ndim, config, present)
    return loss, coef, d, jac, stats


def input_grad(input, target, config, coef, d, jac, grad_output) -> torch.Tensor:
    """dL/d input = activation backward of g * df/dp with g = jac * grad_output."""
    prep = prepare(input, target, config)
    g = jac * (grad_output if grad_output.dim() == 0 else grad_output.reshape(jac.shape))
    grad_p = g.unsqueeze(-1).to(coef.dtype) * df_dprobs(prep, coef, d, config)
    if grad_p.shape[1] != input.shape[1]:
        grad_p = torch.cat((torch.zeros_like(grad_p[:, :1]), grad_p), dim=1)
    grad_p = grad_p.view(input.shape)
    return activation_backward(input, grad_p, config.activation).to(input.dtype)


class _V2Loss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input, target, config):
        loss, coef, d, jac, _ = forward_stats(input.detach(), target, config)
        ctx.config = config
        ctx.save_for_backward(input, target, coef, d, jac)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        input, target, coef, d, jac = ctx.saved_tensors
        grad = input_grad(input, target, ctx.config, coef, d, jac, grad_output)
        return grad, None, None


def v2_ace(input: torch.Tensor, target: torch.Tensor, config) -> torch.Tensor:
    """Registry-style ``fn(input, target, config)`` with the handwritten backward."""
    return _V2Loss.apply(input, target, config)


def register_v2() -> None:
    from ace_kernels.registry import _REGISTRY, register

    if "v2_recompute" not in _REGISTRY:
        register("v2_recompute", description="handwritten backward, torch (oracle)")(v2_ace)
