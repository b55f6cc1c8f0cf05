"""The reference mL1-ACE loss restated on torch CPU tensors (TEST ORACLE ONLY).

Restates, step for step, the upstream loss the reference vendors and freezes:

- ``hard_binned_calibration``: ``src/ace_reference/hardl1ace.py:25-105``
- ``soft_binned_calibration``: ``src/ace_reference/softl1ace.py:25-151``
- the module forward (activation, one-hot target, background removal, empty
  class mask, class weights, reduction): ``hardl1ace.py:182-278`` and
  ``softl1ace.py:230-330`` (identical apart from the binning call)
- the registry adapter that builds a fresh module per call:
  ``src/ace_kernels/impls/reference.py:10-33``

The per-(b, c) Python loop, ``torch.bucketize`` against the float32
``torch.linspace`` edges, ``scatter_add`` / ``scatter_reduce(mean)`` and the
autograd backward are kept as in the reference, because they *are* the
algorithm being matched (its fp32 summation order included).  The monai
``one_hot`` call (``hardl1ace.py:215``) is restated as a zero tensor with a
``scatter_`` of ones along the channel axis, which is what monai 1.6.1 does.

Used as the golden-vector reproducer and as the timed CPU baseline; never by
the product.
"""

from __future__ import annotations

import warnings
from typing import Sequence, Tuple

import torch

EPS32 = torch.finfo(torch.float32).eps


def _check_shapes(input: torch.Tensor, target: torch.Tensor) -> None:
    # hardl1ace.py:61-68 / softl1ace.py:57-64
    if input.shape != target.shape:
        raise ValueError(
            f"Input and target should have the same shapes, got {input.shape} "
            f"and {target.shape}."
        )
    if input.dim() < 3:
        raise ValueError(
            "Input should be at least a three-dimensional tensor, got "
            f"{input.dim()} dimensions."
        )


def hard_binned_calibration(
    input: torch.Tensor, target: torch.Tensor, num_bins: int = 20, right: bool = False
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per (b, c, k): mean p, mean target (NaN for empty bins), count.

    Follows ``hardl1ace.py:70-105``: one bucketize per slice against the upper
    edges of ``linspace(0, 1 + eps32, K + 1)``, a scatter_add of ones for the
    counts and two scatter_reduce(mean) calls for the means.
    """
    _check_shapes(input, target)
    batch, channels = input.shape[:2]
    edges = torch.linspace(0.0, 1.0 + EPS32, num_bins + 1, device=input.device)
    upper = edges[1:]
    mean_p = torch.zeros(batch, channels, num_bins, device=input.device)
    mean_gt = torch.zeros_like(mean_p)
    counts = torch.zeros_like(mean_p)
    x = input.flatten(start_dim=2).float()
    y = target.flatten(start_dim=2).float()
    for b in range(batch):
        for c in range(channels):
            idx = torch.bucketize(x[b, c], upper, right=right)
            counts[b, c, :] = torch.zeros_like(upper).scatter_add(
                0, idx, torch.ones_like(x[b, c])
            )
            mean_p[b, c, :] = torch.empty_like(upper).scatter_reduce(
                0, idx, x[b, c], reduce="mean", include_self=False
            )
            mean_gt[b, c, :] = torch.empty_like(upper).scatter_reduce(
                0, idx, y[b, c], reduce="mean", include_self=False
            )
    mean_p[counts == 0] = torch.nan
    mean_gt[counts == 0] = torch.nan
    return mean_p, mean_gt, counts


def soft_binned_calibration(
    input: torch.Tensor,
    target: torch.Tensor,
    num_bins: int = 20,
    empty_weight: float = 0.01,
    right: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per (b, c, k): weighted mean p, weighted mean target, weight sum.

    Follows ``softl1ace.py:66-151``: half-bin index against
    ``linspace(0, 1 + eps32, 2K + 1)[1:]``; neighbouring bins ``l``, ``r``;
    distances to the replicated centres with +-10000 sentinels; weights
    ``right_dist / S`` and ``left_dist / S``; six scatter_adds; bins whose
    weight is below ``empty_weight`` are NaN.
    """
    _check_shapes(input, target)
    batch, channels = input.shape[:2]
    half_bins = 2 * num_bins
    half = torch.linspace(0.0, 1.0 + EPS32, half_bins + 1, device=input.device)
    centres = half[1::2]
    mean_p = torch.zeros(batch, channels, num_bins, device=input.device)
    mean_gt = torch.zeros_like(mean_p)
    weights = torch.zeros_like(mean_p)
    x = input.flatten(start_dim=2).float()
    y = target.flatten(start_dim=2).float()
    sentinel = torch.full((1,), 10000.0, device=input.device)
    repl = torch.cat((-sentinel, centres.repeat_interleave(2), sentinel))
    for b in range(batch):
        for c in range(channels):
            p = x[b, c]
            h = torch.bucketize(p, half[1:], right=right)
            left = torch.clamp(h - 1, min=0) // 2
            rght = torch.clamp(h + 1, max=half_bins - 1) // 2
            ld = p - repl[h]
            rd = repl[h + 2] - p
            span = ld + rd
            lw = rd / span
            rw = ld / span
            zeros = torch.zeros_like(centres)
            w_sum = zeros.scatter_add(0, left, lw) + zeros.scatter_add(0, rght, rw)
            p_sum = zeros.scatter_add(0, left, lw * p) + zeros.scatter_add(
                0, rght, rw * p
            )
            gt = y[b, c]
            g_sum = zeros.scatter_add(0, left, lw * gt) + zeros.scatter_add(
                0, rght, rw * gt
            )
            mean_p[b, c, :] = p_sum / w_sum
            mean_gt[b, c, :] = g_sum / w_sum
            weights[b, c, :] = w_sum
    mean_p[weights < empty_weight] = torch.nan
    mean_gt[weights < empty_weight] = torch.nan
    return mean_p, mean_gt, weights


def _one_hot(labels: torch.Tensor, num_classes: int) -> torch.Tensor:
    """monai ``one_hot(labels, num_classes)`` along dim 1 (float32)."""
    shape = list(labels.shape)
    if shape[1] != 1:
        raise AssertionError("labels should have a channel with length equal to one.")
    shape[1] = num_classes
    out = torch.zeros(shape, dtype=torch.float32, device=labels.device)
    return out.scatter_(1, labels.long(), 1.0)


def binned_l1ace(
    input: torch.Tensor,
    target: torch.Tensor,
    *,
    binning: str,
    num_bins: int = 20,
    include_background: bool = True,
    to_onehot_y: bool = False,
    sigmoid: bool = False,
    softmax: bool = False,
    reduction: str = "mean",
    weight: "Sequence[float] | float | None" = None,
    right: bool = False,
    ignore_empty_classes: bool = True,
    empty_weight: float = 0.01,
) -> torch.Tensor:
    """``HardL1ACELoss.forward`` / ``SoftL1ACELoss.forward`` (hardl1ace.py:182-278)."""
    if sigmoid and softmax:
        raise ValueError("Incompatible values: more than 1 of [sigmoid=True, softmax=True].")
    if sigmoid:
        input = torch.sigmoid(input)
    n_pred_ch = input.shape[1]
    if softmax:
        if n_pred_ch == 1:
            warnings.warn("single channel prediction, `softmax=True` ignored.")
        else:
            input = torch.softmax(input, 1)
    if to_onehot_y:
        if n_pred_ch == 1:
            warnings.warn("single channel prediction, `to_onehot_y=True` ignored.")
        else:
            target = _one_hot(target, n_pred_ch)
    if not include_background:
        if n_pred_ch == 1:
            warnings.warn("single channel prediction, `include_background=False` ignored.")
        else:
            target = target[:, 1:]
            input = input[:, 1:]
    if target.shape != input.shape:
        raise AssertionError(
            f"ground truth has different shape ({target.shape}) from input ({input.shape})"
        )
    if binning == "hard":
        mean_p, mean_gt, _ = hard_binned_calibration(input, target, num_bins, right)
    else:
        mean_p, mean_gt, _ = soft_binned_calibration(
            input, target, num_bins, empty_weight, right
        )
    f = torch.nanmean(torch.abs(mean_p - mean_gt), dim=-1)
    if ignore_empty_classes:
        non_empty = target.sum(dim=list(range(2, target.dim()))) > 0
        f = f * non_empty.float()
    num_classes = target.shape[1]
    if weight is not None and num_classes != 1:
        w = torch.as_tensor(weight)
        if w.ndim == 0:
            w = torch.as_tensor([float(w)] * num_classes)
        elif w.shape[0] != num_classes:
            raise ValueError(
                "the length of the `weight` sequence should be the same as the number of classes."
            )
        if w.min() < 0:
            raise ValueError("the value/values of the `weight` should be no less than 0.")
        f = f * w.to(f)
    if reduction == "mean":
        return torch.mean(f)
    if reduction == "sum":
        return torch.sum(f)
    if reduction == "none":
        return f.view(list(f.shape[0:2]) + [1] * (input.dim() - 2))
    raise ValueError(f"Unsupported reduction: {reduction}")


def reference_ace(input: torch.Tensor, target: torch.Tensor, config) -> torch.Tensor:
    """Registry-style entry ``fn(input, target, config)`` (impls/reference.py:10-33)."""
    weight = list(config.weight) if isinstance(config.weight, tuple) else config.weight
    return binned_l1ace(
        input,
        target,
        binning=config.binning,
        num_bins=config.num_bins,
        include_background=config.include_background,
        to_onehot_y=config.to_onehot_y,
        sigmoid=config.activation == "sigmoid",
        softmax=config.activation == "softmax",
        reduction=config.reduction,
        weight=weight,
        right=config.right,
        ignore_empty_classes=config.ignore_empty_classes,
        empty_weight=config.empty_weight,
    )


def register_reference() -> None:
    """Register ``reference_ace`` as impl ``"reference"`` (cpu and cuda tensors)."""
    from ace_kernels.registry import _REGISTRY, register

    if "reference" not in _REGISTRY:
        register(
            "reference",
            description="Reference loss restated on torch (B x C loop, autograd)",
        )(reference_ace)
