"""Independent float64 NumPy restatement of mL1-ACE (TEST ORACLE ONLY).

Written from the mathematics (``docs/derivation.md:6-34``, restated after the
reference's own independent oracle ``tests/oracle.py:26-96``): per (b, c) slice
with probabilities p_i, targets y_i and bin weights w_ik,

    W_k = sum_i w_ik,   P_k = sum_i w_ik p_i,   G_k = sum_i w_ik y_i,
    f   = mean over non-empty k of |P_k - G_k| / W_k.

Hard binning: w_ik = 1 for the bin holding p_i (``np.searchsorted`` against the
float32 edge table, the same as ``torch.bucketize``).  Soft binning: linear
interpolation between the two nearest bin centres, all weight to the end bin
outside the first / last centre.

The edge tables come from ``torch.linspace`` in float32, because the reference
defines its bins by that tensor (NumPy's linspace differs by an ulp).  All
arithmetic after that is float64, vectorised with ``np.bincount`` so that the
full benchmark volumes (16 M voxel-channels) take about a second.
"""

from __future__ import annotations

from typing import Tuple

import numpy as np
import torch

EPS32 = float(torch.finfo(torch.float32).eps)


def linspace32(steps: int) -> np.ndarray:
    """The reference's float32 boundaries over [0, 1 + eps32], as float64."""
    return torch.linspace(0.0, 1.0 + EPS32, steps).double().numpy()


def hard_index(p: np.ndarray, num_bins: int, right: bool) -> np.ndarray:
    edges = linspace32(num_bins + 1)[1:]
    return np.searchsorted(edges, p, side="right" if right else "left")


def soft_parts(p: np.ndarray, num_bins: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """(left bin, right bin, left weight, right weight), float64 interpolation."""
    centres = linspace32(2 * num_bins + 1)[1::2]
    j = np.searchsorted(centres, p, side="left") - 1  # c_j < p <= c_{j+1}
    low = j < 0
    high = j >= num_bins - 1
    jj = np.clip(j, 0, max(num_bins - 2, 0))
    left = jj.copy()
    rght = np.minimum(jj + 1, num_bins - 1)
    if num_bins > 1:
        t = (p - centres[jj]) / (centres[rght] - centres[jj])
    else:
        t = np.zeros_like(p)
    lw = 1.0 - t
    rw = t
    left[low], rght[low], lw[low], rw[low] = 0, 0, 1.0, 0.0
    left[high], rght[high], lw[high], rw[high] = num_bins - 1, num_bins - 1, 1.0, 0.0
    return left, rght, lw, rw


def slice_stats(p: np.ndarray, y: np.ndarray, binning: str, num_bins: int, right: bool):
    """(W, P, G) float64 arrays of length K for one slice."""
    p = np.asarray(p, dtype=np.float64).ravel()
    y = np.asarray(y, dtype=np.float64).ravel()
    k = num_bins
    if binning == "hard":
        idx = hard_index(p, k, right)
        w = np.bincount(idx, minlength=k).astype(np.float64)
        sp = np.bincount(idx, weights=p, minlength=k)
        sg = np.bincount(idx, weights=y, minlength=k)
        return w[:k], sp[:k], sg[:k]
    left, rght, lw, rw = soft_parts(p, k)
    w = np.bincount(left, weights=lw, minlength=k) + np.bincount(rght, weights=rw, minlength=k)
    sp = np.bincount(left, weights=lw * p, minlength=k) + np.bincount(rght, weights=rw * p, minlength=k)
    sg = np.bincount(left, weights=lw * y, minlength=k) + np.bincount(rght, weights=rw * y, minlength=k)
    return w, sp, sg


def activate64(x: np.ndarray, activation: str) -> np.ndarray:
    x = x.astype(np.float64)
    if activation == "softmax" and x.shape[1] > 1:
        e = np.exp(x - x.max(axis=1, keepdims=True))
        return e / e.sum(axis=1, keepdims=True)
    if activation == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    return x


def onehot64(target: np.ndarray, channels: int, to_onehot_y: bool) -> np.ndarray:
    if to_onehot_y and channels > 1:
        labels = target.reshape(target.shape[0], -1).astype(np.int64)
        out = np.zeros((target.shape[0], channels, labels.shape[1]))
        for c in range(channels):
            out[:, c] = labels == c
        return out
    return target.reshape(target.shape[0], channels, -1).astype(np.float64)


def stats64(p: np.ndarray, y: np.ndarray, config) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """[B, C', K] W, P, G for probabilities p and targets y already [B, C', N]."""
    b, c = p.shape[:2]
    k = config.num_bins
    out = np.zeros((3, b, c, k))
    for i in range(b):
        for j in range(c):
            out[:, i, j] = slice_stats(p[i, j], y[i, j], config.binning, k, config.right)
    return out[0], out[1], out[2]


def loss_from_stats(w, sp, sg, config, spatial_ndim: int = 3) -> np.ndarray:
    """Per-bin means -> per-class error -> mask, weights, reduction (float64)."""
    empty = (w == 0) if config.binning == "hard" else (w < config.empty_weight)
    safe = np.where(empty, 1.0, w)
    err = np.abs(sp - sg) / safe
    n_ne = (~empty).sum(-1)
    with np.errstate(invalid="ignore", divide="ignore"):
        f = np.where(empty, 0.0, err).sum(-1) / n_ne
    f = np.where(n_ne > 0, f, np.nan)
    if config.ignore_empty_classes:
        f = f * (sg.sum(-1) > 0)
    c = f.shape[1]
    if config.weight is not None and c != 1:
        f = f * np.broadcast_to(np.asarray(config.weight, dtype=np.float64), (c,))
    if config.reduction == "mean":
        return np.asarray(f.mean())
    if config.reduction == "sum":
        return np.asarray(f.sum())
    return f.reshape(*f.shape, *([1] * spatial_ndim))


def oracle_ace(input: np.ndarray, target: np.ndarray, config) -> np.ndarray:
    """float64 mL1-ACE for logits/probabilities ``input`` [B, C, ...]."""
    channels = input.shape[1]
    p = activate64(input, config.activation).reshape(input.shape[0], channels, -1)
    y = onehot64(target, channels, config.to_onehot_y)
    if not config.include_background and channels > 1:
        p, y = p[:, 1:], y[:, 1:]
    w, sp, sg = stats64(p, y, config)
    return loss_from_stats(w, sp, sg, config, input.ndim - 2)
