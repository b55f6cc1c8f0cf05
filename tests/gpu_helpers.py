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
