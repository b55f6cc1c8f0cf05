"""A seeded sweep over the option space at small sizes: every case runs the
HIP path through the C-ABI and compares loss and gradient with the oracle's
reference loss.  It covers channel counts 1..64 (fast and generic kernels),
bin counts 1..64, the three activations, label and one-hot targets,
background kept or dropped, empty classes ignored or not, the three
reductions, right edges, and fp32 / bf16 / fp16 logits.

Inputs follow the reference's domain: probabilities in [0, 1] when no
activation applies (activation "none", or softmax over one channel), class
indices in [0, C) or one-hot float targets.  Tolerances as the parity tests:
loss rtol 1e-5 / atol 1e-6; gradients by the reference's rules (boundary
voxels may differ; soft bins with fewer than 8 voxels take rtol 1e-3 or the
float64 result); 16-bit logits are compared on the same 16-bit values, the
gradient after rounding the oracle's to the logits' dtype.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ace_kernels import ACEConfig
from gpu_helpers import (LOSS_ATOL, LOSS_RTOL, assert_grad_close, assert_lowp_grad_close, kernel_probs, run, say,
                         truth64)

pytestmark = pytest.mark.gpu

CHANNELS = [1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 33, 64]
BINS = [1, 2, 3, 7, 20, 33, 64]
DTYPES = [torch.float32, torch.float32, torch.float32, torch.bfloat16, torch.float16]


def _cases(n: int = 120):
    rng = np.random.default_rng(20261201)
    out = []
    for i in range(n):
        c = int(rng.choice(CHANNELS))
        act = str(rng.choice(["softmax", "softmax", "sigmoid", "none"]))
        onehot = bool(rng.integers(2)) if c > 1 else False
        kw = dict(
            binning=str(rng.choice(["hard", "soft"])),
            num_bins=int(rng.choice(BINS)),
            activation=act,
            to_onehot_y=onehot,
            include_background=bool(rng.integers(2)),
            ignore_empty_classes=bool(rng.integers(2)),
            reduction=str(rng.choice(["mean", "sum", "none"])),
            right=bool(rng.integers(2)),
        )
        b = int(rng.integers(1, 4))
        spatial = tuple(int(v) for v in rng.integers(3, 17, size=int(rng.integers(1, 4))))
        dtype = DTYPES[int(rng.integers(len(DTYPES)))]
        out.append(pytest.param(i, b, c, spatial, dtype, kw, id=f"{i}-{kw['binning']}-C{c}-K{kw['num_bins']}-{act}"))
    return out


def _inputs(seed, b, c, spatial, dtype, cfg):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((b, c, *spatial), generator=gen) * 2.0
    if cfg.activation == "none" or (cfg.activation == "softmax" and c == 1):
        x = torch.sigmoid(x)  # probabilities, the reference's domain without an activation
    x = x.to(dtype)
    labels = torch.randint(0, max(c, 2) if c == 1 else c, (b, 1, *spatial), generator=gen)
    if cfg.to_onehot_y:
        y = labels
    elif c == 1:
        y = labels.float()
    else:
        y = torch.zeros((b, c, *spatial)).scatter_(1, labels, 1.0)
    return x, y


@pytest.mark.parametrize("i,b,c,spatial,dtype,kw", _cases())
def test_sweep(i, b, c, spatial, dtype, kw) -> None:
    from oracle.reference import register_reference

    register_reference()
    cfg = ACEConfig(**kw)
    x, y = _inputs(1000 + i, b, c, spatial, dtype, cfg)
    say(f"sweep {i}: B={b} C={c} {spatial} {dtype} {kw}")
    loss, grad = run("hip_mi355x", x.cuda(), y.cuda(), cfg)
    loss_ref, grad_ref = run("reference", x.float(), y, cfg)
    torch.testing.assert_close(loss.cpu(), loss_ref, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    if dtype != torch.float32:
        # dx in the logits' type: within one unit of the reference's rounded gradient
        assert_lowp_grad_close(grad, grad_ref, x, cfg)
        return
    voxels = x[0, 0].numel()
    if cfg.binning == "soft" and voxels < 8 * cfg.num_bins:
        _, grad64 = truth64(x, y, cfg)
        assert_grad_close(grad, grad_ref, x, cfg, rtol=1e-3, truth=grad64)
    else:
        assert_grad_close(grad, grad_ref, x, cfg)


# 16-bit soft cases with a few voxels per bin from a 16 000-case soak of this
# option space (new draw seeds, input seeds as below) whose one-element
# gradient miss the rule above does not cover: one float16 unit beyond the
# reference and the rounded float64 truth, within one unit of the float64
# gradient at the kernels' own probabilities.
RECORDED_LOWP = [
    (1200107642, 3, 7, (16,), torch.float16,
     dict(binning="soft", num_bins=33, activation="sigmoid", to_onehot_y=False, include_background=True,
          ignore_empty_classes=False, reduction="mean", right=False)),
    (1200208462, 1, 33, (3, 11, 15), torch.float16,
     dict(binning="soft", num_bins=64, activation="softmax", to_onehot_y=False, include_background=True,
          ignore_empty_classes=False, reduction="sum", right=True)),
]


@pytest.mark.parametrize("seed,b,c,spatial,dtype,kw", RECORDED_LOWP)
def test_recorded_lowp_few_voxels(seed, b, c, spatial, dtype, kw) -> None:
    from oracle.reference import register_reference
    from test_gpu_soft_few_voxels import _at64

    register_reference()
    cfg = ACEConfig(**kw)
    x, y = _inputs(seed, b, c, spatial, dtype, cfg)
    say(f"recorded 16-bit few-voxel case: seed {seed} B={b} C={c} {spatial} {dtype} {kw}")
    loss, grad = run("hip_mi355x", x.cuda(), y.cuda(), cfg)
    loss_ref, grad_ref = run("reference", x.float(), y, cfg)
    torch.testing.assert_close(loss.cpu(), loss_ref, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    _, grad64 = truth64(x, y, cfg)
    _, own = _at64(kernel_probs(x, cfg), y, cfg)
    assert_lowp_grad_close(grad, grad_ref, x, cfg, truth=grad64, own=own)


# Soft binning with one bin, from the same soak: every half-bin then has a
# sentinel centre at +-1e4, so the reference's float32 distances keep p only
# to 2^-10 and its loss lands ~1e-6 from the float64 result, beyond the loss
# rule above; the kernels' loss is ~1e-9 from it (exact-arithmetic weights).
RECORDED_SINGLE_BIN = [
    (1200102900, 2, 2, (14, 14, 14), torch.float32,
     dict(binning="soft", num_bins=1, activation="softmax", to_onehot_y=False, include_background=True,
          ignore_empty_classes=True, reduction="none", right=True)),
    (1200104306, 1, 1, (15, 9, 10), torch.float32,
     dict(binning="soft", num_bins=1, activation="none", to_onehot_y=False, include_background=True,
          ignore_empty_classes=False, reduction="sum", right=False)),
]


@pytest.mark.parametrize("seed,b,c,spatial,dtype,kw", RECORDED_SINGLE_BIN)
def test_recorded_single_bin_soft_loss(seed, b, c, spatial, dtype, kw) -> None:
    from oracle.reference import register_reference

    register_reference()
    cfg = ACEConfig(**kw)
    x, y = _inputs(seed, b, c, spatial, dtype, cfg)
    say(f"recorded single-bin soft case: seed {seed} B={b} C={c} {spatial} {kw}")
    loss, grad = run("hip_mi355x", x.cuda(), y.cuda(), cfg)
    loss_ref, grad_ref = run("reference", x, y, cfg)
    loss64, grad64 = truth64(x, y, cfg)
    k, r, t = loss.cpu().double(), loss_ref.double(), loss64.double()
    assert bool(((k - t).abs() <= (r - t).abs()).all()), (k, r, t)
    assert bool(((k - t).abs() <= 1e-6 * t.abs() + 1e-9).all()), (k, t)
    assert_grad_close(grad, grad_ref, x, cfg, truth=grad64)

