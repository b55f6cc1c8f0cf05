"""The oracle is pinned before it is trusted (CPU only).

- ``oracle.reference`` reproduces the reference's 43 golden cases (loss and
  gradient, written by the reference on its own platform) at the reference's
  CPU tolerances (``tests/helpers.py:15-16`` upstream).
- ``oracle.v2`` (handwritten backward) matches the golden cases, float64
  finite differences (gradcheck) and float64 autograd through the scatter-based
  statistics.
- ``oracle.f64`` (float64, written from the mathematics) matches the golden
  losses and closed forms.
"""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch

from ace_kernels.config import ACEConfig
from golden_cases import load_golden
from oracle import f64, v2
from oracle.reference import reference_ace

LOSS_RTOL, LOSS_ATOL = 1e-5, 1e-6
GRAD_RTOL, GRAD_ATOL = 1e-4, 1e-7
GOLDEN = load_golden()
NAMES = sorted(GOLDEN)


def _run(fn, x: torch.Tensor, y: torch.Tensor, config: ACEConfig):
    leaf = x.detach().clone().requires_grad_(True)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", UserWarning)
        loss = fn(leaf, y, config)
    (grad,) = torch.autograd.grad(loss.sum(), leaf)
    return loss.detach(), grad


def test_golden_has_all_cases() -> None:
    assert len(GOLDEN) == 43
    for name in ("paper-3d-hard", "paper-3d-soft", "bin-edges-right-hard", "soft-high-empty-weight"):
        assert name in GOLDEN


@pytest.mark.parametrize("name", NAMES)
def test_reference_matches_golden(name: str) -> None:
    case = GOLDEN[name]
    config = ACEConfig.model_validate(case.config)
    loss, grad = _run(reference_ace, case.input, case.target, config)
    torch.testing.assert_close(loss, case.loss, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    torch.testing.assert_close(grad, case.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)


@pytest.mark.parametrize("name", NAMES)
def test_v2_matches_golden(name: str) -> None:
    case = GOLDEN[name]
    config = ACEConfig.model_validate(case.config)
    loss, grad = _run(v2.v2_ace, case.input, case.target, config)
    torch.testing.assert_close(loss, case.loss, rtol=LOSS_RTOL, atol=LOSS_ATOL)
    torch.testing.assert_close(grad, case.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)


@pytest.mark.parametrize("name", NAMES)
def test_f64_matches_golden_loss(name: str) -> None:
    case = GOLDEN[name]
    config = ACEConfig.model_validate(case.config)
    expected = f64.oracle_ace(case.input.double().numpy(), case.target.numpy(), config)
    np.testing.assert_allclose(case.loss.double().numpy(), expected, rtol=LOSS_RTOL, atol=LOSS_ATOL)


def test_closed_forms() -> None:
    # constant probability 0.5 with 0/1 targets: |0.5 - mean y| averages 0.25
    assert GOLDEN["constant-probs-hard"].loss.item() == 0.25
    assert GOLDEN["constant-probs-soft"].loss.item() == 0.25
    # one bin: soft weights all go to the single bin -> identical to hard
    torch.testing.assert_close(GOLDEN["one-bin-hard"].loss, GOLDEN["one-bin-soft"].loss, rtol=1e-5, atol=0)
    # per-slice sums: hard counts sum to N; soft weights per voxel sum to 1
    gen = np.random.default_rng(0)
    p = gen.random(5000)
    for k in (1, 7, 20):
        w, _, _ = f64.slice_stats(p, np.zeros_like(p), "hard", k, False)
        assert w.sum() == p.size
        w, _, _ = f64.slice_stats(p, np.zeros_like(p), "soft", k, False)
        np.testing.assert_allclose(w.sum(), p.size, rtol=1e-12)


def test_oracle_detects_a_planted_mistake() -> None:
    """A mutant oracle (mean of |P - G| without dividing by W) must disagree."""
    case = GOLDEN["paper-3d-hard"]
    config = ACEConfig.model_validate(case.config)
    p = f64.activate64(case.input.numpy(), config.activation).reshape(2, 4, -1)
    y = f64.onehot64(case.target.numpy(), 4, True)
    w, sp, sg = f64.stats64(p, y, config)
    good = f64.loss_from_stats(w, sp, sg, config)
    mutant = f64.loss_from_stats(np.ones_like(w) * (w > 0), sp, sg, config)
    np.testing.assert_allclose(good, case.loss.double().numpy(), rtol=1e-5)
    assert abs(float(mutant) - case.loss.item()) > 1e-2


V2_CONFIGS = {
    "paper": {"to_onehot_y": True},
    "no-background-weights": {"to_onehot_y": True, "include_background": False, "weight": (2.0, 0.5, 1.0)},
    "reduction-none": {"to_onehot_y": True, "reduction": "none"},
    "reduction-sum-kept-empty": {"to_onehot_y": True, "reduction": "sum", "ignore_empty_classes": False},
    "sigmoid": {"activation": "sigmoid"},
    "onehot-target": {},
}


def _inputs64(name: str, binning: str, seed: int = 7):
    config = ACEConfig.model_validate({"binning": binning, **V2_CONFIGS[name]})
    channels = 1 if name == "sigmoid" else 4
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(2, channels, 5, 5, 4, generator=gen, dtype=torch.float64) * 2.0
    labels = torch.randint(0, channels, (2, 1, 5, 5, 4), generator=gen)
    if channels == 1:
        y = torch.randint(0, 2, (2, 1, 5, 5, 4), generator=gen).double()
    elif config.to_onehot_y:
        y = labels
    else:
        y = torch.zeros(2, channels, 5, 5, 4, dtype=torch.float64).scatter_(1, labels, 1.0)
    return config, x, y


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("name", sorted(V2_CONFIGS))
def test_v2_gradcheck_float64(binning: str, name: str) -> None:
    """Handwritten gradient == finite differences (independent of the reference)."""
    config, x, y = _inputs64(name, binning)
    x.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda inp: v2.v2_ace(inp, y, config), (x,), eps=1e-7, atol=1e-6, rtol=1e-4)


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("name", sorted(V2_CONFIGS))
def test_v2_matches_autograd_float64(binning: str, name: str) -> None:
    """Handwritten formula == autograd through the scatter statistics, to 1e-9."""
    config, x, y = _inputs64(name, binning, seed=11)

    def autograd_loss(inp):
        prep = v2.prepare(inp, y, config)
        stats = v2.bin_stats(prep, config)
        f = torch.nanmean(v2.per_bin_error(stats), dim=-1)
        return v2.reduce_classes(f, prep.spatial_ndim, config, v2.class_present(stats))

    out = []
    for fn in (lambda inp: v2.v2_ace(inp, y, config), autograd_loss):
        leaf = x.clone().requires_grad_(True)
        loss = fn(leaf)
        out.append((loss.detach(), torch.autograd.grad(loss.sum(), leaf)[0]))
    torch.testing.assert_close(out[0][0], out[1][0], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(out[0][1], out[1][1], rtol=1e-9, atol=1e-12)


def test_reference_invariants() -> None:
    """Voxel-order invariance and 0 <= loss <= 1 (upstream tests/test_equivalence.py:60-85)."""
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(2, 4, 6, 6, 6, generator=gen) * 2.0
    y = torch.randint(0, 4, (2, 1, 6, 6, 6), generator=gen)
    perm = torch.randperm(216, generator=torch.Generator().manual_seed(0))
    for binning in ("hard", "soft"):
        config = ACEConfig(binning=binning, to_onehot_y=True)
        a, ga = _run(reference_ace, x, y, config)
        b, _ = _run(reference_ace, x.flatten(2)[..., perm].reshape(x.shape), y.flatten(2)[..., perm].reshape(y.shape), config)
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)
        assert 0.0 <= a.item() <= 1.0
        assert torch.isfinite(ga).all()
