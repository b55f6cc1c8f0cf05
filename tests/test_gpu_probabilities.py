"""``ace_probabilities`` returns the probabilities the kernels bin: the
forward's float64 bin statistics (``stats``: W, P, G per bin) recomputed on
the CPU from the hook's probabilities agree with the forward's own -- exactly
for hard counts, to float64 rounding for the soft moments (exact sums of
the quantised p) and to the fixed-point step for the generic soft sums,
both with the exact-arithmetic weights.  The same statistics from torch's CPU
softmax differ by ~1e-6 (an ulp of p moves a soft weight by ~K ulp), which
a hook returning anything else than the kernels' probabilities would show.
The few-voxel parity tests measure their rounding spread with it."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ace_kernels import ACEConfig
from ace_kernels import measure as m
from ace_kernels.impls.hip_mi355x import bin_tables
from gpu_helpers import hip_stats, kernel_probs, say

pytestmark = pytest.mark.gpu


def _moment_bits(k: int) -> int:
    """m of the moments' fixed point, p held as trunc(p 2^m) / 2^m:
    23 + floor(log2 2K), at most 30 (``csrc/ace_bins.hpp: moment_scale``)."""
    lg = 0
    while (2 << lg) <= 2 * k:
        lg += 1
    return min(23 + lg, 30)


def _stats64(p: torch.Tensor, labels: torch.Tensor, cfg: ACEConfig, moments: bool) -> np.ndarray:
    """float64 [3, B, C', K] W, P, G of probabilities p [B, C, N] and class
    labels [B, N] as the kernels form them: hard counts; soft the
    exact-arithmetic weights (c_R - p) / S and (p - c_L) / S of the soft
    assignment (``common.py:43-61``), of p quantised to 2^-m in the moments
    kernels."""
    b, c, n = p.shape
    off = 0 if cfg.include_background or c == 1 else 1
    k = cfg.num_bins
    soft = cfg.binning == "soft"
    up, repl = bin_tables(k, soft, torch.device("cpu"))
    up = up.numpy()
    side = "right" if cfg.right else "left"
    out = np.zeros((3, b, c - off, k))
    pf = p.float().numpy()
    lab = labels.numpy()
    for bi in range(b):
        for cl in range(c - off):
            pc = pf[bi, cl + off]
            yv = (lab[bi] == cl + off).astype(np.float64)
            h = np.searchsorted(up, pc, side=side)
            if not soft:
                np.add.at(out[0, bi, cl], h, 1.0)
                np.add.at(out[1, bi, cl], h, pc.astype(np.float64))
                np.add.at(out[2, bi, cl], h, yv)
                continue
            left = np.maximum(h - 1, 0) >> 1
            right = np.minimum(h + 1, 2 * k - 1) >> 1
            q = pc.astype(np.float64)
            if moments:
                sc = float(2 ** _moment_bits(k))
                q = np.trunc(q * sc) / sc
            r = repl.double().numpy()
            span = r[h + 2] - r[h]
            for w, idx in (((r[h + 2] - q) / span, left), ((q - r[h]) / span, right)):
                np.add.at(out[0, bi, cl], idx, w)
                np.add.at(out[1, bi, cl], idx, w * q)
                np.add.at(out[2, bi, cl], idx, w * yv)
    return out


CASES = [
    ("hard-c4", 2, 4, (24, 20, 6), dict(binning="hard", num_bins=20)),
    ("soft-c4-moments", 2, 4, (24, 20, 6), dict(binning="soft", num_bins=20)),
    ("soft-c16-moments", 1, 16, (18, 16, 5), dict(binning="soft", num_bins=20, include_background=False)),
    ("soft-c17-generic", 1, 17, (18, 16, 5), dict(binning="soft", num_bins=20)),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_bins_the_hooks_probabilities(case) -> None:
    name, b, c, spatial, kw = case
    cfg = ACEConfig(to_onehot_y=True, activation="softmax", **kw)
    x, y = m.make_inputs(m.ShapeSpec("p", b, c, spatial, logit_scale=10.0), cfg, "cpu", 5)
    say(f"probabilities: {name}")
    st = hip_stats(x.cuda(), y.cuda(), cfg)[5].cpu().numpy()
    pk = kernel_probs(x, cfg).reshape(b, c, -1)
    labels = y.reshape(b, -1)
    moments = cfg.binning == "soft" and c in (2, 3, 4, 16)
    got = _stats64(pk, labels, cfg, moments)
    if cfg.binning == "hard":
        np.testing.assert_array_equal(st[0], got[0])
        np.testing.assert_array_equal(st[2], got[2])
        np.testing.assert_allclose(st[1], got[1], rtol=0, atol=5e-6)  # sums of p at 2^-30
        return
    # moments: float64 rounding of exact sums; generic: 2^-41 per fixed-point term
    rtol, atol = (1e-12, 1e-11) if moments else (0.0, 2e-9)
    np.testing.assert_allclose(st, got, rtol=rtol, atol=atol)
    # torch's CPU softmax is not what the kernels bin: its statistics fail the
    # same comparison (as would a hook returning other probabilities)
    cpu = _stats64(torch.softmax(x.float(), 1).reshape(b, c, -1), labels, cfg, moments)
    assert not np.allclose(st, cpu, rtol=rtol, atol=atol), "torch's softmax gave the kernels' statistics"


def test_probabilities_are_a_softmax() -> None:
    """Within 3 ulp of torch's softmax (neither is correctly rounded) and
    summing to 1, for each dtype; the sigmoid within 5e-7 of torch's."""
    gen = torch.Generator().manual_seed(3)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        x = (torch.randn(3, 5, 17, 9, generator=gen) * 6).to(dtype)
        say(f"probabilities: softmax {dtype}")
        pk = kernel_probs(x, ACEConfig(activation="softmax"))
        pt = torch.softmax(x.float(), 1)
        ulp = torch.finfo(torch.float32).eps * pt.abs().clamp_min(torch.finfo(torch.float32).tiny)
        assert bool(((pk - pt).abs() <= 3 * ulp + 1e-38).all())
        torch.testing.assert_close(pk.sum(1), torch.ones_like(pk.sum(1)), rtol=0, atol=1e-6)
        ps = kernel_probs(x, ACEConfig(activation="sigmoid"))
        torch.testing.assert_close(ps, torch.sigmoid(x.float()), rtol=5e-7, atol=1e-30)
