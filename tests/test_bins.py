"""The kernels' O(1) bin index (``ace::bucket``) equals torch.bucketize.

The reference's v6 kernels use ``floor(p * n)`` plus two correction rounds
(``src/ace_kernels/kernels/bins.py:27-48``) and test them at every float32
within 8 ulp of every edge (``tests/test_triton.py:352-393``).  The HIP kernels
use one round (both neighbours read at once).  This test compiles the very
header the kernels include (``csrc/ace_bins.hpp``) with g++ and checks it
against a binary search over the same float32 ``torch.linspace`` tables:

- every float32 within 4096 ulp of every edge, for K in 1..128 and larger K,
  hard (K edges) and soft (2K half boundaries), right = False / True;
- every float32 in [0, 1 + eps32] (exhaustive) for the benchmark tables
  K = 20 and K = 50;
- out-of-domain values (NaN, +-inf, > 1) stay inside [0, n - 1];
- the softmax variant for probabilities in [0, 1] (``bucket_unit``: first
  guess trunc(p * n - 1/4), one correction) on every float32 of [0, 1] for
  K = 20 and 50, near every edge for every K, NaN, and with its correction
  dropped (a planted mistake the near-edge sweep must catch).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "ace-kernels_amd" / "csrc"
EPS32 = torch.finfo(torch.float32).eps


@pytest.fixture(scope="module")
def harness(tmp_path_factory) -> ctypes.CDLL:
    out = tmp_path_factory.mktemp("bins") / "libbins.so"
    cmd = ["g++", "-O2", "-fopenmp", "-shared", "-fPIC", "-std=c++17", f"-I{CSRC}",
           str(HERE / "bins_harness.cpp"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    lib = ctypes.CDLL(str(out))
    fp = ctypes.POINTER(ctypes.c_float)
    lib.check_values.restype = ctypes.c_longlong
    lib.check_values.argtypes = [fp, ctypes.c_int, ctypes.c_int, fp, ctypes.c_longlong]
    lib.check_near_edges.restype = ctypes.c_longlong
    lib.check_near_edges.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.check_range.restype = ctypes.c_longlong
    lib.check_range.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float]
    lib.check_clamped.restype = ctypes.c_int
    lib.check_clamped.argtypes = [fp, ctypes.c_int]
    lib.check_unit.restype = ctypes.c_longlong
    lib.check_unit.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                               ctypes.c_int, ctypes.c_int]
    lib.check_div.restype = ctypes.c_longlong
    lib.check_div.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                              ctypes.c_int]
    lib.check_moment_offsets.restype = ctypes.c_longlong
    lib.check_moment_offsets.argtypes = [fp, ctypes.c_int, ctypes.c_int]
    lib.check_moment_all.restype = ctypes.c_longlong
    lib.check_moment_all.argtypes = [fp, ctypes.c_int, ctypes.c_int]
    lib.check_fast_margin.restype = ctypes.c_longlong
    lib.check_fast_margin.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_int,
                                      ctypes.c_int]
    lib.check_unit_nan.restype = ctypes.c_int
    lib.check_unit_nan.argtypes = [fp, ctypes.c_int]
    return lib


def _table(n_bins: int, soft: bool) -> np.ndarray:
    steps = (2 * n_bins if soft else n_bins) + 1
    return torch.linspace(0.0, 1.0 + EPS32, steps)[1:].numpy().astype(np.float32).copy()


def _fp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


KS = list(range(1, 129)) + [200, 256, 333, 500, 1000, 4096]


@pytest.mark.parametrize("soft", [False, True])
@pytest.mark.parametrize("right", [False, True])
def test_near_every_edge(harness, soft: bool, right: bool) -> None:
    bad = {}
    for k in KS:
        t = _table(k, soft)
        n = harness.check_near_edges(_fp(t), t.size, int(right), 4096)
        if n:
            bad[k] = n
    assert not bad, bad


@pytest.mark.parametrize("k", [20, 50])
@pytest.mark.parametrize("soft", [False, True])
def test_exhaustive_unit_interval(harness, k: int, soft: bool) -> None:
    t = _table(k, soft)
    for right in (0, 1):
        assert harness.check_range(_fp(t), t.size, right, 0.0, float(1.0 + EPS32)) == 0


def test_random_and_out_of_domain(harness) -> None:
    gen = np.random.default_rng(0)
    p = gen.random(1_000_000, dtype=np.float32)
    for k in (1, 3, 20, 50, 100):
        for soft in (False, True):
            t = _table(k, soft)
            for right in (0, 1):
                assert harness.check_values(_fp(t), t.size, right, _fp(p), p.size) == 0
            assert harness.check_clamped(_fp(t), t.size) == 1


def test_edges_detect_an_uncorrected_index(harness) -> None:
    """Planted mistake: floor(p * n) alone (no correction) must fail near edges,
    so the near-edge sweep above is sensitive to a missing correction."""
    harness.check_near_edges_uncorrected.restype = ctypes.c_longlong
    harness.check_near_edges_uncorrected.argtypes = [
        ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_int, ctypes.c_int]
    total = 0
    for k in (3, 7, 20, 50):
        t = _table(k, False)
        total += harness.check_near_edges_uncorrected(_fp(t), t.size, 0, 8)
    assert total > 0


@pytest.mark.parametrize("soft", [False, True])
def test_unit_interval_variant(harness, soft: bool) -> None:
    """bucket_unit<RIGHT>, used on softmax probabilities: exhaustive on [0, 1]
    for the benchmark tables, near every edge for every K, NaN -> bin 0."""
    for k in (20, 50):
        t = _table(k, soft)
        for right in (0, 1):
            assert harness.check_unit(_fp(t), t.size, right, 0.0, 1.0, 0, 0) == 0
    bad = {}
    for k in KS:
        t = _table(k, soft)
        for right in (0, 1):
            n = harness.check_unit(_fp(t), t.size, right, 0.0, 0.0, 4096, 0)
            if n:
                bad[(k, right)] = n
        assert harness.check_unit_nan(_fp(t), t.size) == 1
    assert not bad, bad


def test_unit_interval_variant_needs_its_correction(harness) -> None:
    """Planted mistake: the first guess trunc(p * n - 1/4) alone must fail near
    edges (it is k - 1 just above every edge), so the sweep above would catch a
    lost correction."""
    total = 0
    for k in (3, 7, 20, 50):
        t = _table(k, False)
        for right in (0, 1):
            total += harness.check_unit(_fp(t), t.size, right, 0.0, 0.0, 8, 1)
    assert total > 0


def _bits(v: float) -> int:
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def test_division_from_rounded_reciprocal(harness) -> None:
    """div_rn(a, b, RN(1/b)) is the IEEE quotient: every float b in [1, 16)
    (softmax sums) with 4 random a of exponents -100..0 each, and a sample of
    spans b in [2^-20, 2^14) with a of exponents -40..14."""
    assert harness.check_div(_bits(1.0), _bits(16.0), 4, -100, 0, 0) == 0
    lo, hi = _bits(2.0 ** -20), _bits(2.0 ** 14)
    for start in range(lo, hi, (hi - lo) // 16):
        assert harness.check_div(start, min(start + (1 << 18), hi), 4, -40, 14, 0) == 0


def test_division_check_catches_a_missing_correction(harness) -> None:
    """Planted mistake: a * RN(1/b) without the residual correction is wrong
    for some a, and the check above reports it."""
    assert harness.check_div(_bits(1.0), _bits(1.0) + (1 << 16), 4, -30, 0, 1) > 0


def test_soft_moment_offsets_every_bin_count(harness) -> None:
    """The soft moments store p in half-bin h as the offset u = trunc(p 2^m)
    - h w (``moment_scale``): u must lie in [0, 2^24) for every half-bin of
    every bin count the moments path takes (K <= 2048), so that h w and u^2
    are 24-bit multiplies and u^2 is exact."""
    bad = {k: harness.check_moment_offsets(_fp(_table(k, True)), k, 0) for k in range(1, 2049)}
    assert not any(bad.values()), {k: v for k, v in bad.items() if v}


@pytest.mark.parametrize("planted", [1, 2])
def test_soft_moment_offsets_check_catches_a_wrong_scale(harness, planted: int) -> None:
    # a scale one bit too fine overflows 24 bits; a base without its margin
    # passes the boundaries below
    assert sum(harness.check_moment_offsets(_fp(_table(k, True)), k, planted) for k in (7, 20, 50, 333)) > 0


@pytest.mark.parametrize("right", [False, True])
def test_soft_moment_offsets_every_probability(harness, right: bool) -> None:
    """Every float32 in [0, 1] at K = 20: offset in range, and base + offset
    is exactly p 2^m for p >= 2^(23 - m)."""
    assert harness.check_moment_all(_fp(_table(20, True)), 20, int(right)) == 0


# the fast probabilities' relative error bound the margin is built on
# (ace_core.hpp: fast_exp; measured on MI355X: 5.4e-7 at C = 4)
FAST_REL = {4: 1.5e-6, 16: 3.0e-6}


@pytest.mark.parametrize("channels", [4, 16])
@pytest.mark.parametrize("k", [1, 2, 7, 20, 40, 50, 64, 100, 256, 512])
def test_fast_bins_margin_covers_the_error_bound(harness, channels: int, k: int) -> None:
    """A fast-path q anywhere inside the error window of a probability p
    that fast_bin_index does not flag as near an edge has the bin of p
    (torch.bucketize, left and right), for every float within 256 ulp of
    every edge and a sample of [0, 1] (the hard forward's fast path)."""
    assert harness.check_fast_margin(_fp(_table(k, False)), k, channels, FAST_REL[channels], 256, 1) == 0


def test_fast_bins_margin_check_catches_a_small_margin(harness) -> None:
    """Planted mistake: a margin eight times too small lets fast bins
    disagree with bucketize near edges."""
    total = sum(harness.check_fast_margin(_fp(_table(k, False)), k, 4, FAST_REL[4], 256, 8)
                for k in (20, 50))
    assert total > 0
