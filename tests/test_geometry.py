"""The launch geometry on the CPU: ``make_geometry`` (``ace_geometry.hpp``,
compiled here with g++) never gives a fast forward kernel more threads per
block than its launch bound, for every configuration the fast kernels serve.

A kernel launched with more threads than its ``__launch_bounds__`` fails on
the device ("unspecified launch failure").  That happened once in the
deep-supervision path, whose launch took its block size from another
geometry; the launchers now refuse such a block size
(``hipErrorInvalidConfiguration``), and this test pins the geometry so that
the refusal is never reached: single problems at the largest block size the
dispatch allows (1024 threads) and the one-launch levels path (256 threads,
``ace_forward_levels``), for C in {2, 3, 4, 16}, hard and soft (moments)
binning, background kept or dropped, 1-65 batch indices, 0 to 27 M voxels
and 1 to 2048 bins.
"""

from __future__ import annotations

import ctypes
import itertools
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "ace-kernels_amd" / "csrc"
MAX_LDS = 160 * 1024  # gfx950 LDS per workgroup


@pytest.fixture(scope="module")
def geo(tmp_path_factory) -> ctypes.CDLL:
    out = tmp_path_factory.mktemp("geometry") / "libgeometry.so"
    cmd = ["g++", "-O2", "-shared", "-fPIC", "-std=c++17", f"-I{CSRC}",
           str(HERE / "geometry_harness.cpp"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    lib = ctypes.CDLL(str(out))
    ll = ctypes.c_longlong
    lib.fast_geometry.restype = None
    lib.fast_geometry.argtypes = [ll, ll, ll, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.POINTER(ll)]
    lib.fast_bound.restype = ctypes.c_int
    lib.fast_bound.argtypes = [ll, ctypes.c_int]
    lib.soft_frac.restype = ctypes.c_int
    lib.soft_frac.argtypes = [ll]
    return lib


def _geometry(lib, b, c, n, k, soft, bg, max_nt):
    out = (ctypes.c_longlong * 5)()
    lib.fast_geometry(b, c, n, k, soft, bg, max_nt, out)
    return tuple(out)


BATCH = [1, 2, 3, 32, 65]
VOXELS = [0, 1, 3, 63, 64, 1000, 4096, 16 ** 3, 32 ** 3, 64 ** 3, 128 ** 3, 512 ** 2, 300 ** 3]
BINS = [1, 2, 20, 50, 64, 200, 512, 513, 1000, 2048]


@pytest.mark.parametrize("c", [2, 3, 4, 16])
@pytest.mark.parametrize("soft", [0, 1])
def test_block_size_within_launch_bound(geo, c, soft) -> None:
    bound = geo.fast_bound(c, soft)
    assert bound == (1024 if c <= 4 and not soft else 256)
    checked = 0
    for b, n, k, bg in itertools.product(BATCH, VOXELS, BINS, [0, 1]):
        nt, vec, lds_fwd, lds_bwd, nblk = _geometry(geo, b, c, n, k, soft, bg, 1024)
        if soft and (k > 2048 or lds_fwd > MAX_LDS or lds_bwd > MAX_LDS):
            continue  # not served by the moments kernels (the generic ones take it)
        assert nt in (256, 1024) and nt <= bound, (b, c, n, k, soft, bg, nt)
        assert nblk >= 1
        # the levels path launches every level with 256-thread blocks
        lv = _geometry(geo, b, c, n, k, soft, bg, 256)
        assert lv[0] == 256 and lv[1] == vec, (b, c, n, k, soft, bg, lv)
        checked += 1
    assert checked > 500


def test_benchmark_configurations(geo) -> None:
    """The block sizes the benchmark configurations run with."""
    assert _geometry(geo, 2, 4, 128 ** 3, 20, 0, 1, 1024)[0] == 1024  # cfg 2
    assert _geometry(geo, 2, 4, 128 ** 3, 20, 1, 1, 1024)[0] == 256   # cfg 3
    assert _geometry(geo, 1, 16, 128 ** 3, 20, 0, 1, 1024)[0] == 256  # cfg 4
    assert _geometry(geo, 32, 4, 512 ** 2, 50, 1, 0, 1024)[0] == 256  # cfg 5


def test_soft_fixed_point_cannot_overflow(geo) -> None:
    """The generic soft sums hold, per bin, at most N terms below 2 that add
    to at most N (a voxel's two weights sum to 1): N 2^f must stay well
    inside int64 at every size, with 40 fraction bits up to 2^19 voxels."""
    assert geo.soft_frac(0) == geo.soft_frac(1) == 40
    assert geo.soft_frac((1 << 19) - 1) == 40
    assert geo.soft_frac(128 ** 3) == 38
    prev = 40
    for bits in range(0, 41):
        for n in sorted({max((1 << bits) - 1, 0), 1 << bits, (1 << bits) + 1}):
            f = geo.soft_frac(n)
            assert 1 <= f <= 40 and f <= prev
            prev = f
            assert n * 2 ** f < 2 ** 61 and 2 * 2 ** f < 2 ** 62, (n, f)
