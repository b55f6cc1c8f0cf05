"""The harness's HBM traffic columns on MI355X: two rocprofv3 counter runs
(FETCH_SIZE, WRITE_SIZE) of a case in child processes, calibrated by a copy
of known size (ace_kernels.counters)."""

from __future__ import annotations

import shutil
from pathlib import Path

import pytest

from ace_kernels import ACEConfig
from ace_kernels import measure as m
from gpu_helpers import say

pytestmark = pytest.mark.gpu

# configuration 2's shape: large enough that the blocks' final-sum atomics
# (a few hundred KB either way) stay within a few percent of the bytes
SHAPE = m.ShapeSpec("kits23", 2, 4, (128, 128, 128))


def have_rocprof() -> bool:
    return Path("/opt/rocm/bin/rocprofv3").exists() or shutil.which("rocprofv3") is not None


@pytest.mark.skipif(not have_rocprof(), reason="rocprofv3 not installed")
@pytest.mark.parametrize("binning,mode,kernels", [("hard", "fwd", 1), ("soft", "fwd_bwd", 2)])
def test_row_hbm_traffic(binning, mode, kernels) -> None:
    """Each call reads and writes about the ideal bytes: the forward reads
    logits and labels once; the backward reads the logits (and the labels for
    soft binning) and writes the gradient -- the hard backward reads no labels,
    so its step moves 7/8 of the ideal bytes at C = 4."""
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    say(f"counter row hip_mi355x {binning} {mode} (two rocprofv3 runs)")
    row = m.measure_case("hip_mi355x", SHAPE, cfg, mode, reps=3, warmup=1, counters=True)
    assert row.status == "ok"
    assert row.error is None, row.error
    assert row.counted_kernels_per_call == kernels
    x_bytes = row.input_bytes
    want_read = row.input_bytes + row.target_bytes + (x_bytes + row.target_bytes if mode == "fwd_bwd" else 0)
    want_write = x_bytes if mode == "fwd_bwd" else 0
    say(f"  read {row.hbm_read_bytes} (ideal {want_read}), write {row.hbm_write_bytes} "
        f"(ideal {want_write}), ratio {row.hbm_bytes_per_ideal:.3f}")
    assert 0.97 * want_read <= row.hbm_read_bytes <= 1.05 * want_read
    assert row.hbm_write_bytes <= 0.08 * want_read + 1.02 * want_write
    if want_write:
        assert row.hbm_write_bytes >= 0.98 * want_write
    assert 0.9 <= row.hbm_bytes_per_ideal <= 1.1
