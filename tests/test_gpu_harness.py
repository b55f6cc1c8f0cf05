"""The measurement harness on MI355X: rows of the reference's schema for this
package's implementations, checked against the CPU restatement of the
reference and its float64 truth (``src/ace_bench/measure.py:280-360``)."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig
from ace_kernels import measure as m
from gpu_helpers import say

pytestmark = pytest.mark.gpu

SHAPE = m.ShapeSpec("t24", 2, 4, (24, 24, 24), logit_scale=2.0, target_bias=2.0)


@pytest.fixture(scope="module")
def references():
    from oracle.reference import register_reference
    from oracle.v2 import register_v2

    register_reference()
    register_v2()
    out = {}
    for binning in ("hard", "soft"):
        cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
        out[binning] = (cfg, m.compute_reference(SHAPE, cfg, "cpu"))
    return out


@pytest.mark.parametrize("impl", ["hip_mi355x", "hip_mi355x_op"])
@pytest.mark.parametrize("mode", ["fwd", "fwd_bwd"])
@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_rows_with_output_check(references, binning, mode, impl) -> None:
    cfg, ref = references[binning]
    say(f"harness row {impl} {binning} {mode}")
    row = m.measure_case(impl, SHAPE, cfg, mode, reps=5, warmup=2, reference=ref)
    assert row.status == "ok", row.error
    assert row.p50_ms is not None and 0 < row.p20_ms <= row.p50_ms <= row.p80_ms
    assert row.ideal_bytes == m.ideal_bytes(row.input_bytes, row.target_bytes, mode)
    assert row.kernels_per_call is not None and row.kernels_per_call >= 1
    # the autograd node keeps coef, d and jac beyond its inputs: a few hundred bytes
    assert row.saved_extra_bytes is not None and row.saved_extra_bytes < 64 * 1024
    assert row.checked_against == "reference"
    assert row.loss_rel_err is not None and row.loss_rel_err < 1e-5
    assert row.loss_err_truth is not None and row.loss_err_truth < 1e-5
    assert row.grad_l2_err is not None and row.grad_l2_err < 1e-4
    assert row.grad_l2_err_truth is not None and row.grad_l2_err_truth < 1e-4


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_graph_rows(references, binning) -> None:
    cfg, _ = references[binning]
    say(f"harness graph row {binning}")
    row = m.measure_case("hip_mi355x", SHAPE, cfg, "fwd_bwd", cuda_graph=True, reps=5, warmup=2)
    assert row.status == "ok", row.error
    assert row.p50_ms is not None and row.peak_extra_bytes is None
