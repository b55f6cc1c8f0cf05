"""The measurement harness's schema, bytes, floors and error metrics (CPU).

``ace_kernels.measure`` mirrors the reference's benchmark harness
(``src/ace_bench/measure.py:27-81`` Row, ``calculator.py:23-44``,
``timing.py:30-45``); these tests pin the parts that need no GPU.
"""

from __future__ import annotations

import math

import pytest
import torch

from ace_kernels import ACEConfig
from ace_kernels import measure as m

# The reference's Row fields (measure.py:27-81), in order.
REFERENCE_ROW_FIELDS = [
    "impl", "binning", "mode", "cuda_graph", "dtype", "shape", "batch", "channels", "spatial",
    "voxels", "status", "error", "p50_ms", "p20_ms", "p80_ms", "mean_ms", "std_ms", "reps",
    "input_bytes", "target_bytes", "ideal_bytes", "effective_gbps", "pct_peak_bw", "bw_floor_ms",
    "launch_floor_ms", "kernels_per_call", "aten_ops_per_call", "saved_extra_bytes",
    "peak_extra_bytes", "allocated_after_bytes", "checked_against", "loss_rel_err",
    "grad_rel_err", "loss_err_truth", "grad_err_truth", "ref_loss_err_truth",
    "ref_grad_err_truth", "grad_l2_err", "grad_l2_err_truth", "ref_grad_l2_err_truth",
]


# This package's rocprofv3 counter columns, after the reference's fields.
COUNTER_FIELDS = ["hbm_read_bytes", "hbm_write_bytes", "hbm_bytes_per_ideal",
                  "counted_kernels_per_call"]


def test_row_schema_matches_the_reference() -> None:
    fields = list(m.Row.model_fields)
    assert fields[:len(REFERENCE_ROW_FIELDS)] == REFERENCE_ROW_FIELDS
    assert fields[len(REFERENCE_ROW_FIELDS):] == COUNTER_FIELDS


def test_ideal_bytes_and_floors() -> None:
    # cfg 2: 2x4x128^3 fp32 logits, int64 labels
    xb, tb = 2 * 4 * 128 ** 3 * 4, 2 * 128 ** 3 * 8
    assert m.ideal_bytes(xb, tb, "fwd") == 100_663_296
    assert m.ideal_bytes(xb, tb, "fwd_bwd") == 268_435_456
    assert m.bandwidth_floor_ms(268_435_456) == pytest.approx(0.033554432)
    assert m.launch_floor_ms(7) == pytest.approx(0.035)
    assert m.effective_gbps(8_000_000, 1.0) == pytest.approx(8.0)


def test_quantiles_are_the_references_nearest_rank() -> None:
    st = m.summarize([5.0, 1.0, 4.0, 2.0, 3.0])
    assert (st.p50_ms, st.p20_ms, st.p80_ms, st.min_ms, st.reps) == (3.0, 2.0, 4.0, 1.0, 5)
    assert st.mean_ms == 3.0 and st.std_ms == pytest.approx(math.sqrt(2.5))


def test_error_metrics() -> None:
    b = torch.tensor([1.0, -2.0, 4.0])
    a = b + torch.tensor([0.0, 0.4, 0.0])
    assert m.rel_err(a, b) == pytest.approx(0.1)
    assert m.rel_l2(a, b) == pytest.approx(0.4 / math.sqrt(21.0))
    assert m.rel_err(b, b) == 0.0


@pytest.mark.parametrize("onehot", [True, False])
def test_inputs_are_seeded_and_biased(onehot: bool) -> None:
    shape = m.ShapeSpec("t", 2, 3, (5, 6), logit_scale=2.0, target_bias=7.0)
    cfg = ACEConfig(to_onehot_y=onehot)
    x1, y1 = m.make_inputs(shape, cfg, "cpu", seed=3)
    x2, y2 = m.make_inputs(shape, cfg, "cpu", seed=3)
    assert torch.equal(x1, x2) and torch.equal(y1, y2)
    labels = y1 if onehot else y1.argmax(1, keepdim=True)
    assert labels.shape == (2, 1, 5, 6)
    # the bias makes the labelled channel the arg-max almost everywhere
    assert (x1.argmax(1, keepdim=True) == labels).float().mean() > 0.9
    if not onehot:
        assert torch.equal(y1.sum(1), torch.ones(2, 5, 6))


def test_reference_against_float64_truth() -> None:
    """compute_reference with the oracle impls: the fp32 reference sits within
    fp32 noise of its float64 truth."""
    from oracle.reference import register_reference
    from oracle.v2 import register_v2

    register_reference()
    register_v2()
    for binning in ("hard", "soft"):
        cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
        ref = m.compute_reference(m.ShapeSpec("s", 2, 4, (8, 8, 8), target_bias=1.0), cfg)
        assert ref.ref_loss_err_truth is not None and ref.ref_loss_err_truth < 1e-5
        assert ref.ref_grad_l2_err_truth is not None and ref.ref_grad_l2_err_truth < 1e-4
