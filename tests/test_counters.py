"""The harness's rocprofv3 counter columns without a GPU: the case a child
run rebuilds, the counter CSV parser, the copy calibration and the per-call
sums (ace_kernels.counters)."""

from __future__ import annotations

import csv

import pytest

from ace_kernels import ACEConfig
from ace_kernels import counters as ct
from ace_kernels import measure as m

HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
          "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
          "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
          "Counter_Value", "Start_Timestamp", "End_Timestamp"]
FWD = "void ace::fwd_kernel_fast<float, 4, 2, false, false, false>(ace::FwdParams)"
BWD = "void ace::bwd_kernel_fast<float, 4, 4, false, false, false>(ace::BwdParams)"
COPY = "__amd_rocclr_copyBuffer"
SUM = "void at::native::reduce_kernel<512, 1>(...)"


def write_csv(path, counter, dispatches):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(HEADER)
        for i, (name, value) in enumerate(dispatches):
            w.writerow([i + 1, i + 1, "Agent 1", 1, 600, 600, 1024, 7, name, 256, 0, 0, 8, 0, 32,
                        counter, value, 1000 + i, 2000 + i])


def test_case_round_trip() -> None:
    cfg = ACEConfig(binning="soft", num_bins=30, to_onehot_y=True, activation="softmax")
    case = ct.CaseArgs(impl="hip_mi355x", config=cfg.model_dump_json(), batch=2, channels=4,
                       spatial=(64, 64, 32), logit_scale=2.0, target_bias=0.5, mode="fwd_bwd",
                       dtype="bfloat16", seed=7, calls=5)
    argv = case.to_argv()
    assert argv[0] == "--child"
    back = ct.CaseArgs.from_json(argv[1])
    assert back == case
    assert ACEConfig.model_validate_json(back.config) == cfg


def test_traffic_scales_by_the_copy(tmp_path) -> None:
    calls = 10
    # FETCH_SIZE reads half of the copy's 256 MiB, WRITE_SIZE all of it
    copy_kib = ct.COPY_BYTES / 1024
    fetch = [(FWD, 1000.0), (SUM, 5.0), (BWD, 3000.0)] * calls + [(COPY, copy_kib / 2)] * calls
    write = [(FWD, 10.0), (SUM, 1.0), (BWD, 4000.0)] * calls + [(COPY, copy_kib)] * calls
    write_csv(tmp_path / "f_counter_collection.csv", "FETCH_SIZE", fetch)
    write_csv(tmp_path / "w_counter_collection.csv", "WRITE_SIZE", write)
    rows = ct.parse_counter_csv(sorted(tmp_path.glob("*counter_collection.csv")))
    assert set(rows) == {"FETCH_SIZE", "WRITE_SIZE"}
    assert rows["FETCH_SIZE"][0] == (FWD, 1000.0)
    tr = ct.traffic_from_rows(rows["FETCH_SIZE"], rows["WRITE_SIZE"], calls)
    assert tr.fetch_scale == pytest.approx(2.0) and tr.write_scale == pytest.approx(1.0)
    assert tr.dispatches == 2  # the torch reduce kernel is not the library's
    assert tr.read_bytes == pytest.approx(4000.0 * 2.0 * 1024)
    assert tr.write_bytes == pytest.approx(4010.0 * 1024)
    assert tr.total_bytes == pytest.approx(tr.read_bytes + tr.write_bytes)


def test_copy_value_ignores_small_copies() -> None:
    rows = [(COPY, 10.0), (COPY, 100.0), (COPY, 101.0), (COPY, 99.0)]
    assert ct.copy_value(rows) == pytest.approx(100.0)
    assert ct.copy_value([(FWD, 1.0)]) is None


def test_missing_copy_or_kernel_raises() -> None:
    copy_kib = ct.COPY_BYTES / 1024
    with pytest.raises(RuntimeError, match="calibration"):
        ct.traffic_from_rows([(FWD, 1.0)], [(FWD, 1.0)], 1)
    with pytest.raises(RuntimeError, match="no dispatch"):
        ct.traffic_from_rows([(COPY, copy_kib)], [(COPY, copy_kib)], 1)


def test_child_usage() -> None:
    assert ct.main([]) == 2
    assert ct.main(["--child"]) == 2


def test_row_counter_columns_default_to_none() -> None:
    row = m.Row(impl="hip_mi355x", binning="hard", mode="fwd", cuda_graph=False, shape="s",
                batch=1, channels=4, spatial="8x8x8", voxels=512, status="ok", input_bytes=8192,
                target_bytes=4096, ideal_bytes=12288)
    assert row.hbm_read_bytes is None and row.hbm_write_bytes is None
    assert row.hbm_bytes_per_ideal is None and row.counted_kernels_per_call is None


def test_bench_live_traffic_case_and_fallback(monkeypatch) -> None:
    """bench.py's live traffic asks for the dominant kernel of the workload's
    loss (forward only for the forward kernel) and returns None when the
    counter runs fail, so that the committed summary is used instead."""
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    sys.path.insert(0, str(root))
    import bench

    seen = []

    def fake_collect(case, timeout=120.0, kernel_filter=ct.KERNEL_FILTER):
        seen.append((case, kernel_filter))
        return ct.Traffic(read_bytes=1.0, write_bytes=2.0, fetch_kib=0.0, write_kib=0.0,
                          fetch_scale=2.0, write_scale=1.0, dispatches=1)

    monkeypatch.setattr(ct, "collect", fake_collect)
    tr = bench.live_traffic(2, "ace_fwd")
    assert tr.total_bytes == 3.0
    case, filt = seen[-1]
    assert case.workload == 2 and case.mode == "fwd" and filt == "ace::fwd_kernel"
    bench.live_traffic(4, "ace_bwd")
    case, filt = seen[-1]
    assert case.workload == 4 and case.mode == "fwd_bwd" and filt == "ace::bwd_kernel"

    def failing_collect(*args, **kwargs):
        raise RuntimeError("rocprofv3 --pmc FETCH_SIZE failed")

    monkeypatch.setattr(ct, "collect", failing_collect)
    assert bench.live_traffic(2, "ace_fwd") is None
